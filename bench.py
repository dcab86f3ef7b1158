#!/usr/bin/env python3
"""Benchmark of the MLX-affine quantized linear on one MI355X.

Headline workload (the metric's "Flux 3072->12288" shape):
the Flux double-block MLP pair on 1536 tokens with bf16 activations -- fc1
3072->12288 at 4 bits, tanh-GELU, fc2 12288->3072 at 8 bits, group 64, f32
scales and biases, weights N(0, 0.02) before quantization.  One step is fc1 +
GELU + fc2 over the whole batch; inputs are resident in HBM before the timed
region starts.  The quantized weights rotate through distinct copies totalling
more than 512 MB (twice the 256 MB Infinity Cache), so every step streams its
weights from HBM.

Protocol (the reference's: docs/handoff.md:2162-2175, minimum of interleaved
repetitions): a fixed-duration untimed clock warm-up, then --warmup steps,
then --reps repetitions that each time exactly --steps steps of the fused form
(GELU in fc1's epilogue) and then --steps steps of the unfused form (fc1, the
GELU kernel, fc2: the reference's sequence of calls); each form reports the
minimum over its repetitions.

Beside the headline: an M sweep of 3072->12288 at 4 and 8 bits, and BASELINE
config 5 (every distinct linear of one Flux-schnell step at 1024x1024 with its
per-step call count, under BASELINE's bit policy and under the reference's
mixed(4), quantized.rs:156-166).  Those points replay a captured HIP graph of
one launch per rotated weight copy, so the timing holds the kernels only (no
host launch overhead); each point rotates more than 512 MB of weights.

The line printed on stdout is the JSON record; everything else goes to
stderr.  Kernels are timed with HIP events recorded on the stream they are
launched on (handed to libsdq's raw entry points).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "stable-diffusion.rs_amd"))

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
RIDGE = PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)  # FLOP per byte
ROTATE_BYTES = 600 << 20    # weight bytes each timed point rotates through (> 512 MB)

M_TOKENS = 1536
HIDDEN = 3072
MLP = 12288
GS = 64

# the distinct quantized linears of one Flux-schnell step at
# 1024x1024 (4096 image + 512 text tokens, hidden 3072), from
# sd-models/src/mlx/flux.rs (double_block 333-420, single_block 424-471,
# embedders 491-502, final layer 580-600).  (name, M, K, N, calls per step,
# bits under BASELINE's policy -- residual writers at 8 --, bits under the
# reference's mixed(4) -- 8 only for the modulation, embedder-in and final
# layers --).
CONFIG5 = [
    ("double img_mod.lin + txt_mod.lin", 1, 3072, 18432, 38, 8, 8),
    ("double img_attn.qkv", 4096, 3072, 9216, 19, 4, 4),
    ("double txt_attn.qkv", 512, 3072, 9216, 19, 4, 4),
    ("double img_attn.proj", 4096, 3072, 3072, 19, 8, 4),
    ("double txt_attn.proj", 512, 3072, 3072, 19, 8, 4),
    ("double img_mlp.0 (fc1)", 4096, 3072, 12288, 19, 4, 4),
    ("double txt_mlp.0 (fc1)", 512, 3072, 12288, 19, 4, 4),
    ("double img_mlp.2 (fc2)", 4096, 12288, 3072, 19, 8, 4),
    ("double txt_mlp.2 (fc2)", 512, 12288, 3072, 19, 8, 4),
    ("single modulation.lin", 1, 3072, 9216, 38, 8, 8),
    ("single linear1", 4608, 3072, 21504, 38, 4, 4),
    ("single linear2", 4608, 15360, 3072, 38, 8, 4),
    ("img_in", 4096, 64, 3072, 1, 8, 8),
    ("txt_in", 512, 4096, 3072, 1, 8, 8),
    ("time_in.in_layer", 1, 256, 3072, 1, 4, 4),
    ("vector_in.in_layer", 1, 768, 3072, 1, 4, 4),
    ("time_in/vector_in.out_layer", 1, 3072, 3072, 2, 4, 4),
    ("final_layer.adaLN_modulation.1", 1, 3072, 6144, 1, 8, 8),
    ("final_layer.linear", 4096, 3072, 64, 1, 8, 8),
]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algorithmic_bytes(M, N, K, bits, x_bytes=2, y_bytes=2, s_bytes=4):
    return N * K * bits // 8 + 2 * N * (K // GS) * s_bytes + M * K * x_bytes + M * N * y_bytes


def roofline_point(M, N, K, bits, ms):
    fl = 2.0 * M * N * K
    by = algorithmic_bytes(M, N, K, bits)
    tf, gbs = fl / ms / 1e9, by / ms / 1e6
    bound = "hbm" if fl / by < RIDGE else "mfma"
    frac = gbs / PEAK_HBM_GBS if bound == "hbm" else tf / PEAK_BF16_TFLOPS
    return {"us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 1), "GB/s": round(gbs, 1), "bound": bound,
            "frac": round(frac, 4)}


TRAFFIC_FILE = REPO / "profiles" / "qmm_config2_step.md"


def measured_traffic(label):
    """Calibrated HBM bytes per call of layer `label` ("fc1"/"fc2") from the
    committed rocprofv3 FETCH_SIZE + WRITE_SIZE summary, with the kernel it was
    measured on; None when the summary is absent."""
    if not TRAFFIC_FILE.exists():
        return None, None
    for line in TRAFFIC_FILE.read_text().splitlines():
        parts = line.split()
        if len(parts) == 4 and parts[0] == "traffic" and parts[1] == label:
            return int(parts[3]), parts[2]
    return None, None


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50, help="steps timed per repetition and form")
    ap.add_argument("--warmup", type=int, default=20, help="untimed steps after the clock warm-up")
    ap.add_argument("--clock-warmup", type=float, default=1.5,
                    help="seconds of untimed steps first: the GPU's clocks ramp over ~0.1 s after idle")
    ap.add_argument("--reps", type=int, default=5, help="interleaved repetitions (minimum reported)")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-config5", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="target CPU baseline work")
    ap.add_argument("--unfused", action="store_true",
                    help="report the unfused form (fc1, GELU kernel, fc2) as the headline")
    ap.add_argument("--no-config3", action="store_true")
    ap.add_argument("--only", choices=["step", "sweep", "config3", "config5", "refgemm"], default=None,
                    help="run one part only (for profiling its kernels)")
    ap.add_argument("--sweep-m", default="1,4,16,32,64,128,256,512,1024,1536,4608",
                    help="comma-separated M values of the 3072->12288 sweep")
    ap.add_argument("--sweep-bits", default="4,8", help="comma-separated bit widths of the sweep")
    ap.add_argument("--copy-probe", action="store_true",
                    help="at the end, run one f32->bf16 copy of 2^27 elements (512 MiB read, 256 MiB "
                         "written): the known-size kernel that calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE")
    return ap.parse_args()


class Raw:
    """ctypes access to the raw entry points on torch-owned device memory."""

    def __init__(self, sdq):
        self.sdq = sdq
        self.L = sdq.lib()

    def matmul(self, y, x, w, s, b, M, N, K, bits, hs, act=0, s_dtype=None):
        sdq = self.sdq
        sdt = sdq.FLOAT32 if s_dtype is None else s_dtype
        if act:
            rc = self.L.sdq_quantized_matmul_epilogue_raw(y, sdq.BFLOAT16, x, sdq.BFLOAT16, K, w, s, b, sdt,
                                                          M, N, K, GS, bits, None, 0, act, hs)
        else:
            rc = self.L.sdq_quantized_matmul_raw(y, sdq.BFLOAT16, x, sdq.BFLOAT16, K, w, s, b, sdt,
                                                 M, N, K, GS, bits, hs)
        if rc:
            sdq._check(rc, "quantized_matmul_raw")

    def gated(self, y, x, w, s, b, M, N2, K, bits, hs):
        """T5's gelu(wi_0 x) * (wi_1 x) from the paired weight (N2 rows)."""
        sdq = self.sdq
        rc = self.L.sdq_quantized_linear_gated_raw(y, 0, sdq.BFLOAT16, x, sdq.BFLOAT16, K, w, s, b, sdq.FLOAT32,
                                                   M, N2, K, GS, bits, None, 0, sdq.ACT_GELU_APPROX, hs)
        if rc:
            sdq._check(rc, "quantized_linear_gated_raw")

    def gelu(self, out, inp, n, hs):
        rc = self.L.sdq_gelu_approx_raw(out, inp, self.sdq.BFLOAT16, n, hs)
        if rc:
            self.sdq._check(rc, "gelu_approx_raw")


class Layer:
    """One quantized linear (real MLX-affine quantization of N(0, 0.02)
    weights), with `rotate` distinct device copies."""

    def __init__(self, sdq, stream, N, K, bits, seed, rotate):
        rng = np.random.default_rng(seed)
        w = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
        self.w_host = w
        q = sdq.QuantizedArray.quantize(sdq.Array.from_numpy(w), GS, bits, stream)
        self.copies = [q]
        for _ in range(rotate - 1):
            self.copies.append(sdq.QuantizedArray(q.weight.contiguous(stream), q.scales.contiguous(stream),
                                                  q.biases.contiguous(stream), GS, bits))
        stream.synchronize()
        self.N, self.K, self.bits = N, K, bits
        self.ptrs = [(c.weight.device_ptr, c.scales.device_ptr, c.biases.device_ptr) for c in self.copies]

    def resident_bytes(self):
        return sum(c.resident_bytes() for c in self.copies)


class SynthLayer:
    """Device-generated quantized weights for timing-only points: uniform
    random codes and scales/biases of the magnitude N(0, 0.02) weights give
    (the kernels' work does not depend on the values).  Copies rotate through
    more than ROTATE_BYTES."""

    def __init__(self, torch, dev, N, K, bits, seed):
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        words = N * K * bits // 32
        per_copy = words * 4 + 2 * N * (K // GS) * 4
        # Tiny weights (the embedders) would need thousands of copies: they are
        # capped, and then sit in the caches as they do in a real step.
        self.rotate = min(64, max(2, -(-ROTATE_BYTES // per_copy)))
        self.w = torch.randint(-2**31, 2**31 - 1, (self.rotate, words), device=dev, dtype=torch.int32, generator=g)
        self.s = torch.rand((self.rotate, N * (K // GS)), device=dev, generator=g) * 0.004 + 0.0005
        self.b = -self.s * (2 ** (bits - 1))
        self.N, self.K, self.bits = N, K, bits
        self.ptrs = [(self.w[i].data_ptr(), self.s[i].data_ptr(), self.b[i].data_ptr()) for i in range(self.rotate)]


def graph_time(torch, raw, layer, M, x, y, reps=6):
    """Per-launch ms of `layer` at M rows: a HIP graph of one launch per weight
    copy, replayed `reps` times; the minimum replay.  y is written row-major
    [M, N]; the graph's output is checked bit-for-bit against an eager launch
    of the same (last) copy."""
    s = torch.cuda.Stream()
    nrot = len(layer.ptrs)
    with torch.cuda.stream(s):
        hs = s.cuda_stream
        for i in range(2 * nrot):  # warm the stream's workspace and the clocks
            w, sc, b = layer.ptrs[i % nrot]
            raw.matmul(y.data_ptr(), x.data_ptr(), w, sc, b, M, layer.N, layer.K, layer.bits, hs)
    s.synchronize()
    out = y.view(-1)[:M * layer.N]
    ref = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(nrot):
            w, sc, b = layer.ptrs[i]
            raw.matmul(y.data_ptr(), x.data_ptr(), w, sc, b, M, layer.N, layer.K, layer.bits, s.cuda_stream)
    best = float("inf")
    with torch.cuda.stream(s):
        for r in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            g.replay()
            e1.record(s)
            e1.synchronize()
            if r > 0:  # the first replay uploads the graph
                best = min(best, e0.elapsed_time(e1) / nrot)
    s.synchronize()
    if not torch.equal(out, ref):
        raise RuntimeError(f"graph replay of M={M} N={layer.N} K={layer.K} differs from the eager launch")
    del g
    return best


def graph_time_fn(torch, launch, nrot, reps=6):
    """Per-iteration ms of `launch(i, hip_stream)` for i in range(nrot) (one
    weight copy each), captured in one HIP graph and replayed `reps` times;
    the minimum replay."""
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for i in range(2 * nrot):
            launch(i % nrot, s.cuda_stream)
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(nrot):
            launch(i, s.cuda_stream)
    best = float("inf")
    with torch.cuda.stream(s):
        for r in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            g.replay()
            e1.record(s)
            e1.synchronize()
            if r > 0:
                best = min(best, e0.elapsed_time(e1) / nrot)
    s.synchronize()
    del g
    return best


def config3(torch, raw, sdq, dev, g):
    """BASELINE config 3, T5-XXL's gated-GELU FFN (t5.rs:201-214): wi_0 and
    wi_1 4096->10240 4-bit, wo 10240->4096 8-bit, at M = 512 and the GEMV
    sweep M = 1, 4, 16.  Two forms of the FFN input are timed: the paired
    weight in one launch (sdq_quantized_linear_gated_raw), and the reference's
    sequence with the GELU fused into wi_0's epilogue -- wi_0+GELU, wi_1, an
    elementwise product -- each as HIP-graph replays over rotated weights."""
    D, F = 4096, 10240
    pair = SynthLayer(torch, dev, 2 * F, D, 4, seed=31)
    wi0 = SynthLayer(torch, dev, F, D, 4, seed=32)
    wi1 = SynthLayer(torch, dev, F, D, 4, seed=33)
    wo = SynthLayer(torch, dev, D, F, 8, seed=34)
    x = torch.randn(512, D, device=dev, generator=g).to(torch.bfloat16)
    hg = torch.empty(512, F, device=dev, dtype=torch.bfloat16)
    hu = torch.empty_like(hg)
    a = torch.empty_like(hg)
    y = torch.empty(512, D, device=dev, dtype=torch.bfloat16)
    rows = []
    for M in (512, 1, 4, 16):
        def gated(i, hs):
            w, sc, b = pair.ptrs[i]
            raw.gated(a.data_ptr(), x.data_ptr(), w, sc, b, M, 2 * F, D, 4, hs)

        def two(i, hs):
            w, sc, b = wi0.ptrs[i % wi0.rotate]
            raw.matmul(hg.data_ptr(), x.data_ptr(), w, sc, b, M, F, D, 4, hs, act=sdq.ACT_GELU_APPROX)
            w, sc, b = wi1.ptrs[i % wi1.rotate]
            raw.matmul(hu.data_ptr(), x.data_ptr(), w, sc, b, M, F, D, 4, hs)
            torch.mul(hg[:M], hu[:M], out=a[:M])

        def out(i, hs):
            w, sc, b = wo.ptrs[i]
            raw.matmul(y.data_ptr(), a.data_ptr(), w, sc, b, M, D, F, 8, hs)

        t_gated = graph_time_fn(torch, gated, pair.rotate)
        t_two = graph_time_fn(torch, two, max(wi0.rotate, wi1.rotate))
        t_wo = graph_time_fn(torch, out, wo.rotate)
        pt = roofline_point(M, 2 * F, D, 4, t_gated)
        rows.append({"M": M, "ms_gated_pair": round(t_gated, 4), "ms_wi0_gelu_wi1_mul": round(t_two, 4),
                     "ms_wo": round(t_wo, 4), "ms_ffn": round(t_gated + t_wo, 4),
                     "ms_ffn_two_linear_form": round(t_two + t_wo, 4),
                     "gated_pair_roofline": {k: pt[k] for k in ("TFLOP/s", "GB/s", "bound", "frac")}})
        log(f"config3 T5 FFN M={M:4d}: gated pair {t_gated * 1e3:8.2f} us ({pt['bound']} {pt['frac'] * 100:5.1f}%), "
            f"wi_0+gelu, wi_1, mul {t_two * 1e3:8.2f} us; wo {t_wo * 1e3:8.2f} us; "
            f"FFN {(t_gated + t_wo) * 1e3:8.2f} vs {(t_two + t_wo) * 1e3:8.2f} us")
    del pair, wi0, wi1, wo, x, hg, hu, a, y
    return {"note": "T5-XXL FFN (d_model 4096, d_ff 10240; wi 4-bit, wo 8-bit, group 64): the paired gated "
                    "launch vs wi_0 with the GELU epilogue + wi_1 + an elementwise product; HIP-graph replays "
                    "over device-random weights rotated through > 512 MB", "points": rows}


def reference_gemm(torch, dev, g):
    """The vendor library's dense bf16 GEMM (torch.mm, hipBLASLt) on the
    config-2/4 shapes with the weight already bf16 -- the practical MFMA
    ceiling the quantized kernel is compared with (it also dequantizes).
    Only with --only refgemm."""
    rows = []
    for (M, K, N) in [(1536, 3072, 12288), (4608, 3072, 12288), (4608, 12288, 3072), (8192, 8192, 8192)]:
        a = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
        b = torch.randn(N, K, device=dev, generator=g).to(torch.bfloat16)
        for _ in range(5):
            torch.mm(a, b.t())
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(5):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(20):
                torch.mm(a, b.t())
            e1.record()
            e1.synchronize()
            best = min(best, e0.elapsed_time(e1) / 20)
        tf = 2.0 * M * N * K / best / 1e9
        rows.append({"M": M, "K": K, "N": N, "ms": round(best, 4), "TFLOP/s": round(tf, 1),
                     "frac": round(tf / PEAK_BF16_TFLOPS, 4)})
        log(f"reference bf16 GEMM {M}x{K}->{N}: {best * 1e3:8.1f} us {tf:7.1f} TFLOP/s "
            f"({tf / PEAK_BF16_TFLOPS * 100:.1f}% of peak)")
        del a, b
    return rows


def cpu_baseline(args, fc1, fc2):
    """The oracle's blocked OpenMP qmatmul (the CPU restatement; MLX's CPU
    backend is not available) on the same step: fc1 and fc2 at full size on
    all 1536 rows, repeated until about --cpu-seconds of work (the GELU
    between them is excluded: it is the same elementwise pass either way)."""
    sys.path.insert(0, str(REPO / "oracle"))
    import sdq_oracle as oracle

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    rng = np.random.default_rng(7)
    x1 = rng.standard_normal((M_TOKENS, HIDDEN), dtype=np.float32)
    x2 = rng.standard_normal((M_TOKENS, MLP), dtype=np.float32)
    q1 = oracle.quantize(fc1.w_host, GS, 4)
    q2 = oracle.quantize(fc2.w_host, GS, 8)
    flops_step = 2.0 * M_TOKENS * (MLP * HIDDEN + HIDDEN * MLP)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.qmatmul_omp(x1, *q1, GS, 4, threads)
        oracle.qmatmul_omp(x2, *q2, GS, 8, threads)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= args.cpu_seconds:
            break
    return {
        "value": flops_step * reps / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": cpu_model(),
        "sample": (f"{reps} full config-2 steps (x[1536,3072] @ fc1[12288,3072]^T 4-bit + "
                   f"x[1536,12288] @ fc2[3072,12288]^T 8-bit) with the oracle's OpenMP f32 qmatmul on "
                   f"{threads} threads of {cpu_model()}, {flops_step * reps / 1e9:.0f} GFLOP in {dt:.1f} s; "
                   f"MLX's CPU backend is absent, this is the CPU restatement"),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    import sdq

    raw = Raw(sdq)
    if sdq.device_count() < 1 or not torch.cuda.is_available():
        log("no GPU visible")
        return 1
    dev = torch.device("cuda:0")
    s = sdq.Stream.gpu()
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    do_step = args.only in (None, "step")

    # ---- headline: the config-2 MLP pair -------------------------------------------------
    fc1 = fc2 = None
    rec_step = {}
    if do_step:
        t_setup = time.perf_counter()
        per_pair = (MLP * HIDDEN // 2 + 2 * MLP * (HIDDEN // GS) * 4) + (HIDDEN * MLP + 2 * HIDDEN * (MLP // GS) * 4)
        rotate = max(2, -(-ROTATE_BYTES // per_pair))
        fc1 = Layer(sdq, s, MLP, HIDDEN, 4, seed=11, rotate=rotate)
        fc2 = Layer(sdq, s, HIDDEN, MLP, 8, seed=12, rotate=rotate)
        log(f"weights: {rotate} copies, {(fc1.resident_bytes() + fc2.resident_bytes()) / 2**20:.0f} MiB resident, "
            f"setup {time.perf_counter() - t_setup:.1f} s")
        x = torch.randn(M_TOKENS, HIDDEN, device=dev, generator=g).to(torch.bfloat16)
        h = torch.empty(M_TOKENS, MLP, device=dev, dtype=torch.bfloat16)
        a = torch.empty_like(h)
        y = torch.empty(M_TOKENS, HIDDEN, device=dev, dtype=torch.bfloat16)
        ts = torch.cuda.current_stream()
        hs = ts.cuda_stream

        def step(i, fused, ev=None):
            # fused: GELU in fc1's epilogue (sdq_quantized_matmul_epilogue_raw);
            # unfused: fc1, then the GELU kernel, then fc2 (flux.rs:400-413).
            w1, s1, b1 = fc1.ptrs[i % rotate]
            w2, s2, b2 = fc2.ptrs[i % rotate]
            if ev:
                ev[0].record(ts)
            if fused:
                raw.matmul(a.data_ptr(), x.data_ptr(), w1, s1, b1, M_TOKENS, MLP, HIDDEN, 4, hs,
                           act=sdq.ACT_GELU_APPROX)
            else:
                raw.matmul(h.data_ptr(), x.data_ptr(), w1, s1, b1, M_TOKENS, MLP, HIDDEN, 4, hs)
            if ev:
                ev[1].record(ts)
            if not fused:
                raw.gelu(a.data_ptr(), h.data_ptr(), h.numel(), hs)
            if ev:
                ev[2].record(ts)
            raw.matmul(y.data_ptr(), a.data_ptr(), w2, s2, b2, M_TOKENS, HIDDEN, MLP, 8, hs)
            if ev:
                ev[3].record(ts)

        # Clock warm-up for a fixed time, then the requested warmup steps.
        t0 = time.perf_counter()
        n_clock = 0
        while time.perf_counter() - t0 < args.clock_warmup:
            for _ in range(20):
                step(n_clock, fused=not args.unfused)
                n_clock += 1
            torch.cuda.synchronize()
        for i in range(args.warmup):
            step(i, fused=not args.unfused)
        torch.cuda.synchronize()

        # Interleaved repetitions: each times exactly --steps steps of each form.
        times = {True: [], False: []}
        t_wall = time.perf_counter()
        for r in range(args.reps):
            for fused in (True, False):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                e0.record(ts)
                for i in range(args.steps):
                    step(i, fused)
                e1.record(ts)
                torch.cuda.synchronize()
                times[fused].append(e0.elapsed_time(e1) / args.steps)
        wall = time.perf_counter() - t_wall
        head_fused = not args.unfused
        ms_step = min(times[head_fused])
        other_ms = min(times[not head_fused])
        # Per-call times: a separate pass with events around each call (events
        # between kernels add gaps, so they are not in the timed region above).
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
        for i in range(args.steps):
            step(i, head_fused, evs[i])
        torch.cuda.synchronize()
        k_fc1 = float(np.median([e[0].elapsed_time(e[1]) for e in evs]))
        k_gelu = float(np.median([e[1].elapsed_time(e[2]) for e in evs]))
        k_fc2 = float(np.median([e[2].elapsed_time(e[3]) for e in evs]))
        flops_fc1 = 2.0 * M_TOKENS * HIDDEN * MLP
        flops_fc2 = 2.0 * M_TOKENS * MLP * HIDDEN
        form, other_form = ("fused", "unfused") if head_fused else ("unfused", "fused")
        log(f"step {ms_step:.4f} ms ({form}; reps {', '.join(f'{t:.4f}' for t in times[head_fused])}), "
            f"{other_form} {other_ms:.4f} ms; per call: fc1 {k_fc1:.4f} ms, gelu {k_gelu:.4f} ms, "
            f"fc2 {k_fc2:.4f} ms; clock warm-up {n_clock} steps; timed wall {wall:.2f} s")
        # Dominant kernel's roofline (MFMA-bound at M = 1536: AI far above the
        # ridge).  A call is the tile kernel plus, when the plan splits K, the
        # reduction kernel of its partial tiles; the events bracket the call.
        if k_fc1 >= k_fc2:
            epi = ", GELU epilogue" if head_fused else ""
            dom, dom_ms, dom_flops, dom_layer, label = (
                f"qmm fc1 4-bit 1536x3072->12288 (qmm_kernel + qmm_reduce_kernel{epi})", k_fc1, flops_fc1, fc1, "fc1")
        else:
            dom, dom_ms, dom_flops, dom_layer, label = (
                "qmm fc2 8-bit 1536x12288->3072 (qmm_kernel + qmm_reduce_kernel)", k_fc2, flops_fc2, fc2, "fc2")
        achieved = dom_flops / (dom_ms / 1e3) / 1e12
        traffic, traffic_kernel = measured_traffic(label)
        rec_step = {
            "ms_per_step": round(ms_step, 4),
            f"ms_per_step_{other_form}": round(other_ms, 4),
            "value": round((flops_fc1 + flops_fc2) / (ms_step / 1e3) / 1e12, 2),
            "kernels_ms": {"fc1": round(k_fc1, 4), "gelu": round(k_gelu, 4), "fc2": round(k_fc2, 4)},
            "protocol": {"clock_warmup_s": args.clock_warmup, "clock_warmup_steps": n_clock,
                         "warmup_steps": args.warmup, "reps": args.reps, "steps_per_rep": args.steps,
                         "reported": "minimum over interleaved repetitions (fused, unfused alternating)",
                         "weight_copies_rotated": rotate,
                         "rotated_mib": round((fc1.resident_bytes() + fc2.resident_bytes()) / 2**20)},
            "roofline": {
                "kernel": dom,
                "bound": "mfma",
                "achieved": round(achieved, 2),
                "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                "traffic": traffic,
                "traffic_source": (f"{TRAFFIC_FILE.relative_to(REPO)} ({traffic_kernel}, rocprofv3 FETCH_SIZE + "
                                   "WRITE_SIZE, copy-calibrated)") if traffic else None,
                "flops_per_launch": dom_flops,
                "algorithmic_bytes_per_launch": algorithmic_bytes(M_TOKENS, dom_layer.N, dom_layer.K, dom_layer.bits),
                "avg_launch_ms": round(dom_ms, 4),
            },
        }
        del h, a, y

    # ---- M sweep of 3072->12288 ---------------------------------------------------------------
    sweep = []
    if args.only in (None, "sweep") and not args.no_sweep:
        xs = torch.randn(4608, HIDDEN, device=dev, generator=g).to(torch.bfloat16)
        ys = torch.empty(4608, MLP, device=dev, dtype=torch.bfloat16)
        for bits in (int(b) for b in args.sweep_bits.split(",")):
            layer = SynthLayer(torch, dev, MLP, HIDDEN, bits, seed=20 + bits)
            for M in (int(m) for m in args.sweep_m.split(",")):
                ms = graph_time(torch, raw, layer, M, xs, ys)
                pt = {"M": M, "bits": bits, **roofline_point(M, MLP, HIDDEN, bits, ms), "copies": layer.rotate}
                sweep.append(pt)
                log(f"sweep 3072->12288 {bits}-bit M={M:5d}: {pt['us']:9.2f} us {pt['TFLOP/s']:8.1f} TFLOP/s "
                    f"{pt['GB/s']:8.1f} GB/s  {pt['bound']} {pt['frac'] * 100:5.1f}%  ({layer.rotate} copies)")
            del layer
        del xs, ys

    # ---- config 3: T5-XXL's gated FFN ------------------------------------------------------------
    c3 = None
    if args.only in (None, "config3") and not args.no_config3:
        c3 = config3(torch, raw, sdq, dev, g)

    refgemm = reference_gemm(torch, dev, g) if args.only == "refgemm" else None

    # ---- config 5: one Flux-schnell step's quantized linears ------------------------------------
    config5 = None
    if args.only in (None, "config5") and not args.no_config5:
        xs = torch.randn(4608 * 15360, device=dev, generator=g).to(torch.bfloat16)
        ys = torch.empty(4608 * 21504, device=dev, dtype=torch.bfloat16)
        shapes = {}
        for name, M, K, N, calls, b_bl, b_ref in CONFIG5:
            for bits in {b_bl, b_ref}:
                key = (M, K, N, bits)
                if key in shapes:
                    continue
                layer = SynthLayer(torch, dev, N, K, bits, seed=M + K + N + bits)
                ms = graph_time(torch, raw, layer, M, xs, ys)
                shapes[key] = ms
                del layer
        flops_step = 0.0
        per_policy = {}
        for policy, idx in (("baseline", 5), ("reference_mixed4", 6)):
            rows, total_ms = [], 0.0
            for entry in CONFIG5:
                name, M, K, N, calls = entry[:5]
                bits = entry[idx]
                ms = shapes[(M, K, N, bits)]
                total_ms += calls * ms
                if policy == "baseline":
                    flops_step += calls * 2.0 * M * N * K
                rows.append({"linear": name, "M": M, "K": K, "N": N, "bits": bits, "calls": calls,
                             "ms_total": round(calls * ms, 4), **roofline_point(M, N, K, bits, ms)})
            per_policy[policy] = {"ms_per_step": round(total_ms, 3), "shapes": rows}
        for policy, v in per_policy.items():
            v["TFLOP/s"] = round(flops_step / (v["ms_per_step"] / 1e3) / 1e12, 1)
            v["mfma_frac"] = round(v["TFLOP/s"] / PEAK_BF16_TFLOPS, 4)
            log(f"config5 [{policy}]: {v['ms_per_step']:.3f} ms of quantized matmul per step, "
                f"{v['TFLOP/s']:.0f} TFLOP/s ({v['mfma_frac'] * 100:.1f}% of MFMA peak)")
            for r in v["shapes"]:
                log(f"    {r['linear']:34s} {r['M']:5d}x{r['K']:5d}->{r['N']:5d} {r['bits']}-bit x{r['calls']:2d}: "
                    f"{r['us']:8.2f} us/call  {r['bound']} {r['frac'] * 100:5.1f}%")
        config5 = {"tflop_per_step": round(flops_step / 1e12, 3),
                   "note": "summed quantized-matmul time of one Flux-schnell step at 1024x1024 (graph replays "
                           "per distinct shape, times its per-step call count); baseline = BASELINE's bits "
                           "(residual writers 8-bit), reference_mixed4 = quantized.rs:156-166",
                   **per_policy}
        del xs, ys

    if args.copy_probe:
        src = torch.zeros(1 << 27, device=dev, dtype=torch.float32)
        dst = torch.empty(1 << 27, device=dev, dtype=torch.bfloat16)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    cpu = None
    if do_step and not args.no_cpu_baseline:
        t = time.perf_counter()
        cpu = cpu_baseline(args, fc1, fc2)
        log(f"cpu baseline {cpu['value'] * 1e3:.2f} GFLOP/s on {cpu['cores']} threads of {cpu['cpu_model']} "
            f"({time.perf_counter() - t:.1f} s)")

    rec = {
        "metric": "quantized-matmul TFLOP/s + HBM GB/s (% roofline), Flux 3072->12288, 4/8-bit, M=1..4608",
        "value": rec_step.get("value"),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": rec_step.get("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: weights N(0,0.02) f32 quantized MLX-affine group 64 (headline); sweep and config-5 "
                "points use device-random codes and scales of the same magnitude; activations N(0,1) bf16",
        "config": {
            "workload": "BASELINE config 2: Flux double-block MLP pair, 1536 tokens (512x512): "
                        "fc1 3072->12288 4-bit, tanh-GELU, fc2 12288->3072 8-bit, group 64, "
                        "f32 scales, bf16 activations in and out",
            "global_batch": M_TOKENS,
            "seq_len": M_TOKENS,
            "parallelism": "single GPU",
            "gelu": "separate kernel between the matmuls (sdq_gelu_approx_raw)" if args.unfused else
                    "fused into fc1's epilogue (sdq_quantized_matmul_epilogue_raw)",
        },
        **{k: v for k, v in rec_step.items() if k not in ("value", "ms_per_step")},
        "cpu_baseline": cpu,
        "sweep_3072x12288": sweep,
        "config3": c3,
        "config5": config5,
        **({"reference_gemm_bf16": refgemm} if refgemm else {}),
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
