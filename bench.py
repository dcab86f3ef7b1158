#!/usr/bin/env python3
"""Benchmark of the MLX-affine quantized linear on one MI355X.

Workload (the metric's "Flux 3072->12288" shape): the
Flux double-block MLP pair on 1536 tokens with bf16 activations --
fc1 3072->12288 at 4 bits, tanh-GELU, fc2 12288->3072 at 8 bits, group 64,
f32 scales and biases, weights N(0, 0.02) before quantization.  One step is
fc1 + GELU + fc2 over the whole batch; inputs are resident in HBM before the
timed region starts.  The quantized weights rotate through distinct copies
totalling more than the 256 MB Infinity Cache, so every step streams its
weights from HBM.

The line printed on stdout is the JSON record; everything else goes to
stderr.  Kernels are timed with HIP events recorded on the stream they are
launched on (torch's current stream, handed to libsdq's raw entry point).
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

M_TOKENS = 1536
HIDDEN = 3072
MLP = 12288
GS = 64


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algorithmic_bytes(M, N, K, bits, x_bytes=2, y_bytes=2, s_bytes=4):
    return N * K * bits // 8 + 2 * N * (K // GS) * s_bytes + M * K * x_bytes + M * N * y_bytes


TRAFFIC_FILE = REPO / "profiles" / "bench_config2_hbm_traffic.md"


def measured_traffic(label):
    """Calibrated HBM bytes per dispatch of layer `label` ("fc1"/"fc2") from
    the committed rocprofv3 FETCH_SIZE + WRITE_SIZE summary, with the kernel
    it was measured on; None when the summary is absent."""
    if not TRAFFIC_FILE.exists():
        return None, None
    for line in TRAFFIC_FILE.read_text().splitlines():
        parts = line.split()
        if len(parts) == 4 and parts[0] == "traffic" and parts[1] == label:
            return int(parts[3]), parts[2]
    return None, None


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # The GPU's clocks ramp over the first ~100-150 steps (~40 ms) after idle:
    # per-step time falls from ~340 to ~277 us.  The warmup covers the ramp.
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--rotate", type=int, default=10, help="distinct weight copies (>= 9 exceeds the MALL)")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="target CPU baseline work")
    ap.add_argument("--unfused", action="store_true",
                    help="time the step with GELU as its own kernel between the two matmuls (the reference's "
                         "sequence of calls) instead of fused into fc1's epilogue; the other form is timed "
                         "and reported beside it either way")
    ap.add_argument("--no-compare", action="store_true",
                    help="skip timing the other GELU form (keeps a profiler's trace to one form)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="after the timed steps, run one f32->bf16 copy of 2^27 elements (512 MiB read, "
                         "256 MiB written): the known-size kernel that calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE")
    return ap.parse_args()


class Layer:
    """One quantized linear, with `rotate` distinct device copies."""

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


def launch(L, layer, copy, y_ptr, x_ptr, M, hstream, sdq, act=0):
    w, s, b = layer.ptrs[copy % len(layer.ptrs)]
    if act:
        rc = L.sdq_quantized_matmul_epilogue_raw(y_ptr, sdq.BFLOAT16, x_ptr, sdq.BFLOAT16, layer.K, w, s, b,
                                                 sdq.FLOAT32, M, layer.N, layer.K, GS, layer.bits, None, 0,
                                                 act, hstream)
    else:
        rc = L.sdq_quantized_matmul_raw(y_ptr, sdq.BFLOAT16, x_ptr, sdq.BFLOAT16, layer.K, w, s, b,
                                        sdq.FLOAT32, M, layer.N, layer.K, GS, layer.bits, hstream)
    if rc:
        sdq._check(rc, "quantized_matmul")


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
        "sample": (f"{reps} full config-2 steps (x[1536,3072] @ fc1[12288,3072]^T 4-bit + "
                   f"x[1536,12288] @ fc2[3072,12288]^T 8-bit) with the oracle's OpenMP f32 qmatmul, "
                   f"{flops_step * reps / 1e9:.0f} GFLOP in {dt:.1f} s; MLX's CPU backend is absent, "
                   f"this is the CPU restatement"),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    import sdq

    L = sdq.lib()
    if sdq.device_count() < 1 or not torch.cuda.is_available():
        log("no GPU visible")
        return 1
    dev = torch.device("cuda:0")
    s = sdq.Stream.gpu()
    t_setup = time.perf_counter()
    fc1 = Layer(sdq, s, MLP, HIDDEN, 4, seed=11, rotate=args.rotate)
    fc2 = Layer(sdq, s, HIDDEN, MLP, 8, seed=12, rotate=args.rotate)
    log(f"weights: {args.rotate} copies, {(fc1.resident_bytes() + fc2.resident_bytes()) / 2**20:.0f} MiB "
        f"resident, setup {time.perf_counter() - t_setup:.1f} s")

    g = torch.Generator(device=dev)
    g.manual_seed(5)
    x = torch.randn(M_TOKENS, HIDDEN, device=dev, generator=g).to(torch.bfloat16)
    h = torch.empty(M_TOKENS, MLP, device=dev, dtype=torch.bfloat16)
    a = torch.empty_like(h)
    y = torch.empty(M_TOKENS, HIDDEN, device=dev, dtype=torch.bfloat16)
    ts = torch.cuda.current_stream()
    hs = ts.cuda_stream

    def step(i, ev=None, fused=not args.unfused):
        # fused: GELU in fc1's epilogue (sdq_quantized_matmul_epilogue_raw);
        # unfused: fc1, then the GELU kernel, then fc2 (the reference's
        # sequence of calls, flux.rs:400-413).
        if ev:
            ev[0].record(ts)
        if fused:
            launch(L, fc1, i, a.data_ptr(), x.data_ptr(), M_TOKENS, hs, sdq, act=sdq.ACT_GELU_APPROX)
        else:
            launch(L, fc1, i, h.data_ptr(), x.data_ptr(), M_TOKENS, hs, sdq)
        if ev:
            ev[1].record(ts)
        if not fused:
            rc = L.sdq_gelu_approx_raw(a.data_ptr(), h.data_ptr(), sdq.BFLOAT16, h.numel(), hs)
            if rc:
                sdq._check(rc, "gelu_approx_raw")
        if ev:
            ev[2].record(ts)
        launch(L, fc2, i, y.data_ptr(), a.data_ptr(), M_TOKENS, hs, sdq)
        if ev:
            ev[3].record(ts)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # The timed region holds only the steps: per-call events between kernels
    # would themselves add gaps, so the per-call times come from a second,
    # separately timed pass below.
    e_start, e_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e_start.record(ts)
    for i in range(args.steps):
        step(args.warmup + i)
    e_end.record(ts)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    for i in range(args.steps):
        step(args.warmup + args.steps + i, evs[i])
    torch.cuda.synchronize()
    # The other form of the step, timed the same way, for comparison.
    other_ms = float("nan")
    if not args.no_compare:
        for i in range(args.warmup):
            step(i, fused=args.unfused)
        o_start, o_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        o_start.record(ts)
        for i in range(args.steps):
            step(args.warmup + i, fused=args.unfused)
        o_end.record(ts)
        torch.cuda.synchronize()
        other_ms = o_start.elapsed_time(o_end) / args.steps
    if args.copy_probe:
        src = torch.zeros(1 << 27, device=dev, dtype=torch.float32)
        dst = torch.empty(1 << 27, device=dev, dtype=torch.bfloat16)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    total_ms = e_start.elapsed_time(e_end)
    ms_step = total_ms / args.steps
    k_fc1 = float(np.mean([e[0].elapsed_time(e[1]) for e in evs]))
    k_gelu = float(np.mean([e[1].elapsed_time(e[2]) for e in evs]))
    k_fc2 = float(np.mean([e[2].elapsed_time(e[3]) for e in evs]))
    flops_fc1 = 2.0 * M_TOKENS * HIDDEN * MLP
    flops_fc2 = 2.0 * M_TOKENS * MLP * HIDDEN
    flops_step = flops_fc1 + flops_fc2
    value = flops_step / (ms_step / 1e3) / 1e12
    form, other_form = ("unfused", "fused") if args.unfused else ("fused", "unfused")
    log(f"step {ms_step:.3f} ms (wall {wall / args.steps * 1e3:.3f} ms, GELU {form}): fc1 {k_fc1:.3f} ms "
        f"({flops_fc1 / k_fc1 / 1e9:.0f} TFLOP/s), gelu {k_gelu:.3f} ms, fc2 {k_fc2:.3f} ms "
        f"({flops_fc2 / k_fc2 / 1e9:.0f} TFLOP/s); {other_form} step {other_ms:.3f} ms")

    # Dominant kernel's roofline (MFMA-bound at M = 1536: AI far above the ridge).
    # One call is the tile kernel plus, when the plan splits K, the reduction
    # kernel of its partial tiles; the events bracket the whole call.
    if k_fc1 >= k_fc2:
        epi = "" if args.unfused else ", GELU epilogue"
        dom, dom_ms, dom_flops, dom_layer, label = (f"qmm fc1 4-bit 1536x3072->12288 (qmm_kernel + qmm_reduce_kernel{epi})",
                                                    k_fc1, flops_fc1, fc1, "fc1")
    else:
        dom, dom_ms, dom_flops, dom_layer, label = ("qmm fc2 8-bit 1536x12288->3072 (qmm_kernel + qmm_reduce_kernel)",
                                                    k_fc2, flops_fc2, fc2, "fc2")
    achieved = dom_flops / (dom_ms / 1e3) / 1e12
    traffic, traffic_kernel = measured_traffic(label)
    roofline = {
        "kernel": dom,
        "bound": "mfma",
        "achieved": round(achieved, 2),
        "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
        "traffic": traffic,
        "traffic_source": (f"{TRAFFIC_FILE.relative_to(REPO)} ({traffic_kernel}, rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                           "copy-calibrated)") if traffic else None,
        "flops_per_launch": dom_flops,
        "algorithmic_bytes_per_launch": algorithmic_bytes(M_TOKENS, dom_layer.N, dom_layer.K, dom_layer.bits),
        "avg_launch_ms": round(dom_ms, 4),
    }

    sweep = []
    if not args.no_sweep:
        fc1_8 = Layer(sdq, s, MLP, HIDDEN, 8, seed=13, rotate=args.rotate)
        xs = torch.randn(4608, HIDDEN, device=dev, generator=g).to(torch.bfloat16)
        ys = torch.empty(4608, MLP, device=dev, dtype=torch.bfloat16)
        for bits, layer in ((4, fc1), (8, fc1_8)):
            for M in (1, 4, 16, 32, 64, 256, 1024, 1536, 4608):
                reps = 30 if M <= 64 else 10
                for i in range(3):
                    launch(L, layer, i, ys.data_ptr(), xs.data_ptr(), M, hs, sdq)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                e0.record(ts)
                for i in range(reps):
                    launch(L, layer, i, ys.data_ptr(), xs.data_ptr(), M, hs, sdq)
                e1.record(ts)
                torch.cuda.synchronize()
                ms = e0.elapsed_time(e1) / reps
                fl = 2.0 * M * MLP * HIDDEN
                by = algorithmic_bytes(M, MLP, HIDDEN, bits)
                tf, gbs = fl / ms / 1e9, by / ms / 1e6
                bound = "hbm" if fl / by < RIDGE else "mfma"
                frac = gbs / PEAK_HBM_GBS if bound == "hbm" else tf / PEAK_BF16_TFLOPS
                sweep.append({"M": M, "bits": bits, "us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 1),
                              "GB/s": round(gbs, 1), "bound": bound, "frac": round(frac, 4)})
                log(f"sweep 3072->12288 {bits}-bit M={M:5d}: {ms * 1e3:9.2f} us {tf:8.1f} TFLOP/s "
                    f"{gbs:8.1f} GB/s  {bound} {frac * 100:5.1f}%")
        del fc1_8

    cpu = None
    if not args.no_cpu_baseline:
        t = time.perf_counter()
        cpu = cpu_baseline(args, fc1, fc2)
        log(f"cpu baseline {cpu['value'] * 1e3:.2f} GFLOP/s on {cpu['cores']} threads ({time.perf_counter() - t:.1f} s)")

    rec = {
        "metric": "quantized-matmul TFLOP/s + HBM GB/s (% roofline), Flux 3072->12288, 4/8-bit, M=1..4608",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: weights N(0,0.02) f32 quantized MLX-affine group 64; activations N(0,1) bf16",
        "config": {
            "workload": "BASELINE config 2: Flux double-block MLP pair, 1536 tokens (512x512): "
                        "fc1 3072->12288 4-bit, tanh-GELU, fc2 12288->3072 8-bit, group 64, "
                        "f32 scales, bf16 activations in and out",
            "global_batch": M_TOKENS,
            "seq_len": M_TOKENS,
            "parallelism": "single GPU",
            "weight_copies_rotated": args.rotate,
            "gelu": "separate kernel between the matmuls (sdq_gelu_approx_raw)" if args.unfused else
                    "fused into fc1's epilogue (sdq_quantized_matmul_epilogue_raw)",
        },
        f"ms_per_step_{other_form}": None if args.no_compare else round(other_ms, 4),
        "kernels_ms": {"fc1": round(k_fc1, 4), "gelu": round(k_gelu, 4), "fc2": round(k_fc2, 4)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "sweep_3072x12288": sweep,
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
