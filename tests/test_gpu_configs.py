"""BASELINE configs 1, 3 and 5 at full size, and the fused epilogue at the
reference's call sites, through the C ABI against the CPU oracle.

Every full-size case quantizes the oracle's seeded N(0, 0.02) weight on the
GPU (codes checked bit for bit against the oracle), multiplies the whole x on
the GPU, and checks a sample of output rows against the f64 product of the
oracle's dequantized weight: max |d| / max |ref| <= 2e-2 and cosine >= 0.9999
(the north star's tolerances)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import cosine, max_rel_err

pytestmark = pytest.mark.gpu

MAX_REL = 2e-2
MIN_COS = 0.9999


def _gelu64(v):
    c = np.float64(np.float32(0.7978845238685608))
    return 0.5 * v * (1.0 + np.tanh((v + 0.044715 * v ** 3) * c))


def _weight(oracle, sdq, stream, seed, N, K, bits, sdt="f32"):
    """GPU-quantized weight, checked against the oracle's codes, and the
    oracle's dequantized weight."""
    w = oracle.normals(seed, N * K, 0.02).reshape(N, K)
    if sdt == "bf16":
        wb = sdq.f32_to_bf16_bits(w)
        w_dev, w = sdq.Array.from_numpy(wb, sdq.BFLOAT16), sdq.bf16_bits_to_f32(wb).reshape(N, K)
        code = 12
    else:
        w_dev, code = sdq.Array.from_numpy(w), 10
    q = sdq.QuantizedArray.quantize(w_dev, 64, bits, stream)
    wq, s, b = oracle.quantize(w, 64, bits, code)
    assert np.array_equal(q.weight.to_numpy(), wq)
    return q, oracle.dequantize(wq, s, b, 64, bits, code)


def _x(oracle, sdq, seed, shape, xdt="bf16"):
    x = oracle.normals(seed, int(np.prod(shape))).reshape(shape)
    if xdt == "bf16":
        bits = sdq.f32_to_bf16_bits(x)
        return sdq.Array.from_numpy(bits, sdq.BFLOAT16), sdq.bf16_bits_to_f32(bits).reshape(shape)
    return sdq.Array.from_numpy(x), x


def _rows(M, n=40):
    return np.unique(np.concatenate([np.linspace(0, M - 1, min(n, M)).astype(int), [M - 1]]))


def _check(got, want):
    err, cos = max_rel_err(got, want), cosine(got, want)
    assert err <= MAX_REL and cos >= MIN_COS, (err, cos)
    assert np.all(np.isfinite(got))
    return err, cos


def _full(oracle, sdq, stream, M, K, N, bits, seed, xdt="bf16"):
    print(f"full-size M={M} K={K} N={N} bits={bits} x={xdt}", flush=True)
    q, deq = _weight(oracle, sdq, stream, seed, N, K, bits)
    x_dev, x = _x(oracle, sdq, seed + 1, (M, K), xdt)
    y = q.matmul(x_dev, stream)
    assert y.shape == [M, N] and y.dtype == sdq.FLOAT32
    got = y.to_numpy()
    pick = _rows(M)
    _check(got[pick], x[pick].astype(np.float64) @ deq.astype(np.float64).T)


def test_config1_f32_activations_at_full_size(oracle, sdq, stream):
    # f32 x[1024, 3072] @ W[3072, 3072]^T at 4 bits, f32
    # scales and output (the MLX CPU backend's --cpu case).
    _full(oracle, sdq, stream, 1024, 3072, 3072, 4, seed=2100, xdt="f32")


@pytest.mark.parametrize("M,K,N,bits", [
    (512, 10240, 4096, 8),   # wo at 512 tokens
    (4, 4096, 10240, 4),     # wi at 4 tokens
    (4, 10240, 4096, 8),     # wo at 4 tokens
    (16, 4096, 10240, 4),    # wi at 16 tokens
    (1, 10240, 4096, 8),     # wo at 1 token
])
def test_config3_t5_ffn_shapes(oracle, sdq, stream, M, K, N, bits):
    # BASELINE config 3 (t5.rs:209-214; T5Config::xxl t5.rs:41-52).
    _full(oracle, sdq, stream, M, K, N, bits, seed=2200 + M + bits)


# The distinct linears of a Flux-schnell step at 1024x1024 (flux.rs:333-600)
# not covered elsewhere, at the bit widths of both policies.
@pytest.mark.parametrize("M,K,N,bits", [
    (1, 3072, 18432, 8),     # double img_mod.lin / txt_mod.lin
    (4096, 3072, 9216, 4),   # double img_attn.qkv
    (512, 3072, 9216, 4),    # double txt_attn.qkv
    (4096, 3072, 3072, 8),   # double img_attn.proj (BASELINE: 8-bit)
    (4096, 3072, 3072, 4),   # double img_attn.proj (reference mixed(4))
    (512, 3072, 3072, 8),    # double txt_attn.proj
    (4096, 3072, 12288, 4),  # double img_mlp.0
    (512, 3072, 12288, 4),   # double txt_mlp.0
    (4096, 12288, 3072, 8),  # double img_mlp.2
    (512, 12288, 3072, 4),   # double txt_mlp.2 (reference mixed(4))
    (4608, 15360, 3072, 4),  # single linear2 (reference mixed(4))
    (512, 4096, 3072, 8),    # txt_in
    (1, 256, 3072, 4),       # time_in.in_layer
    (1, 768, 3072, 4),       # vector_in.in_layer
    (1, 3072, 3072, 4),      # time_in / vector_in out_layer
    (1, 3072, 6144, 8),      # final_layer.adaLN_modulation.1
])
def test_config5_flux_step_shapes(oracle, sdq, stream, M, K, N, bits):
    _full(oracle, sdq, stream, M, K, N, bits, seed=2300 + M + K + N + bits)


def test_t5_gated_gelu_ffn_at_full_size(oracle, sdq, stream):
    # t5.rs:209-214: gelu(wi_0 x) * (wi_1 x), the product fused into wi_0's
    # call, at config 3's 512 tokens.
    M, K, N = 512, 4096, 10240
    print("t5 product full size", flush=True)
    q0, d0 = _weight(oracle, sdq, stream, 2400, N, K, 4)
    q1, d1 = _weight(oracle, sdq, stream, 2401, N, K, 4)
    x_dev, x = _x(oracle, sdq, 2402, (M, K))
    lin = q1.matmul(x_dev, stream)
    y = q0.linear_combine(x_dev, stream, lin, sdq.COMBINE_PRODUCT, activation=sdq.ACT_GELU_APPROX)
    assert y.shape == [M, N]
    pick = _rows(M)
    xs = x[pick].astype(np.float64)
    want = _gelu64(xs @ d0.astype(np.float64).T) * (xs @ d1.astype(np.float64).T)
    _check(y.to_numpy()[pick], want)


def test_flux_gated_residual_at_full_size(oracle, sdq, stream):
    # flux.rs:464-470: x + gate * linear2(...), config 4's 4608 tokens, with
    # bf16 scales so the output, residual and gate are all bf16 (Flux's
    # residual stream).
    M, K, N = 4608, 15360, 3072
    print("flux gated residual full size", flush=True)
    q, deq = _weight(oracle, sdq, stream, 2500, N, K, 8, sdt="bf16")
    x_dev, x = _x(oracle, sdq, 2501, (1, M, K))
    r_bits = sdq.f32_to_bf16_bits(oracle.normals(2502, M * N).reshape(1, M, N))
    g_bits = sdq.f32_to_bf16_bits(oracle.normals(2503, N, 0.5))
    res = sdq.Array.from_numpy(r_bits, sdq.BFLOAT16)
    gate = sdq.Array.from_numpy(g_bits, sdq.BFLOAT16)
    y = q.linear_combine(x_dev, stream, res, sdq.COMBINE_GATED_RESIDUAL, gate=gate)
    assert y.shape == [1, M, N] and y.dtype == sdq.BFLOAT16
    got = sdq.bf16_bits_to_f32(y.to_numpy()).reshape(M, N)
    pick = _rows(M)
    r = sdq.bf16_bits_to_f32(r_bits).reshape(M, N)[pick].astype(np.float64)
    g = sdq.bf16_bits_to_f32(g_bits).astype(np.float64)
    want = r + g * (x[0][pick].astype(np.float64) @ deq.astype(np.float64).T)
    _check(got[pick], want)


# ---- the combine stage over every operand dtype ----------------------------------------

_CODE = {"f32": 10, "bf16": 12, "f16": 9}


def _host_array(sdq, vals, dt):
    if dt == "bf16":
        bits = sdq.f32_to_bf16_bits(vals)
        return sdq.Array.from_numpy(bits, sdq.BFLOAT16), sdq.bf16_bits_to_f32(bits).reshape(vals.shape)
    if dt == "f16":
        h = vals.astype(np.float16)
        return sdq.Array.from_numpy(h), h.astype(np.float32)
    return sdq.Array.from_numpy(vals.astype(np.float32)), vals.astype(np.float32)


# (gate dtype, mode): a gate applies to the gated residual only.
_GATE_MODES = [(g, "gated") for g in (None, "bf16", "f16", "f32")] + [(None, "product")]


@pytest.mark.parametrize("M,N", [(160, 256), (150, 100)])   # 16-byte path, element path
@pytest.mark.parametrize("sdt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("rdt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("gdt,mode", _GATE_MODES)
def test_combine_over_operand_dtypes(oracle, sdq, stream, M, N, sdt, rdt, gdt, mode):
    # The combine stage in the large-M kernel's store (M > 128 here), for every output,
    # residual and gate dtype: against the f64 composition, and bit for bit
    # against the unfused sequence where that sequence rounds the same way
    # (a product, or a residual without gate: one rounding in both).
    K = 256
    print(f"combine M={M} N={N} s={sdt} r={rdt} g={gdt} {mode}", flush=True)
    xdt = "f16" if sdt == "f16" else "bf16"
    w = oracle.normals(2600 + N, N * K, 0.02).reshape(N, K)
    w_dev, w_vals = _host_array(sdq, w, sdt)
    q = sdq.QuantizedArray.quantize(w_dev, 64, 4, stream)
    wq, s, b = oracle.quantize(w_vals, 64, 4, _CODE[sdt])
    deq = oracle.dequantize(wq, s, b, 64, 4, _CODE[sdt])
    x_dev, x = _host_array(sdq, oracle.normals(2601 + M, M * K).reshape(M, K), xdt)
    r_dev, r = _host_array(sdq, oracle.normals(2602 + M, M * N).reshape(M, N), rdt)
    g_dev, g = (None, None) if gdt is None else _host_array(sdq, oracle.normals(2603, N, 0.5), gdt)
    v = x.astype(np.float64) @ deq.astype(np.float64).T
    if mode == "product":
        y = q.linear_combine(x_dev, stream, r_dev, sdq.COMBINE_PRODUCT, activation=sdq.ACT_GELU_APPROX)
        want = _gelu64(v) * r
    else:
        y = q.linear_combine(x_dev, stream, r_dev, sdq.COMBINE_GATED_RESIDUAL, gate=g_dev)
        want = r + (g if g is not None else 1.0) * v
    out_code = {10: "f32", 12: "bf16", 9: "f16"}[y.dtype]
    got = y.to_float32()
    _check(got, want)
    if mode == "product" or gdt is None:
        lin = q.linear(x_dev, stream, activation=sdq.ACT_GELU_APPROX if mode == "product" else 0)
        seq = lin.mul(r_dev, stream) if mode == "product" else lin.add(r_dev, stream)
        if seq.dtype == y.dtype:
            assert np.array_equal(seq.to_numpy(), y.to_numpy()), out_code


# ---- the small-M kernel's launch shapes -----------------------------------------------------


@pytest.mark.parametrize("M,N,K,bits,note", [
    (1, 100, 192, 4, "x staged per wave; half 128-chunk at the end of K"),
    (3, 4100, 3072, 8, "x staged per wave; ragged last tile"),
    (4, 64, 16384, 4, "x staged per wave, long K: many waves per tile"),
    (8, 12288, 1024, 4, "x staged once per block, several tiles per block"),
    (16, 3072, 3072, 8, "x staged once per block"),
    (16, 512, 16384, 4, "x too large to stage: read per chunk"),
    (24, 512, 512, 8, "two row blocks, x staged once per block"),
    (32, 300, 8192, 4, "two row blocks, x read per chunk"),
])
def test_small_m_launch_shapes(oracle, sdq, stream, M, N, K, bits, note):
    print(f"small-M M={M} N={N} K={K} bits={bits}: {note}", flush=True)
    q, deq = _weight(oracle, sdq, stream, 2700 + M + N, N, K, bits)
    x_dev, x = _x(oracle, sdq, 2701 + M, (M, K))
    got = q.matmul(x_dev, stream).to_numpy()
    err, _ = _check(got, x.astype(np.float64) @ deq.astype(np.float64).T)
    # Scales and biases act once per group on exact integer-code products.
    assert err < 1e-4
    assert np.array_equal(q.matmul(x_dev, stream).to_numpy(), got)


def test_small_m_with_a_row_stride(oracle, sdq, stream):
    # x rows further apart than K (a view into a wider buffer), raw entry
    # point, every staging mode.
    L = sdq.lib()
    for M, K in ((2, 1024), (12, 1024), (20, 8192)):
        N, ldx = 256, 0
        ldx = K + 64
        q, deq = _weight(oracle, sdq, stream, 2800 + M, N, K, 4)
        xw = oracle.normals(2801 + M, M * ldx).reshape(M, ldx)
        bits = sdq.f32_to_bf16_bits(xw)
        x_dev = sdq.Array.from_numpy(bits, sdq.BFLOAT16)
        x = sdq.bf16_bits_to_f32(bits).reshape(M, ldx)[:, :K]
        out = sdq.Array.from_numpy(np.zeros((M, N), np.float32))
        rc = L.sdq_quantized_matmul_raw(out.device_ptr, sdq.FLOAT32, x_dev.device_ptr, sdq.BFLOAT16, ldx,
                                        q.weight.device_ptr, q.scales.device_ptr, q.biases.device_ptr,
                                        sdq.FLOAT32, M, N, K, 64, 4, stream.native)
        assert rc == 0
        stream.synchronize()
        _check(out.to_numpy(), x.astype(np.float64) @ deq.astype(np.float64).T)
