"""GPU quantized_matmul through the C ABI against the oracle (the north
star's second parity level): max relative error <= 2e-2 (max |d| / max |ref|)
and cosine >= 0.9999 against the f64 product of the oracle's dequantized
weight, on the same seeded inputs.  Covers both kernels (M <= 32: the
bandwidth kernel; M > 32: the MFMA tile kernel), tails in M and N, split-K,
dtype promotion, group size 128, and the BASELINE shapes at full size."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import cosine, max_rel_err

pytestmark = pytest.mark.gpu

MAX_REL = 2e-2
MIN_COS = 0.9999
XDT = {"f32": 10, "bf16": 12, "f16": 9}


def _x(oracle, sdq, seed, shape, xdt):
    x = oracle.normals(seed, int(np.prod(shape))).reshape(shape)
    if xdt == "bf16":
        bits = sdq.f32_to_bf16_bits(x)
        return sdq.Array.from_numpy(bits, sdq.BFLOAT16), sdq.bf16_bits_to_f32(bits).reshape(shape)
    if xdt == "f16":
        h = x.astype(np.float16)
        return sdq.Array.from_numpy(h, sdq.FLOAT16), h.astype(np.float32)
    return sdq.Array.from_numpy(x, sdq.FLOAT32), x


def _qweight(oracle, sdq, stream, seed, N, K, bits, gs=64, sdt="f32"):
    w = oracle.normals(seed, N * K, 0.02).reshape(N, K)
    if sdt == "bf16":
        wb = sdq.f32_to_bf16_bits(w)
        w_dev = sdq.Array.from_numpy(wb, sdq.BFLOAT16)
        w = sdq.bf16_bits_to_f32(wb).reshape(N, K)
    else:
        w_dev = sdq.Array.from_numpy(w)
    q = sdq.QuantizedArray.quantize(w_dev, gs, bits, stream)
    s_code = 12 if sdt == "bf16" else 10
    wq, s, b = oracle.quantize(w, gs, bits, s_code)
    deq = oracle.dequantize(wq, s, b, gs, bits, s_code)
    return q, deq


def _check(got, x_vals, deq):
    want = x_vals.reshape(-1, x_vals.shape[-1]).astype(np.float64) @ deq.astype(np.float64).T
    got = got.reshape(want.shape)
    err, cos = max_rel_err(got, want), cosine(got, want)
    assert err <= MAX_REL and cos >= MIN_COS, (err, cos)
    return err, cos


CASES = [
    # (M, N, K, bits) -- M <= 32 is the bandwidth kernel, above is the MFMA tile kernel
    (1, 256, 512, 4), (1, 100, 512, 8), (2, 96, 256, 4), (3, 64, 64, 4), (4, 320, 1024, 8),
    (7, 256, 192, 4), (15, 128, 512, 8), (16, 256, 512, 4), (17, 200, 256, 4), (31, 64, 512, 8),
    (32, 288, 384, 4), (33, 256, 512, 4), (48, 300, 256, 8), (64, 512, 256, 4), (100, 96, 128, 8),
    (128, 256, 512, 4), (129, 320, 256, 4), (255, 256, 192, 8), (256, 512, 512, 4),
    (257, 64, 128, 4), (300, 500, 320, 8), (513, 1024, 256, 4),
]


@pytest.mark.parametrize("M,N,K,bits", CASES)
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_quantized_matmul_matches_the_oracle(oracle, sdq, stream, M, N, K, bits, xdt):
    print(f"qmatmul M={M} N={N} K={K} bits={bits} x={xdt}", flush=True)
    q, deq = _qweight(oracle, sdq, stream, 400 + N + K + bits, N, K, bits)
    x_dev, x_vals = _x(oracle, sdq, 500 + M, (M, K), xdt)
    y = q.matmul(x_dev, stream)
    assert y.shape == [M, N]
    assert y.dtype == sdq.FLOAT32  # promote(x, f32 scales) = f32
    _check(y.to_numpy(), x_vals, deq)


@pytest.mark.parametrize("M", [1, 16, 200])
@pytest.mark.parametrize("bits", [4, 8])
def test_bf16_scales_give_bf16_output(oracle, sdq, stream, M, bits):
    print(f"bf16 scales M={M} bits={bits}", flush=True)
    q, deq = _qweight(oracle, sdq, stream, 600 + M, 192, 256, bits, sdt="bf16")
    x_dev, x_vals = _x(oracle, sdq, 601 + M, (M, 256), "bf16")
    y = q.matmul(x_dev, stream)
    assert y.dtype == sdq.BFLOAT16
    _check(sdq.bf16_bits_to_f32(y.to_numpy()), x_vals, deq)


@pytest.mark.parametrize("M", [1, 9, 40, 77])
def test_group_size_128(oracle, sdq, stream, M):
    print(f"gs128 M={M}", flush=True)
    q, deq = _qweight(oracle, sdq, stream, 700 + M, 160, 512, 4, gs=128)
    x_dev, x_vals = _x(oracle, sdq, 701 + M, (M, 512), "bf16")
    _check(q.matmul(x_dev, stream).to_numpy(), x_vals, deq)


@pytest.mark.parametrize("xdt", ["f16"])
@pytest.mark.parametrize("M", [5, 50, 70])
def test_f16_activations(oracle, sdq, stream, xdt, M):
    q, deq = _qweight(oracle, sdq, stream, 750 + M, 128, 256, 8)
    x_dev, x_vals = _x(oracle, sdq, 751 + M, (M, 256), xdt)
    _check(q.matmul(x_dev, stream).to_numpy(), x_vals, deq)


def test_leading_dimensions_of_x(oracle, sdq, stream):
    # Flux feeds [1, seq, K] token tensors (flux.rs:352-357).
    q, deq = _qweight(oracle, sdq, stream, 800, 96, 128, 4)
    x_dev, x_vals = _x(oracle, sdq, 801, (1, 40, 128), "bf16")
    y = q.matmul(x_dev, stream)
    assert y.shape == [1, 40, 96]
    _check(y.to_numpy(), x_vals, deq)


@pytest.mark.parametrize("M", [1, 4, 16, 32])
def test_split_k_is_deterministic_and_correct(oracle, sdq, stream, M):
    # Few 32-row tiles and a long K force the K split across blocks; the
    # last block sums the partials in split order, so repeated calls agree
    # bit for bit and the per-tile counters are left ready for the next call.
    print(f"split-K M={M}", flush=True)
    q, deq = _qweight(oracle, sdq, stream, 900 + M, 64, 8192, 4)
    x_dev, x_vals = _x(oracle, sdq, 901 + M, (M, 8192), "bf16")
    first = q.matmul(x_dev, stream).to_numpy()
    _check(first, x_vals, deq)
    for _ in range(3):
        assert np.array_equal(q.matmul(x_dev, stream).to_numpy(), first)


@pytest.mark.parametrize("M,N,K,bits", [
    (300, 512, 8192, 4),    # 4 tiles of 256 x 256: every tile split along K
    (100, 640, 4096, 8),    # 128-row tiles, 3 tiles, split
    (48, 640, 4096, 8),     # 64-row tiles (M <= 64), 3 tiles, split
    (64, 12288, 4096, 4),   # 64 tokens at K = 4096: 48 tiles of 64 x 256, split
    (4352, 4096, 512, 4),   # 272 tiles: one whole round, the last 16 tiles split
])
def test_large_m_split_k_is_deterministic_and_correct(oracle, sdq, stream, M, N, K, bits):
    # When the tiles do not fill whole rounds of CUs, the MFMA kernel splits
    # the tiles of the last round along K; a second kernel adds the ranges'
    # partial tiles in range order, so repeated calls agree bit for bit.
    print(f"qmm split-K M={M} N={N} K={K} bits={bits}", flush=True)
    q, deq = _qweight(oracle, sdq, stream, 930 + M + bits, N, K, bits)
    x_dev, x_vals = _x(oracle, sdq, 931 + M, (M, K), "bf16")
    first = q.matmul(x_dev, stream).to_numpy()
    last = np.arange(max(0, M - 256), M)  # the split tiles are the last M tile
    pick = np.unique(np.concatenate([last, np.linspace(0, M - 1, 32).astype(int)]))
    _check(first[pick], x_vals[pick], deq)
    for _ in range(2):
        assert np.array_equal(q.matmul(x_dev, stream).to_numpy(), first)


@pytest.mark.parametrize("sdt", ["f32", "bf16"])
@pytest.mark.parametrize("M,N", [(70, 97), (300, 250), (33, 6)])
def test_ragged_output_rows(oracle, sdq, stream, sdt, M, N):
    # Output rows that are not a whole number of 16-byte pieces (f32 or bf16
    # output) take the element-store path of the MFMA kernel's epilogue.
    print(f"ragged N M={M} N={N} scales={sdt}", flush=True)
    q, deq = _qweight(oracle, sdq, stream, 970 + N, N, 192, 4, sdt=sdt)
    x_dev, x_vals = _x(oracle, sdq, 971 + M, (M, 192), "bf16")
    y = q.matmul(x_dev, stream)
    got = y.to_numpy()
    if y.dtype == sdq.BFLOAT16:
        got = sdq.bf16_bits_to_f32(got).reshape(M, N)
    _check(got, x_vals, deq)


def test_repeated_calls_are_identical(oracle, sdq, stream):
    q, _ = _qweight(oracle, sdq, stream, 950, 512, 1024, 8)
    x_dev, _ = _x(oracle, sdq, 951, (300, 1024), "bf16")
    a = q.matmul(x_dev, stream).to_numpy()
    b = q.matmul(x_dev, stream).to_numpy()
    assert np.array_equal(a, b)


def test_small_m_kernel_is_near_exact(oracle, sdq, stream):
    # The bandwidth kernel applies scale and bias once per group to exact
    # integer-code products, so it tracks the f64 reference to ~1e-6.
    q, deq = _qweight(oracle, sdq, stream, 960, 256, 2048, 4)
    x_dev, x_vals = _x(oracle, sdq, 961, (8, 2048), "bf16")
    err, _ = _check(q.matmul(x_dev, stream).to_numpy(), x_vals, deq)
    assert err < 1e-5


# ---- BASELINE shapes at full size -------------------------------------------------


def _sampled_check(oracle, sdq, stream, M, N, K, bits, seed, rows=48):
    print(f"full-size M={M} N={N} K={K} bits={bits}", flush=True)
    w = oracle.normals(seed, N * K, 0.02).reshape(N, K)
    q = sdq.QuantizedArray.quantize(sdq.Array.from_numpy(w), 64, bits, stream)
    wq, s, b = oracle.quantize(w, 64, bits)
    # Quantization itself is bit-exact at full size too.
    assert np.array_equal(q.weight.to_numpy(), wq)
    deq = oracle.dequantize(wq, s, b, 64, bits)
    x_dev, x_vals = _x(oracle, sdq, seed + 1, (M, K), "bf16")
    y = q.matmul(x_dev, stream).to_numpy()
    pick = np.unique(np.linspace(0, M - 1, min(rows, M)).astype(int))
    _check(y[pick], x_vals[pick], deq)
    assert np.all(np.isfinite(y))


@pytest.mark.parametrize("M,N,K,bits", [
    (1536, 12288, 3072, 4),   # config 2: Flux fc1
    (1536, 3072, 12288, 8),   # config 2: Flux fc2
    (512, 10240, 4096, 4),    # config 3: T5 wi_0 / wi_1
    (16, 4096, 10240, 8),     # config 3: T5 wo, M = 16
    (1, 10240, 4096, 4),      # config 3: T5 wi, M = 1
    (4608, 21504, 3072, 4),   # config 4: Flux linear1
    (4608, 3072, 15360, 8),   # config 4: Flux linear2
    (1, 9216, 3072, 8),       # config 4: adaLN modulation
    (4096, 64, 3072, 8),      # config 5: final_layer.linear (N = 64)
    (4096, 3072, 64, 8),      # config 5: img_in (K = 64, one group)
])
def test_baseline_shapes(oracle, sdq, stream, M, N, K, bits):
    _sampled_check(oracle, sdq, stream, M, N, K, bits, seed=1000 + M + N + K)


# ---- fused epilogue: act(x @ dequantize(w).T + bias) -----------------------------------


def _gelu64(v):
    c = np.float64(np.float32(0.7978845238685608))
    return 0.5 * v * (1.0 + np.tanh((v + 0.044715 * v ** 3) * c))


@pytest.mark.parametrize("M,N,K,bits", [
    (1, 200, 512, 4),       # small-M kernel, direct store
    (16, 64, 8192, 8),      # small-M kernel, K in ranges (the reduction kernel stores)
    (100, 300, 256, 4),     # narrow layer: the small-M kernel's row groups
    (100, 300, 4096, 4),    # tile kernel, 128-row tiles
    (300, 512, 8192, 4),    # tile kernel, split K (the reduction kernel stores)
    (40, 300, 256, 8),      # tile kernel, 64-row tiles
    (48, 512, 8192, 4),     # tile kernel, 64-row tiles, split K
])
@pytest.mark.parametrize("act", [0, 1])
@pytest.mark.parametrize("bias_dtype", ["f32", "bf16", None])
def test_linear_epilogue_matches_the_composition(oracle, sdq, stream, M, N, K, bits, act, bias_dtype):
    # quantized.rs:314-317 (bias after the matmul) and flux.rs:400-413 (GELU
    # after the MLP's first linear), fused into the matmul's store.
    print(f"linear M={M} N={N} K={K} bits={bits} act={act} bias={bias_dtype}", flush=True)
    q, deq = _qweight(oracle, sdq, stream, 1100 + N + bits, N, K, bits)
    x_dev, x_vals = _x(oracle, sdq, 1101 + M, (M, K), "bf16")
    b = oracle.normals(1102 + N, N)
    bias = None
    if bias_dtype == "f32":
        bias = sdq.Array.from_numpy(b)
    elif bias_dtype == "bf16":
        bits16 = sdq.f32_to_bf16_bits(b)
        bias, b = sdq.Array.from_numpy(bits16, sdq.BFLOAT16), sdq.bf16_bits_to_f32(bits16)
    y = q.linear(x_dev, stream, bias=bias, activation=act)
    assert y.dtype == sdq.FLOAT32 and y.shape == [M, N]
    got = y.to_numpy()
    v = x_vals.astype(np.float64) @ deq.astype(np.float64).T + (b if bias is not None else 0.0)
    want = _gelu64(v) if act else v
    err, cos = max_rel_err(got, want), cosine(got, want)
    assert err <= MAX_REL and cos >= MIN_COS, (err, cos)
    # With f32 output the fused sum equals the unfused sequence exactly, and
    # the GELU equals the elementwise op on it to its own bound.
    plain = q.matmul(x_dev, stream).to_numpy()
    pre = (plain + b.astype(np.float32)).astype(np.float32) if bias is not None else plain
    if act:
        assert np.max(np.abs(got - oracle.gelu_approx(pre))) <= 2e-6 + 1e-6 * np.max(np.abs(pre))
    else:
        assert np.array_equal(got, pre)


def test_linear_epilogue_bf16_output_and_raw_entry(oracle, sdq, stream):
    # bf16 scales give bf16 output: the epilogue works on the f32 accumulator
    # and rounds once; the raw entry point computes the same bits.
    import ctypes
    M, N, K = 40, 96, 256
    q, deq = _qweight(oracle, sdq, stream, 1200, N, K, 4, sdt="bf16")
    x_dev, x_vals = _x(oracle, sdq, 1201, (M, K), "bf16")
    b = oracle.normals(1202, N)
    bias = sdq.Array.from_numpy(b)
    y = q.linear(x_dev, stream, bias=bias, activation=sdq.ACT_GELU_APPROX)
    assert y.dtype == sdq.BFLOAT16
    got = sdq.bf16_bits_to_f32(y.to_numpy()).reshape(M, N)
    want = _gelu64(x_vals.astype(np.float64) @ deq.astype(np.float64).T + b)
    err, cos = max_rel_err(got, want), cosine(got, want)
    assert err <= MAX_REL and cos >= MIN_COS, (err, cos)
    out = sdq.Array.from_numpy(np.zeros((M, N), np.uint16), sdq.BFLOAT16)
    L = sdq.lib()
    rc = L.sdq_quantized_matmul_epilogue_raw(
        out.device_ptr, sdq.BFLOAT16, x_dev.device_ptr, sdq.BFLOAT16, K, q.weight.device_ptr,
        q.scales.device_ptr, q.biases.device_ptr, sdq.BFLOAT16, M, N, K, 64, 4,
        bias.device_ptr, sdq.FLOAT32, sdq.ACT_GELU_APPROX, stream.native)
    assert rc == 0
    stream.synchronize()
    assert np.array_equal(out.to_numpy(), y.to_numpy())


def test_linear_epilogue_rejects_bad_arguments(oracle, sdq, stream):
    q, _ = _qweight(oracle, sdq, stream, 1300, 64, 128, 4)
    x_dev, _ = _x(oracle, sdq, 1301, (4, 128), "bf16")
    with pytest.raises(sdq.Error, match="bias must be"):
        q.linear(x_dev, stream, bias=sdq.Array.from_numpy(np.zeros(63, np.float32)))
    with pytest.raises(sdq.Error, match="activation"):
        q.linear(x_dev, stream, activation=7)


@pytest.mark.parametrize("M,N,K,bits", [
    (1, 200, 512, 4),       # small-M kernel: combine in the store
    (16, 64, 8192, 8),      # small-M kernel, K in ranges: combine in the reduction kernel
    (100, 300, 256, 4),     # narrow layer: row groups, combine in their store
    (100, 300, 4096, 4),    # tile kernel: combine in its store
    (300, 512, 8192, 4),    # tile kernel with split K: combine in the reduction kernel
    (40, 300, 256, 8),      # 64-row tiles: combine in the store
    (48, 512, 8192, 4),     # 64-row tiles, split K: combine in the reduction kernel
])
@pytest.mark.parametrize("mode", ["gated", "residual", "product"])
def test_linear_combine_matches_the_composition(oracle, sdq, stream, M, N, K, bits, mode):
    # Flux's gated residual x + gate * linear(h) (flux.rs:389-398) and T5's
    # gelu(wi_0 x) * (wi_1 x) (t5.rs:209-214), as one call.
    print(f"combine M={M} N={N} K={K} bits={bits} mode={mode}", flush=True)
    q, deq = _qweight(oracle, sdq, stream, 1400 + N + bits, N, K, bits)
    x_dev, x_vals = _x(oracle, sdq, 1401 + M, (M, K), "bf16")
    b = oracle.normals(1402 + N, N)
    r = oracle.normals(1403 + M, M * N).reshape(M, N)
    g = oracle.normals(1404 + N, N, 0.5)
    bits16 = sdq.f32_to_bf16_bits(r)
    res, r = sdq.Array.from_numpy(bits16, sdq.BFLOAT16), sdq.bf16_bits_to_f32(bits16).reshape(M, N)
    v = x_vals.astype(np.float64) @ deq.astype(np.float64).T + b
    if mode == "product":
        y = q.linear_combine(x_dev, stream, res, sdq.COMBINE_PRODUCT, bias=sdq.Array.from_numpy(b),
                             activation=sdq.ACT_GELU_APPROX)
        want = _gelu64(v) * r
    elif mode == "gated":
        y = q.linear_combine(x_dev, stream, res, sdq.COMBINE_GATED_RESIDUAL, bias=sdq.Array.from_numpy(b),
                             gate=sdq.Array.from_numpy(g))
        want = r + g * v
    else:
        y = q.linear_combine(x_dev, stream, res, sdq.COMBINE_GATED_RESIDUAL, bias=sdq.Array.from_numpy(b))
        want = r + v
    assert y.dtype == sdq.FLOAT32 and y.shape == [M, N]
    got = y.to_numpy()
    err, cos = max_rel_err(got, want), cosine(got, want)
    assert err <= MAX_REL and cos >= MIN_COS, (err, cos)
    # Repeated calls agree bit for bit.
    if mode == "gated":
        again = q.linear_combine(x_dev, stream, res, sdq.COMBINE_GATED_RESIDUAL, bias=sdq.Array.from_numpy(b),
                                 gate=sdq.Array.from_numpy(g)).to_numpy()
        assert np.array_equal(again, got)


def test_linear_combine_rejects_bad_arguments(oracle, sdq, stream):
    q, _ = _qweight(oracle, sdq, stream, 1500, 64, 128, 4)
    x_dev, _ = _x(oracle, sdq, 1501, (4, 128), "bf16")
    good = sdq.Array.from_numpy(np.zeros((4, 64), np.float32))
    with pytest.raises(sdq.Error, match="residual must be"):
        q.linear_combine(x_dev, stream, sdq.Array.from_numpy(np.zeros((4, 63), np.float32)),
                         sdq.COMBINE_GATED_RESIDUAL)
    with pytest.raises(sdq.Error, match="gate applies"):
        q.linear_combine(x_dev, stream, good, sdq.COMBINE_PRODUCT, gate=sdq.Array.from_numpy(np.ones(64, np.float32)))
    with pytest.raises(sdq.Error, match="combine must be"):
        q.linear_combine(x_dev, stream, good, 9)


@pytest.mark.parametrize("M", [3, 80])
def test_linear_epilogue_f16_activations_and_scales(oracle, sdq, stream, M):
    # f16 x with f16 scales give f16 output; bias in f16; GELU epilogue.
    N, K = 160, 256
    w = oracle.normals(1600 + M, N * K, 0.02).reshape(N, K)
    wh = w.astype(np.float16)
    q = sdq.QuantizedArray.quantize(sdq.Array.from_numpy(wh), 64, 4, stream)
    wq, s, b = oracle.quantize(wh.astype(np.float32), 64, 4, 9)
    deq = oracle.dequantize(wq, s, b, 64, 4, 9)
    x = oracle.normals(1601 + M, M * K).reshape(M, K).astype(np.float16)
    bias = oracle.normals(1602, N).astype(np.float16)
    y = q.linear(sdq.Array.from_numpy(x), stream, bias=sdq.Array.from_numpy(bias),
                 activation=sdq.ACT_GELU_APPROX)
    assert y.dtype == sdq.FLOAT16 and y.shape == [M, N]
    got = y.to_numpy().astype(np.float32)
    want = _gelu64(x.astype(np.float64) @ deq.astype(np.float64).T + bias.astype(np.float64))
    err, cos = max_rel_err(got, want), cosine(got, want)
    assert err <= MAX_REL and cos >= MIN_COS, (err, cos)


@pytest.mark.parametrize("M", [12, 300])
def test_linear_combine_on_flux_token_layout(oracle, sdq, stream, M):
    # Flux feeds [1, seq, K] tokens and adds the gated output to a [1, seq, N]
    # residual stream (flux.rs:389-398).
    N, K = 256, 512
    q, deq = _qweight(oracle, sdq, stream, 1700 + M, N, K, 4)
    x_dev, x_vals = _x(oracle, sdq, 1701 + M, (1, M, K), "bf16")
    r = oracle.normals(1702 + M, M * N).reshape(1, M, N)
    g = oracle.normals(1703, N, 0.3)
    y = q.linear_combine(x_dev, stream, sdq.Array.from_numpy(r), sdq.COMBINE_GATED_RESIDUAL,
                         gate=sdq.Array.from_numpy(g))
    assert y.shape == [1, M, N]
    want = r[0] + g * (x_vals[0].astype(np.float64) @ deq.astype(np.float64).T)
    got = y.to_numpy().reshape(M, N)
    err, cos = max_rel_err(got, want), cosine(got, want)
    assert err <= MAX_REL and cos >= MIN_COS, (err, cos)
