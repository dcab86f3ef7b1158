"""T5's gated feed-forward input in one launch, through the C ABI:
y = gelu_new(x @ wi_0.T) * (x @ wi_1.T) (t5.rs:201-214) from the two
quantized weights with their rows interleaved in blocks of eight
(sdq_pair_rows, sdq_quantized_linear_gated, sdq_quantized_linear_gated_raw).

The fused op computes the product in f32 from the two accumulators, so it is
compared with a tolerance, not bit for bit: against the oracle's quantized
matmul and GELU at small shapes, to the north star's bar (max |d| / max |ref|
<= 2e-2, cosine >= 0.9999: the large-M kernel multiplies bf16-rounded
dequantized weights), and against the composition of the two
device linears (each checked against the oracle elsewhere) at T5-XXL's
shapes (d_model 4096, d_ff 10240) for the small-M kernel (M = 1, 4, 16, 32)
and the large-M kernel (512 tokens), and at shapes that take the split-K
reduction, the stream-K path and a ragged last tile.  A mistake in the
pairing (a wrong partner column, a wrong output column) moves values by
O(1), far outside the tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import cosine, max_rel_err

pytestmark = pytest.mark.gpu

# f32 products of two ~1-sized dot products over K <= 16384 terms, summed in
# a different order (the paired launch splits K differently from the two
# single launches) and through the device GELU: agreement to ~1e-6 relative
# is expected; 1e-4 leaves room and still catches any misplaced column.
RTOL, ATOL = 1e-4, 1e-4


def _gelu(v):
    v = v.astype(np.float64)
    return 0.5 * v * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (v + 0.044715 * v ** 3)))


def _x(oracle, sdq, seed, M, K):
    bits = sdq.f32_to_bf16_bits(oracle.normals(seed, M * K).reshape(M, K))
    return bits, sdq.Array.from_numpy(bits, sdq.BFLOAT16)


def _pair(oracle, sdq, stream, seed, N, K, bits):
    ws = [oracle.normals(seed + i, N * K, 0.02).reshape(N, K) for i in range(2)]
    qs = [sdq.QuantizedArray.quantize(sdq.Array.from_numpy(w), 64, bits, stream) for w in ws]
    return qs, sdq.QuantizedArray.pair(qs[0], qs[1], stream)


def test_pair_rows_interleaves_blocks_of_eight(sdq, stream):
    g = np.arange(24 * 5, dtype=np.uint32).reshape(24, 5)
    u = (1000 + np.arange(24 * 5, dtype=np.uint32)).reshape(24, 5)
    got = sdq.pair_rows(sdq.Array.from_numpy(g), sdq.Array.from_numpy(u), stream).to_numpy()
    want = np.concatenate([g.reshape(3, 8, 5), u.reshape(3, 8, 5)], axis=1).reshape(48, 5)
    assert got.shape == (48, 5) and np.array_equal(got, want)
    b = sdq.pair_rows(sdq.Array.from_numpy(np.arange(16, dtype=np.float32)),
                      sdq.Array.from_numpy(-np.arange(16, dtype=np.float32)), stream).to_numpy()
    assert np.array_equal(b, np.r_[0:8, -np.r_[0:8], 8:16, -np.r_[8:16]].astype(np.float32))
    with pytest.raises(sdq.Error, match="multiple of 8"):
        sdq.pair_rows(sdq.Array.from_numpy(np.zeros((12, 4), np.float32)),
                      sdq.Array.from_numpy(np.zeros((12, 4), np.float32)), stream)
    with pytest.raises(sdq.Error, match="share one shape"):
        sdq.pair_rows(sdq.Array.from_numpy(np.zeros((16, 4), np.float32)),
                      sdq.Array.from_numpy(np.zeros((16, 8), np.float32)), stream)


@pytest.mark.parametrize("M,N,K,bits", [(1, 256, 512, 4), (5, 136, 256, 8), (40, 264, 512, 4)])
def test_gated_matches_the_oracle(oracle, sdq, stream, M, N, K, bits):
    print(f"gated vs oracle M={M} N={N} K={K} bits={bits}", flush=True)
    xb, x = _x(oracle, sdq, 6000 + M, M, K)
    ws = [oracle.normals(6001 + i, N * K, 0.02).reshape(N, K) for i in range(2)]
    qs = [sdq.QuantizedArray.quantize(sdq.Array.from_numpy(w), 64, bits, stream) for w in ws]
    pair = sdq.QuantizedArray.pair(qs[0], qs[1], stream)
    got = pair.linear_gated(x, stream).to_numpy()
    assert got.shape == (M, N)
    xf = sdq.bf16_bits_to_f32(xb)
    ys = []
    for w in ws:
        wq, sc, bi = oracle.quantize(w, 64, bits)
        ys.append(oracle.qmatmul(xf, wq, sc, bi, 64, bits).astype(np.float64))
    want = _gelu(ys[0]) * ys[1]
    err, cos = max_rel_err(got, want), cosine(got, want)
    assert err <= 2e-2 and cos >= 0.9999, (err, cos)


@pytest.mark.parametrize("M,N,K,bits", [
    (1, 10240, 4096, 4),     # T5-XXL wi_0/wi_1, one token (small-M kernel)
    (4, 10240, 4096, 8),
    (16, 10240, 4096, 4),
    (32, 10240, 4096, 4),    # two 16-row blocks
    (512, 10240, 4096, 4),   # T5-XXL at 512 tokens (large-M kernel, whole tiles)
    (512, 10240, 4096, 8),
    (300, 512, 8192, 4),     # split K: the pair is formed in the reduction kernel
    (48, 10240, 4096, 4),    # 64-row tiles, split K
    (64, 512, 256, 8),       # 64-row tiles, whole
    (200, 520, 512, 8),      # a ragged last tile (1040 paired rows)
    (4096, 1536, 12288, 4),  # stream-K (long K, tiles just short of the CUs)
])
def test_gated_matches_the_composition(oracle, sdq, stream, M, N, K, bits):
    print(f"gated vs composition M={M} N={N} K={K} bits={bits}", flush=True)
    _, x = _x(oracle, sdq, 6100 + M, M, K)
    (qg, qu), pair = _pair(oracle, sdq, stream, 6101 + N, N, K, bits)
    got = pair.linear_gated(x, stream).to_numpy()
    g = qg.linear(x, stream).to_numpy().astype(np.float64)
    u = qu.linear(x, stream).to_numpy().astype(np.float64)
    np.testing.assert_allclose(got, _gelu(g) * u, rtol=RTOL, atol=ATOL)


def test_gated_bias_and_bf16_output(oracle, sdq, stream):
    M, N, K = 64, 512, 1024
    _, x = _x(oracle, sdq, 6200, M, K)
    ws = [oracle.normals(6201 + i, N * K, 0.02).reshape(N, K) for i in range(2)]
    qs = [sdq.QuantizedArray.quantize(sdq.Array.from_numpy(sdq.f32_to_bf16_bits(w), sdq.BFLOAT16), 64, 4,
                                      stream) for w in ws]
    pair = sdq.QuantizedArray.pair(qs[0], qs[1], stream)
    bg, bu = oracle.normals(6203, N), oracle.normals(6204, N)
    bias = sdq.pair_rows(sdq.Array.from_numpy(bg), sdq.Array.from_numpy(bu), stream)
    got = pair.linear_gated(x, stream, bias=bias)
    assert got.dtype == sdq.BFLOAT16
    got = sdq.bf16_bits_to_f32(got.to_numpy())
    # The composition in f32: the same products, bf16 operands, f32 outputs.
    g = qs[0].linear(x, stream).astype(sdq.FLOAT32, stream).to_numpy().astype(np.float64)
    u = qs[1].linear(x, stream).astype(sdq.FLOAT32, stream).to_numpy().astype(np.float64)
    # bf16 linears round their outputs: compare at bf16 resolution (2^-8).
    want = _gelu(g + bg) * (u + bu)
    np.testing.assert_allclose(got, want, rtol=2e-2, atol=2e-2)
    # Without the activation: a plain product of the two biased linears.
    plain = sdq.bf16_bits_to_f32(pair.linear_gated(x, stream, bias=bias, activation=sdq.ACT_NONE).to_numpy())
    np.testing.assert_allclose(plain, (g + bg) * (u + bu), rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("M", [3, 200])
def test_gated_raw_honours_the_row_stride(oracle, sdq, stream, M):
    L = sdq.lib()
    N, K = 256, 512
    _, x = _x(oracle, sdq, 6300 + M, M, K)
    (qg, qu), pair = _pair(oracle, sdq, stream, 6301, N, K, 4)
    ld = N + 40
    out = sdq.Array.from_numpy(np.zeros((M, ld), np.float32))
    stream.synchronize()
    rc = L.sdq_quantized_linear_gated_raw(
        out.device_ptr, ld, sdq.FLOAT32, x.device_ptr, sdq.BFLOAT16, K, pair.weight.device_ptr,
        pair.scales.device_ptr, pair.biases.device_ptr, sdq.FLOAT32, M, 2 * N, K, 64, 4, None, 0,
        sdq.ACT_GELU_APPROX, stream.native)
    if rc:
        sdq._check(rc, "gated_raw")
    stream.synchronize()
    got = out.to_numpy()
    want = pair.linear_gated(x, stream).to_numpy()
    assert np.array_equal(got[:, :N], want)  # the same launch shape: the same bits
    assert not got[:, N:].any()
    rc = L.sdq_quantized_linear_gated_raw(
        out.device_ptr, 0, sdq.FLOAT32, x.device_ptr, sdq.BFLOAT16, K, pair.weight.device_ptr,
        pair.scales.device_ptr, pair.biases.device_ptr, sdq.FLOAT32, M, 2 * N - 8, K, 64, 4, None, 0,
        sdq.ACT_GELU_APPROX, stream.native)
    assert rc != 0
    with pytest.raises(sdq.Error, match="multiple of 16"):
        sdq._check(rc, "gated_raw")
