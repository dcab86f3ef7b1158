"""The fused output layouts on the GPU, through the C ABI:

* sdq_quantized_linear_split_raw: columns [0, split) to one buffer, columns
  [split, N) to another at its own row stride and activation.  Each part
  must equal, bit for bit, the same columns of sdq_quantized_linear's output
  with that part's activation (the same kernel and epilogue, only the store
  moves), for the small-M and the large-M kernel, with and without split K.
* sdq_flux_single_linear1_attention (flux.rs:440-465): the result's first
  heads*128 columns equal, bit for bit, sdq_flux_attention on linear1's full
  output, and its remaining columns equal linear1 with the GELU epilogue on
  the MLP columns.  The pieces are themselves checked against the oracle
  elsewhere (test_gpu_matmul.py, test_gpu_block.py); this checks that the
  fused layout moves the same bits.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _weight(oracle, sdq, stream, seed, N, K, bits):
    w = oracle.normals(seed, N * K, 0.02).reshape(N, K)
    return sdq.QuantizedArray.quantize(sdq.Array.from_numpy(w), 64, bits, stream)


def _x(oracle, sdq, seed, shape):
    bits = sdq.f32_to_bf16_bits(oracle.normals(seed, int(np.prod(shape))).reshape(shape))
    return sdq.Array.from_numpy(bits, sdq.BFLOAT16)


@pytest.mark.parametrize("M,N,K,split,bits", [
    (4, 1280, 512, 768, 4),       # small-M kernel
    (200, 1280, 512, 512, 8),     # large-M kernel, whole tiles
    (300, 1024, 8192, 256, 4),    # large-M kernel, split K (reduction kernel stores)
])
def test_split_store_matches_the_plain_linear(oracle, sdq, stream, M, N, K, split, bits):
    print(f"split store M={M} N={N} K={K} split={split} bits={bits}", flush=True)
    L = sdq.lib()
    q = _weight(oracle, sdq, stream, 5000 + N + bits, N, K, bits)
    x = _x(oracle, sdq, 5001 + M, (M, K))
    bias = sdq.Array.from_numpy(oracle.normals(5002, N))
    ld2 = (N - split) + 64  # a wider second buffer: the row stride is honoured
    lo = sdq.Array.from_numpy(np.zeros((M, split), np.uint16), sdq.BFLOAT16)
    hi = sdq.Array.from_numpy(np.zeros((M, ld2), np.uint16), sdq.BFLOAT16)
    stream.synchronize()
    rc = L.sdq_quantized_linear_split_raw(
        lo.device_ptr, split, sdq.ACT_NONE, hi.device_ptr, ld2, sdq.ACT_GELU_APPROX, split, sdq.BFLOAT16,
        x.device_ptr, sdq.BFLOAT16, K, q.weight.device_ptr, q.scales.device_ptr, q.biases.device_ptr,
        sdq.FLOAT32, M, N, K, 64, bits, bias.device_ptr, sdq.FLOAT32, stream.native)
    if rc:
        sdq._check(rc, "split")
    stream.synchronize()
    xs = sdq.Array.from_numpy(x.to_numpy(), sdq.BFLOAT16)  # same bits, as a bf16 array
    plain = q.linear(xs, stream, bias=bias).astype(sdq.BFLOAT16, stream).to_numpy()
    gelu = q.linear(xs, stream, bias=bias, activation=sdq.ACT_GELU_APPROX).astype(sdq.BFLOAT16, stream).to_numpy()
    got_lo, got_hi = lo.to_numpy(), hi.to_numpy()
    assert np.array_equal(got_lo, plain[:, :split])
    assert np.array_equal(got_hi[:, :N - split], gelu[:, split:])
    assert not got_hi[:, N - split:].any()  # the padding columns are untouched


@pytest.mark.parametrize("T,heads,hidden,mlp,bits", [
    (256, 2, 256, 512, 4),
    (4608, 24, 3072, 12288, 4),  # Flux single block at 1024x1024 (config 4's linear1)
])
def test_single_linear1_attention_matches_the_composition(oracle, sdq, stream, T, heads, hidden, mlp, bits):
    from sdq import flux

    print(f"single linear1+attention T={T} heads={heads} hidden={hidden} mlp={mlp}", flush=True)
    h = heads * 128
    N1 = 3 * h + mlp
    q1 = _weight(oracle, sdq, stream, 5100 + T, N1, hidden, bits)
    x = _x(oracle, sdq, 5101 + T, (1, T, hidden))
    bias = sdq.Array.from_numpy(oracle.normals(5102, N1))
    rng = np.random.default_rng(5103)
    nq = sdq.Array.from_numpy(sdq.f32_to_bf16_bits((1 + 0.2 * rng.standard_normal(128)).astype(np.float32)),
                              sdq.BFLOAT16)
    nk = sdq.Array.from_numpy(sdq.f32_to_bf16_bits((1 + 0.2 * rng.standard_normal(128)).astype(np.float32)),
                              sdq.BFLOAT16)
    ids = np.stack([np.zeros(T), np.arange(T) // 64, np.arange(T) % 64], 1).astype(np.float32)
    pe = flux.embed_nd(ids, T, [16, 56, 56], 10000.0)
    joined = flux.single_linear1_attention(x, q1, bias, nq, nk, pe, heads, stream)
    assert joined.shape == [1, T, h + mlp]
    projected = q1.linear(x, stream, bias=bias)
    attn = flux.attention(projected, nq, nk, pe, heads, stream)
    act = q1.linear(x, stream, bias=bias, activation=sdq.ACT_GELU_APPROX)
    got = joined.to_numpy().reshape(T, h + mlp)
    assert joined.dtype == attn.dtype == act.dtype
    assert np.array_equal(got[:, :h], attn.to_numpy().reshape(T, h))
    assert np.array_equal(got[:, h:], act.to_numpy().reshape(T, N1)[:, 3 * h:])


def test_layout_errors(oracle, sdq, stream):
    L = sdq.lib()
    q = _weight(oracle, sdq, stream, 5200, 512, 256, 4)
    x = _x(oracle, sdq, 5201, (8, 256))
    out = sdq.Array.from_numpy(np.zeros((8, 512), np.float32))
    for split, msg in ((100, "multiple of 256"), (512, "inside \\(0, N\\)")):
        rc = L.sdq_quantized_linear_split_raw(
            out.device_ptr, 512, 0, out.device_ptr, 512, 0, split, sdq.FLOAT32, x.device_ptr, sdq.BFLOAT16,
            256, q.weight.device_ptr, q.scales.device_ptr, q.biases.device_ptr, sdq.FLOAT32, 8, 512, 256, 64, 4,
            None, 0, stream.native)
        assert rc != 0
        with pytest.raises(sdq.Error, match=msg):
            sdq._check(rc, "split")
    from sdq import flux

    pe = flux.embed_nd(np.zeros((8, 3), np.float32), 8, [16, 56, 56], 10000.0)
    nrm = sdq.Array.from_numpy(np.ones(128, np.float32))
    with pytest.raises(sdq.Error, match="even head count"):
        flux.single_linear1_attention(sdq.Array.from_numpy(np.zeros((1, 8, 256), np.float32)),
                                      _weight(oracle, sdq, stream, 5202, 3 * 128 + 256, 256, 4), None, nrm, nrm,
                                      pe, 1, stream)
