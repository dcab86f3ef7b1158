"""The elementwise ops around the linear, and argument validation of the
path's entry points (a status and a message, never an abort)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_gelu_approx_matches_the_oracle(oracle, sdq, stream):
    x = np.concatenate([np.linspace(-8, 8, 1001, dtype=np.float32), oracle.normals(3, 5000) * 3]).astype(np.float32)
    got = sdq.Array.from_numpy(x).gelu_approx(stream).to_numpy()
    assert np.max(np.abs(got - oracle.gelu_approx(x))) < 2e-6


@pytest.mark.parametrize("n", [1, 7, 8, 4096 + 5])
def test_gelu_approx_bf16_and_ragged_lengths(oracle, sdq, stream, n):
    # bf16 in and out, 16-byte groups of eight plus a ragged tail: within the
    # f32 bound of the test above plus one bf16 rounding of the output, against
    # the oracle applied to the same (bf16) inputs.
    x = (oracle.normals(5 + n, n) * 3).astype(np.float32)
    bits = sdq.f32_to_bf16_bits(x)
    xr = sdq.bf16_bits_to_f32(bits)
    got = sdq.bf16_bits_to_f32(sdq.Array.from_numpy(bits, sdq.BFLOAT16).gelu_approx(stream).to_numpy())
    want = oracle.gelu_approx(xr)
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -8 + 2e-6)
    f = sdq.Array.from_numpy(x).gelu_approx(stream).to_numpy()
    assert np.max(np.abs(f - oracle.gelu_approx(x))) < 2e-6


def test_astype_round_trips(oracle, sdq, stream):
    x = oracle.normals(4, 4096)
    a = sdq.Array.from_numpy(x)
    b = a.astype(sdq.BFLOAT16, stream)
    assert np.array_equal(b.to_numpy(), sdq.f32_to_bf16_bits(x))
    h = a.astype(sdq.FLOAT16, stream)
    assert np.array_equal(h.to_numpy(), x.astype(np.float16))
    assert np.array_equal(b.astype(sdq.FLOAT32, stream).to_numpy(), sdq.bf16_bits_to_f32(sdq.f32_to_bf16_bits(x)))


def test_add_and_multiply(oracle, sdq, stream):
    a = oracle.normals(8, 6 * 32).reshape(6, 32)
    b = oracle.normals(9, 6 * 32).reshape(6, 32)
    bias = oracle.normals(10, 32)
    A, B = sdq.Array.from_numpy(a), sdq.Array.from_numpy(b)
    assert np.array_equal(A.add(B, stream).to_numpy(), a + b)
    assert np.array_equal(A.mul(B, stream).to_numpy(), a * b)
    assert np.array_equal(A.add(sdq.Array.from_numpy(bias), stream).to_numpy(), a + bias)
    with pytest.raises(sdq.Error, match="broadcast"):
        A.add(sdq.Array.from_numpy(np.zeros(7, np.float32)), stream)


def _q(sdq, stream, shape=(64, 128), bits=4, gs=64):
    w = np.random.default_rng(0).standard_normal(shape).astype(np.float32) * 0.02
    return sdq.QuantizedArray.quantize(sdq.Array.from_numpy(w), gs, bits, stream)


def test_quantize_rejects_bad_arguments(sdq, stream):
    w = sdq.Array.from_numpy(np.zeros((32, 100), np.float32))
    with pytest.raises(sdq.Error, match="divisible by the quantization group size 64"):
        sdq.QuantizedArray.quantize(w, 64, 4, stream)
    w2 = sdq.Array.from_numpy(np.zeros((32, 128), np.float32))
    with pytest.raises(sdq.Error, match="group size 48"):
        sdq.QuantizedArray.quantize(w2, 48, 4, stream)
    with pytest.raises(sdq.Error, match="bits 3"):
        sdq.QuantizedArray.quantize(w2, 64, 3, stream)
    with pytest.raises(sdq.Error, match="at least 2 dimensions"):
        sdq.QuantizedArray.quantize(sdq.Array.from_numpy(np.zeros(128, np.float32)), 64, 4, stream)
    L = sdq.lib()
    out = sdq.CVectorArray(None)
    rc = L.sdq_quantize(ctypes.byref(out), w2._raw, sdq.COptionalInt(64, True), sdq.COptionalInt(4, True),
                        b"mxfp4", sdq.CArray(None), stream._raw)
    assert rc != 0
    with pytest.raises(sdq.Error, match="mode"):
        sdq._check(rc, "quantize")


def test_matmul_rejects_mismatches(sdq, stream):
    q = _q(sdq, stream)
    with pytest.raises(sdq.Error, match="Last dimension"):
        q.matmul(sdq.Array.from_numpy(np.zeros((4, 100), np.float32)), stream)
    wrong_bits = sdq.QuantizedArray(q.weight, q.scales, q.biases, 64, 8)
    with pytest.raises(sdq.Error):
        wrong_bits.matmul(sdq.Array.from_numpy(np.zeros((4, 128), np.float32)), stream)
    L = sdq.lib()
    res = sdq.CArray(None)
    x = sdq.Array.from_numpy(np.zeros((4, 128), np.float32))
    rc = L.sdq_quantized_matmul(ctypes.byref(res), x._raw, q.weight._raw, q.scales._raw, q.biases._raw,
                                False, sdq.COptionalInt(64, True), sdq.COptionalInt(4, True), b"affine",
                                stream._raw)
    assert rc != 0 and res.ctx is None
    with pytest.raises(sdq.Error, match="transpose"):
        sdq._check(rc, "quantized_matmul")
    # A failed call leaves an existing result handle untouched.
    good = q.matmul(x, stream)
    before = good.to_numpy().copy()
    rc = L.sdq_quantized_matmul(ctypes.byref(good._raw), x._raw, q.weight._raw, q.scales._raw,
                                q.biases._raw, False, sdq.COptionalInt(64, True),
                                sdq.COptionalInt(4, True), b"affine", stream._raw)
    assert rc != 0
    sdq._take_last_error()
    assert np.array_equal(good.to_numpy(), before)


def test_dequantize_rejects_mismatched_scales(sdq, stream):
    q = _q(sdq, stream)
    bad = sdq.QuantizedArray(q.weight, q.scales, q.biases, 32, 4)
    with pytest.raises(sdq.Error, match="does not match"):
        bad.dequantize(stream)


def test_empty_batch_gives_an_empty_result(sdq, stream):
    q = _q(sdq, stream)
    y = q.matmul(sdq.Array.from_numpy(np.zeros((0, 128), np.float32)), stream)
    assert y.shape == [0, 64]


def test_memory_accounting_moves(sdq, stream):
    before = sdq.active_memory()
    a = sdq.Array.from_numpy(np.zeros((1024, 1024), np.float32))
    assert sdq.active_memory() >= before + 4 * 1024 * 1024
    assert sdq.peak_memory() >= sdq.active_memory()
    del a
    assert sdq.cache_memory() >= 4 * 1024 * 1024
