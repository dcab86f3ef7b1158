"""GPU quantize / dequantize through the C ABI, bit-exact against the oracle
on the same seeded inputs (the north star's first parity level)."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

WDT = {"f32": 10, "bf16": 12, "f16": 9}


def _weights(oracle, sdq, seed, shape, wdt):
    """Seeded N(0, 0.02) weights as a device array of dtype `wdt`, and the f32
    values the oracle sees (exact widenings of the stored values)."""
    w = oracle.normals(seed, int(np.prod(shape)), 0.02).reshape(shape)
    code = WDT[wdt]
    if code == 12:
        bits = sdq.f32_to_bf16_bits(w)
        return sdq.Array.from_numpy(bits, sdq.BFLOAT16), sdq.bf16_bits_to_f32(bits).reshape(shape)
    if code == 9:
        h = w.astype(np.float16)
        return sdq.Array.from_numpy(h, sdq.FLOAT16), h.astype(np.float32)
    return sdq.Array.from_numpy(w, sdq.FLOAT32), w


def _raw(a):
    """Device scales/biases as the oracle stores them (f32, or uint16 bits)."""
    v = a.to_numpy()
    return v.view(np.uint16) if v.dtype == np.float16 else v


@pytest.mark.parametrize("wdt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_quantize_is_bit_exact(oracle, sdq, stream, wdt, bits, gs):
    print(f"quantize wdt={wdt} bits={bits} gs={gs}", flush=True)
    w_dev, w_vals = _weights(oracle, sdq, 100 + bits + gs, (64, 512), wdt)
    q = sdq.QuantizedArray.quantize(w_dev, gs, bits, stream)
    assert q.weight.shape == [64, 512 * bits // 32]
    assert q.scales.shape == [64, 512 // gs] and q.scales.dtype == WDT[wdt]
    wq, s, b = oracle.quantize(w_vals, gs, bits, WDT[wdt])
    assert np.array_equal(q.weight.to_numpy(), wq)
    assert np.array_equal(_raw(q.scales), s)
    assert np.array_equal(_raw(q.biases), b)


@pytest.mark.parametrize("sdt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("odt", [None, "f32", "bf16", "f16"])
@pytest.mark.parametrize("bits", [2, 4, 8])
def test_dequantize_is_bit_exact(oracle, sdq, stream, sdt, odt, bits):
    print(f"dequantize sdt={sdt} odt={odt} bits={bits}", flush=True)
    w_dev, w_vals = _weights(oracle, sdq, 200 + bits, (96, 256), sdt)
    q = sdq.QuantizedArray.quantize(w_dev, 64, bits, stream)
    out_code = None if odt is None else WDT[odt]
    d = q.dequantize(stream, out_code)
    assert d.shape == [96, 256]
    assert d.dtype == (WDT[sdt] if odt is None else out_code)
    wq, s, b = oracle.quantize(w_vals, 64, bits, WDT[sdt])
    want_t = oracle.dequantize(wq, s, b, 64, bits, WDT[sdt])  # values in the scale dtype
    got = d.to_numpy()
    oc = d.dtype
    if oc == 10:
        assert np.array_equal(got, want_t)
    elif oc == 12:
        assert np.array_equal(got, sdq.f32_to_bf16_bits(want_t))
    else:
        assert np.array_equal(got, want_t.astype(np.float16))


def test_config1_weight_is_bit_exact(oracle, sdq, stream):
    # W [3072, 3072] ~ N(0, 0.02) f32, 4-bit, group 64;
    # dequantized weights compared bit for bit.
    print("config1 quantize+dequantize 3072x3072", flush=True)
    w = oracle.normals(1001, 3072 * 3072, 0.02).reshape(3072, 3072)
    q = sdq.QuantizedArray.quantize(sdq.Array.from_numpy(w), 64, 4, stream)
    wq, s, b = oracle.quantize(w, 64, 4)
    assert np.array_equal(q.weight.to_numpy(), wq)
    assert np.array_equal(q.scales.to_numpy(), s)
    assert np.array_equal(q.biases.to_numpy(), b)
    assert np.array_equal(q.dequantize(stream).to_numpy(), oracle.dequantize(wq, s, b, 64, 4))


def test_known_answer_groups_on_the_gpu(sdq, stream):
    print("KAT groups", flush=True)
    ramp = np.array([list(range(16)) + [15] * 48], dtype=np.float32)
    ties = np.array([[0.0, 15.0, 0.5, 2.5, 13.5] + [15.0] * 59], dtype=np.float32)
    const = np.full((1, 64), 0.5, dtype=np.float32)
    zero = np.zeros((1, 64), dtype=np.float32)
    w = np.concatenate([ramp, -ramp, ties, const, zero])
    q = sdq.QuantizedArray.quantize(sdq.Array.from_numpy(w), 64, 4, stream)
    wq = q.weight.to_numpy()
    assert wq[0, 0] == 0x89ABCDEF and wq[0, 1] == 0x01234567
    assert wq[1, 0] == 0x89ABCDEF
    assert [(int(wq[2, 0]) >> (4 * e)) & 15 for e in range(5)] == [15, 0, 14, 12, 2]
    assert np.all(wq[3:] == 0)
    d = q.dequantize(stream).to_numpy()
    assert np.array_equal(d[[0, 1, 3, 4]], w[[0, 1, 3, 4]])


def test_leading_dimensions_are_kept(oracle, sdq, stream):
    w = oracle.normals(300, 2 * 16 * 128, 0.02).reshape(2, 16, 128)
    q = sdq.QuantizedArray.quantize(sdq.Array.from_numpy(w), 64, 4, stream)
    assert q.weight.shape == [2, 16, 16] and q.scales.shape == [2, 16, 2]
    wq, s, b = oracle.quantize(w.reshape(32, 128), 64, 4)
    assert np.array_equal(q.weight.to_numpy().reshape(32, 16), wq)
    assert q.dequantize(stream).shape == [2, 16, 128]
