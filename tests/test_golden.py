"""Golden vectors (tests/golden/quantized_linear.npz, written by
tests/golden/make_golden.py from the oracle).

CPU: the oracle must still reproduce every array bit for bit.
GPU: libsdq's quantize and dequantize must match the fixture bit for bit and
its quantized_matmul must meet the tolerance against the fixture's output,
for every stored-scale dtype, bit width and group size the fixture holds.
The fixture is read with numpy's default loader (no pickles).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

from conftest import cosine, max_rel_err

GOLDEN_DIR = Path(__file__).resolve().parent / "golden"
GOLDEN = GOLDEN_DIR / "quantized_linear.npz"
if str(GOLDEN_DIR) not in sys.path:
    sys.path.insert(0, str(GOLDEN_DIR))
STORE = {"f32": 10, "bf16": 12, "f16": 9}


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN) as d:
        return {k: d[k] for k in d.files}


def test_fixture_is_complete(golden):
    for s in STORE:
        for bits in (2, 4, 8):
            for gs in (32, 64, 128):
                for part in ("wq", "scales", "biases", "deq", "y"):
                    assert f"{part}_{s}_b{bits}_g{gs}" in golden
    assert golden["x"].shape == (5, 256) and golden["w"].shape == (6, 256)


def test_oracle_reproduces_the_fixture(golden):
    import make_golden

    fresh = make_golden.make()
    assert sorted(fresh) == sorted(golden)
    for k, v in fresh.items():
        assert v.dtype == golden[k].dtype, k
        assert np.array_equal(v.view(np.uint8), golden[k].view(np.uint8)), k


def _raw(a):
    v = a.to_numpy()
    return v.view(np.uint16) if v.dtype == np.float16 else v


def _device_weight(sdq, w, store):
    if store == 12:
        return sdq.Array.from_numpy(sdq.f32_to_bf16_bits(w), sdq.BFLOAT16)
    if store == 9:
        return sdq.Array.from_numpy(w.astype(np.float16), sdq.FLOAT16)
    return sdq.Array.from_numpy(w, sdq.FLOAT32)


@pytest.mark.gpu
@pytest.mark.parametrize("sname", list(STORE))
@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_gpu_matches_the_fixture(golden, sdq, stream, sname, bits, gs):
    key = f"{sname}_b{bits}_g{gs}"
    print(f"golden {key}", flush=True)
    store = STORE[sname]
    q = sdq.QuantizedArray.quantize(_device_weight(sdq, golden[f"w_{sname}"], store), gs, bits, stream)
    assert np.array_equal(q.weight.to_numpy(), golden[f"wq_{key}"])
    assert np.array_equal(_raw(q.scales), golden[f"scales_{key}"])
    assert np.array_equal(_raw(q.biases), golden[f"biases_{key}"])
    d = q.dequantize(stream, 10).to_numpy()  # values in the scale dtype, widened
    assert np.array_equal(d, golden[f"deq_{key}"])
    if bits in (4, 8) and gs in (64, 128):
        x = sdq.Array.from_numpy(golden["x"])
        y = q.matmul(x, stream).to_numpy()
        want = golden[f"y_{key}"]
        assert max_rel_err(y, want) <= 2e-2 and cosine(y, want) >= 0.9999
