"""T5's gated feed-forward through the host mirror (sdq/t5.py, after
crates/sd-models/src/mlx/t5.rs:201-214): with quantized wi_0/wi_1 it pairs
them once and runs the gated launch; with a dense projection it issues the
reference's sequence.  Both against the oracle's f64 composition
gelu_new(x W0^T) * (x W1^T) @ Wo^T, to the north star's bar (max |d| /
max |ref| <= 2e-2, cosine >= 0.9999), at the small-M and the large-M kernel.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import cosine, max_rel_err

pytestmark = pytest.mark.gpu


def _gelu64(v):
    return 0.5 * v * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (v + 0.044715 * v ** 3)))


@pytest.mark.parametrize("T", [8, 96])
@pytest.mark.parametrize("dense_up", [False, True])
def test_feed_forward_matches_the_oracle(oracle, sdq, stream, T, dense_up):
    from sdq import t5
    from sdq.quantized import QuantizedWeights

    D, F = 512, 1024
    print(f"t5 feed_forward T={T} dense_up={dense_up}", flush=True)
    ws = {"wi_0": oracle.normals(8000, F * D, 0.05).reshape(F, D),
          "wi_1": oracle.normals(8001, F * D, 0.05).reshape(F, D),
          "wo": oracle.normals(8002, D * F, 0.05).reshape(D, F)}
    bits = {"wi_0": 4, "wi_1": 4, "wo": 8}
    quantized, dense, deq = {}, {}, {}
    for name, w in ws.items():
        key = f"enc.ff.{name}.weight"
        if dense_up and name == "wi_1":
            dense[key] = sdq.Array.from_numpy(w)
            deq[name] = w.astype(np.float64)
            continue
        quantized[key] = sdq.QuantizedArray.quantize(sdq.Array.from_numpy(w), 64, bits[name], stream)
        wq, sc, bi = oracle.quantize(w, 64, bits[name])
        deq[name] = oracle.dequantize(wq, sc, bi, 64, bits[name]).astype(np.float64)
    w = QuantizedWeights(quantized, dense)
    xb = sdq.f32_to_bf16_bits(oracle.normals(8003 + T, T * D).reshape(1, T, D))
    x = sdq.Array.from_numpy(xb, sdq.BFLOAT16)
    y = t5.feed_forward(x, w, "enc.ff", stream)
    assert y.shape == [1, T, D]
    got = y.to_float32().reshape(T, D)
    xv = sdq.bf16_bits_to_f32(xb).reshape(T, D).astype(np.float64)
    h = _gelu64(xv @ deq["wi_0"].T) * (xv @ deq["wi_1"].T)
    want = h @ deq["wo"].T
    err, cos = max_rel_err(got, want), cosine(got, want)
    assert err <= 2e-2 and cos >= 0.9999, (err, cos)
    # The paired operand is built once and reused.
    assert (("_t5_pairs" in w.__dict__) == (not dense_up))
    if not dense_up:
        pairs = dict(w.__dict__["_t5_pairs"])
        t5.feed_forward(x, w, "enc.ff", stream)
        assert w.__dict__["_t5_pairs"].keys() == pairs.keys()
