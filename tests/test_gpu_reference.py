"""The reference's own hot-path tests (crates/sd-models/tests/mlx_quantized.rs),
restated over libsdq on the GPU with the same inputs and thresholds."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import cosine, ramp_activation, ramp_weight

pytestmark = pytest.mark.gpu


def test_the_round_trip_cost_is_what_the_bit_width_says(sdq, stream):
    # mlx_quantized.rs:53-75
    w = sdq.Array.from_numpy(ramp_weight(256, 512))
    dense = w.to_vec_f32(stream)
    previous = 0.0
    for bits in (4, 8):
        q = sdq.QuantizedArray.quantize(w, 64, bits, stream)
        back = q.dequantize(stream)
        assert back.shape == w.shape
        c = cosine(dense, back.to_vec_f32(stream))
        print(f"{bits}-bit round trip: cosine {c:.6f}")
        assert c > 0.99
        assert c > previous
        previous = c


def test_the_quantized_matmul_agrees_with_the_dense_one(sdq, stream):
    # mlx_quantized.rs:83-117
    out, inp = 256, 512
    w = sdq.Array.from_numpy(ramp_weight(out, inp))
    x = sdq.Array.from_numpy(ramp_activation(8, inp))
    want = x.matmul_nt(w, stream).to_vec_f32(stream)
    for bits in (4, 8):
        q = sdq.QuantizedArray.quantize(w, 64, bits, stream)
        got = q.matmul(x, stream)
        assert got.shape == [8, out]
        c = cosine(want, got.to_vec_f32(stream))
        print(f"{bits}-bit matmul: cosine {c:.6f}")
        assert c > 0.999


def test_quantising_shrinks_the_weight_by_what_it_claims(sdq, stream):
    # mlx_quantized.rs:120-141
    w = sdq.Array.from_numpy(ramp_weight(1024, 1024))
    dense_bytes = 1024 * 1024 * 4
    for bits, most in ((4, 0.20), (8, 0.35)):
        q = sdq.QuantizedArray.quantize(w, 64, bits, stream)
        ratio = q.resident_bytes() / dense_bytes
        assert ratio < most
        assert ratio == {4: 0.15625, 8: 0.28125}[bits]


def test_the_split_leaves_norms_and_odd_widths_dense(sdq, stream):
    # mlx_quantized.rs:148-179
    from sdq import quantized

    w = {
        "blk.0.attn.weight": sdq.Array.from_numpy(ramp_weight(128, 256)),
        "blk.0.attn.bias": sdq.Array.from_numpy(np.zeros(128, np.float32)),
        "blk.0.norm.weight": sdq.Array.from_numpy(np.ones(128, np.float32)),
        "blk.0.odd.weight": sdq.Array.from_numpy(ramp_weight(32, 100)),
    }
    q = quantized.from_dense(w, quantized.DEFAULT_BITS, stream)
    assert "blk.0.attn.weight" in q.quantized
    assert "blk.0.attn.bias" in q.dense
    assert "blk.0.norm.weight" in q.dense
    assert "blk.0.odd.weight" in q.dense
    assert len(q) == 4
    for name in w:
        assert q.contains_key(name)


def test_the_linear_dispatches_to_the_right_kernel(sdq, stream):
    # mlx_quantized.rs:182-228
    from sdq import quantized

    dense_map = {
        "big.weight": sdq.Array.from_numpy(ramp_weight(128, 256)),
        "small.weight": sdq.Array.from_numpy(ramp_weight(8, 32)),
    }
    x_big = sdq.Array.from_numpy(ramp_activation(4, 256))
    x_small = sdq.Array.from_numpy(ramp_activation(4, 32))
    want_big = ramp_activation(4, 256).astype(np.float64) @ ramp_weight(128, 256).astype(np.float64).T
    want_small = ramp_activation(4, 32).astype(np.float64) @ ramp_weight(8, 32).astype(np.float64).T

    q = quantized.from_dense(dense_map, 8, stream)
    assert "big.weight" in q.quantized
    assert "small.weight" in q.dense

    got_big = quantized.linear(x_big, "big.weight", None, q, stream)
    assert cosine(want_big, got_big.to_vec_f32(stream)) > 0.999

    got_small = np.array(quantized.linear(x_small, "small.weight", None, q, stream).to_vec_f32(stream))
    worst = np.max(np.abs(want_small.ravel() - got_small))
    assert worst < 1e-5, "the dense branch is not the dense matmul"

    with pytest.raises(sdq.Error):
        quantized.linear(x_big, "absent.weight", None, q, stream)


def test_the_bias_is_added_after_the_matmul(sdq, stream, oracle):
    # quantized.rs:314-317
    from sdq import quantized

    w = {"lin.weight": sdq.Array.from_numpy(oracle.normals(5, 96 * 128, 0.02).reshape(96, 128))}
    q = quantized.from_dense(w, 4, stream)
    x = sdq.Array.from_numpy(oracle.normals(6, 3 * 128).reshape(3, 128))
    bias_np = oracle.normals(7, 96)
    plain = np.array(quantized.linear(x, "lin.weight", None, q, stream).to_vec_f32(stream)).reshape(3, 96)
    with_bias = quantized.linear(x, "lin.weight", sdq.Array.from_numpy(bias_np), q, stream)
    got = np.array(with_bias.to_vec_f32(stream)).reshape(3, 96)
    assert np.array_equal(got, (plain + bias_np).astype(np.float32))


def test_dense_reach_into_a_quantized_name_is_refused(sdq, stream):
    # quantized.rs:364-375
    from sdq import quantized

    q = quantized.from_dense({"w": sdq.Array.from_numpy(ramp_weight(64, 64))}, 4, stream)
    with pytest.raises(sdq.Error, match="quantised"):
        q.dense_tensor("w")
    with pytest.raises(sdq.Error, match="missing"):
        q.dense_tensor("nope")
    assert q.optional("w") is None
