"""GGUF blocks decoded and requantized on the device (gguf.hip, through
sdq_gguf_dequantize / sdq_gguf_quantize) against the oracle's decoders
(oracle/sdq_oracle_gguf.c, pinned in test_oracle_gguf.py).

Decoding is bit-exact: every value as mlx_gguf.rs:324-438 computes it, NaN
scales included (the reference's canonical NaN).  Requantization is
bit-exact against the oracle's quantize of the oracle's decoded f32 values:
the loader's dequantize -> from_slice_f32 -> quantize (quantized.rs:190-196).
"""
from __future__ import annotations

import numpy as np
import pytest

import gguf_blocks as gb

pytestmark = pytest.mark.gpu


def _same_bits(got: np.ndarray, want: np.ndarray) -> None:
    """Every bit pattern equal, NaNs included: F32 and BF16 NaNs keep their
    payload, f16-scaled values carry the reference's canonical NaN."""
    got = np.asarray(got, np.float32).ravel()
    want = np.asarray(want, np.float32).ravel()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, (f"{bad.size} values differ, first at {bad[:4]}: "
                           f"{got.view(np.uint32)[bad[:4]]} vs {want.view(np.uint32)[bad[:4]]}")


# Element counts: one whole launch block (2048 values), a ragged last block,
# and several blocks.  For the per-element types also counts that are not a
# multiple of 8.
SIZES = {
    gb.F32: [1, 7, 2048, 5003, 70001], gb.F16: [3, 2048, 4099, 70001], gb.BF16: [5, 2048, 9001],
    gb.Q4_0: [32, 2048, 2080, 65536 + 96], gb.Q8_0: [32, 2048, 4128, 65536 + 32],
    gb.Q4_K: [256, 2048, 2304, 65536 + 768], gb.Q5_K: [256, 2304, 65536 + 256],
    gb.Q6_K: [256, 2048, 2560, 65536 + 512],
}


@pytest.mark.parametrize("kind", gb.ALL_TYPES)
@pytest.mark.parametrize("finite", [True, False])
def test_dequantize_bit_exact(sdq, oracle, stream, kind, finite):
    rng = np.random.default_rng(100 + kind + (0 if finite else 1000))
    for n in SIZES[kind]:
        print(f"gguf dequantize type={kind} n={n} finite={finite}", flush=True)
        raw = gb.random_tensor(kind, n, rng, finite=finite)
        got = sdq.gguf_dequantize(raw, kind, [n], stream).to_numpy()
        want = oracle.gguf_dequantize(np.frombuffer(raw, np.uint8), kind, n)
        _same_bits(got, want)


def test_every_f16_pattern(sdq, oracle, stream):
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = sdq.gguf_dequantize(pats.tobytes(), gb.F16, [256, 256], stream).to_numpy()
    assert got.shape == (256, 256)
    _same_bits(got, oracle.gguf_dequantize(pats.view(np.uint8), gb.F16, 65536))


@pytest.mark.parametrize("kind", gb.ALL_TYPES)
@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_requantize_bit_exact(sdq, oracle, stream, kind, bits, gs):
    rng = np.random.default_rng(7 * kind + bits + gs)
    for rows, cols in ((3, 256), (17, 512), (40, 768)):
        print(f"gguf quantize type={kind} bits={bits} gs={gs} shape=[{rows},{cols}]", flush=True)
        raw = gb.random_tensor(kind, rows * cols, rng)
        q = sdq.QuantizedArray.from_gguf_blocks(raw, kind, [rows, cols], gs, bits, stream)
        w = oracle.gguf_dequantize(np.frombuffer(raw, np.uint8), kind, rows * cols).reshape(rows, cols)
        wq, sc, bi = oracle.quantize(w, gs, bits)
        assert q.weight.shape == [rows, cols * bits // 32]
        assert q.scales.shape == [rows, cols // gs] and q.scales.dtype == sdq.FLOAT32
        assert np.array_equal(q.weight.to_numpy(), wq)
        assert np.array_equal(q.scales.to_numpy().view(np.uint32), sc.view(np.uint32))
        assert np.array_equal(q.biases.to_numpy().view(np.uint32), bi.view(np.uint32))


@pytest.mark.parametrize("kind,bits", [(gb.Q4_K, 4), (gb.Q6_K, 8), (gb.Q8_0, 8), (gb.BF16, 4)])
def test_requantize_equals_dequantize_then_quantize_at_flux_size(sdq, stream, kind, bits):
    """Flux's 3072 x 3072 attention projection: the fused kernel against the
    device's own two-step path, every word."""
    rng = np.random.default_rng(kind * 31 + bits)
    rows, cols = 3072, 3072
    print(f"gguf flux-size type={kind} bits={bits}", flush=True)
    raw = gb.random_tensor(kind, rows * cols, rng)
    fused = sdq.QuantizedArray.from_gguf_blocks(raw, kind, [rows, cols], 64, bits, stream)
    dense = sdq.gguf_dequantize(raw, kind, [rows, cols], stream)
    two = sdq.QuantizedArray.quantize(dense, 64, bits, stream)
    for a, b in ((fused.weight, two.weight), (fused.scales, two.scales), (fused.biases, two.biases)):
        assert np.array_equal(a.to_numpy().view(np.uint32), b.to_numpy().view(np.uint32))


def test_errors(sdq, stream):
    with pytest.raises(sdq.Error, match="type 3 is not one this project's checkpoints use"):
        sdq.gguf_dequantize(bytes(20), 3, [32], stream)
    with pytest.raises(sdq.Error, match="30 elements, not a multiple of 32"):
        sdq.gguf_dequantize(bytes(18), gb.Q4_0, [3, 10], stream)
    with pytest.raises(sdq.Error, match="raw bytes given"):
        sdq.gguf_dequantize(bytes(17), gb.Q4_0, [32], stream)
    with pytest.raises(sdq.Error, match="at least 2 dimensions"):
        sdq.QuantizedArray.from_gguf_blocks(bytes(144), gb.Q4_K, [256], 64, 4, stream)
    with pytest.raises(sdq.Error, match="divisible by the quantization group size"):
        sdq.QuantizedArray.from_gguf_blocks(bytes(4 * 96), gb.F32, [2, 48], 64, 4, stream)
    with pytest.raises(sdq.Error, match="supported bits"):
        sdq.QuantizedArray.from_gguf_blocks(bytes(144), gb.Q4_K, [1, 256], 64, 3, stream)
    raw = sdq.Array.from_numpy(np.zeros(8, np.float32))
    with pytest.raises(sdq.Error, match="uint8"):
        sdq.gguf_dequantize(raw, gb.F32, [8], stream)


def test_from_gguf_splits_and_values(sdq, oracle, stream, tmp_path):
    """quantized.rs:181-216 end to end on a small Flux-named file: the policy
    (mixed(4)) picks 8 bits for img_in, 4 for the MLP weight, dense for the 1-D
    and the K % 64 != 0 tensors, and every value matches the oracle."""
    from sdq.quantized import from_gguf, from_gguf_renamed

    rng = np.random.default_rng(5)
    ts = [
        ("double_blocks.0.img_mlp.0.weight", [128, 512], gb.Q4_K),
        ("img_in.weight", [64, 256], gb.Q8_0),
        ("double_blocks.0.img_attn.norm.query_norm.scale", [128], gb.F32),
        ("double_blocks.0.img_mlp.0.bias", [128], gb.F16),
        ("txt_in.weight", [32, 96], gb.BF16),        # 96 % 64 != 0: stays dense
        ("time_in.in_layer.weight", [64, 256], gb.Q6_K),
    ]
    files = [(n, s, k, gb.random_tensor(k, int(np.prod(s)), rng)) for n, s, k in ts]
    path = tmp_path / "flux-small.gguf"
    gb.write_gguf(path, files, [("general.architecture", 8, "flux")])
    w = from_gguf(path, 4, stream)
    assert sorted(w.quantized) == ["double_blocks.0.img_mlp.0.weight", "img_in.weight",
                                   "time_in.in_layer.weight"]
    assert w.quantized["img_in.weight"].bits == 8
    assert w.quantized["double_blocks.0.img_mlp.0.weight"].bits == 4
    assert w.quantized["time_in.in_layer.weight"].bits == 4
    for name, shape, kind, raw in files:
        vals = oracle.gguf_dequantize(np.frombuffer(raw, np.uint8), kind, int(np.prod(shape)))
        if name in w.quantized:
            q = w.quantized[name]
            wq, sc, bi = oracle.quantize(vals.reshape(shape), 64, q.bits)
            assert np.array_equal(q.weight.to_numpy(), wq)
            assert np.array_equal(q.scales.to_numpy(), sc) and np.array_equal(q.biases.to_numpy(), bi)
        else:
            got = w.dense[name].to_numpy()
            assert list(got.shape) == shape
            _same_bits(got, vals)

    r = from_gguf_renamed(path, 4, lambda n: n.replace("img_in", "x_embedder") if "mlp" not in n else None,
                          stream)
    assert "x_embedder.weight" in r.quantized and not any("mlp" in k for k in list(r.quantized) + list(r.dense))
    with pytest.raises(sdq.Error, match="carries no tensors this model recognises"):
        from_gguf_renamed(path, 4, lambda n: None, stream)
