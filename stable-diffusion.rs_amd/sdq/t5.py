"""T5-XXL's gated feed-forward on the HIP backend: the caller of the quantized
linear that BASELINE config 3 measures.

`feed_forward` mirrors `feed_forward` in crates/sd-models/src/mlx/t5.rs:201-214:
`wo(gelu_new(wi_0(x)) * wi_1(x))` through a `WeightSource`.  When both input
projections are quantized with the same group size and bits, their packed
weights are paired once (rows interleaved in blocks of eight,
`QuantizedArray.pair`) and kept on the weight source, and the two linears,
the GELU and the product run as one launch (`QuantizedArray.linear_gated`).
Otherwise it issues the reference's sequence of calls.
"""
from __future__ import annotations

from typing import Dict, Tuple

from . import ACT_GELU_APPROX, Array, QuantizedArray, Stream


def _paired(w, gate: str, up: str, s: Stream):
    """The paired wi_0/wi_1 operand of `w`, built on first use and cached on
    the weight source (load-time work: one strided copy per array)."""
    quantized = getattr(w, "quantized", None)
    if not quantized or gate not in quantized or up not in quantized:
        return None
    g, u = quantized[gate], quantized[up]
    if (g.group_size, g.bits) != (u.group_size, u.bits) or g.weight.shape != u.weight.shape:
        return None
    if g.weight.shape[0] % 8 != 0:
        return None
    cache: Dict[Tuple[str, str], QuantizedArray] = w.__dict__.setdefault("_t5_pairs", {})
    key = (gate, up)
    if key not in cache:
        cache[key] = QuantizedArray.pair(g, u, s)
    return cache[key]


def feed_forward(x: Array, w, prefix: str, s: Stream) -> Array:
    """`wo(gelu_new(wi_0(x)) * wi_1(x))` (t5.rs:209-214): the tanh GELU
    (`gelu_new`, t5.rs:203-207), no biases."""
    gate, up, out = f"{prefix}.wi_0.weight", f"{prefix}.wi_1.weight", f"{prefix}.wo.weight"
    pair = _paired(w, gate, up, s)
    if pair is not None:
        h = pair.linear_gated(x, s, activation=ACT_GELU_APPROX)
    else:
        h = w.linear(x, gate, None, s).gelu_approx(s).mul(w.linear(x, up, None, s), s)
    return w.linear(h, out, None, s)
