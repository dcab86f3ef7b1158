"""The Flux block ops around the quantized linears (sd-models/src/mlx/flux.rs),
over libsdq.

    embed_nd / Rope        flux.rs:116-156   rotary tables, built on the host in f64
    rotate                 flux.rs:165-205   interleaved RoPE       (sdq_flux_rope)
    norm_modulate          flux.rs:255-275   LayerNorm * (1 + scale) + shift
                                             (sdq_flux_norm_modulate)
    attention              flux.rs:300-327, 352-381, 446-461: split_qkv ->
                           qk_norm -> concat -> rotate -> sdpa -> merge_heads as
                           one call (sdq_flux_attention)

Every call goes through the C ABI; errors raise sdq.Error.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import Array, CArray, QuantizedArray, Stream, _check, _h, _some_int, lib

EPS = 1e-6  # flux.rs:28


@dataclass
class Rope:
    """cos and sin, each [1, seq, head_dim/2] float32 (flux.rs:120-123)."""

    cos: Array
    sin: Array


def embed_nd(ids: Sequence[float], seq: int, axes_dim: Sequence[int], theta: float) -> Rope:
    """(cos, sin) for [seq, n_axes] positions (flux.rs:126-156): frequencies
    and angles in f64 on the host, stored as f32."""
    from . import Error

    n_axes = len(axes_dim)
    ids = np.asarray(ids, dtype=np.float32).reshape(-1)
    if ids.size != seq * n_axes:
        raise Error(f"mlx: {ids.size} ids for {seq} tokens across {n_axes} axes")
    cols_cos, cols_sin = [], []
    pos_all = ids.reshape(seq, n_axes).astype(np.float64)
    for axis, dim in enumerate(axes_dim):
        half = dim // 2
        i = np.arange(half, dtype=np.float64)
        omega = 1.0 / np.power(float(np.float32(theta)), 2.0 * i / dim)
        angle = pos_all[:, axis:axis + 1] * omega[None, :]
        cols_cos.append(np.cos(angle))
        cols_sin.append(np.sin(angle))
    cos = np.concatenate(cols_cos, axis=1).astype(np.float32)
    sin = np.concatenate(cols_sin, axis=1).astype(np.float32)
    half_total = cos.shape[1]
    return Rope(Array.from_numpy(cos.reshape(1, seq, half_total)), Array.from_numpy(sin.reshape(1, seq, half_total)))


def rotate(x: Array, pe: Rope, s: Stream) -> Array:
    """Interleaved rotary application on [b, h, n, d] (flux.rs:165-205)."""
    out = CArray(None)
    _check(lib().sdq_flux_rope(ctypes.byref(out), x._raw, pe.cos._raw, pe.sin._raw, s._raw), "rope")
    return Array(out)


def norm_modulate(x: Array, shift: Array, scale: Array, s: Stream) -> Array:
    """layer_norm(x) * (1 + scale) + shift with no learned affine
    (flux.rs:255-275); x [b, n, c], shift and scale [b, 1, c]."""
    out = CArray(None)
    _check(lib().sdq_flux_norm_modulate(ctypes.byref(out), x._raw, shift._raw, scale._raw, EPS, s._raw),
           "norm_modulate")
    return Array(out)


def attention(qkv: Array, query_norm: Array, key_norm: Array, pe: Rope, heads: int, s: Stream,
              qkv2: Optional[Array] = None, query_norm2: Optional[Array] = None,
              key_norm2: Optional[Array] = None, scale: Optional[float] = None) -> Array:
    """A block's attention from its qkv projection(s) to [b, n, heads*128]:
    the single block passes linear1's output (flux.rs:446-461); the double
    block passes the text stream first and the image stream as qkv2, each
    with its own q/k norm scales (flux.rs:352-381)."""
    hd = 128
    if scale is None:
        scale = 1.0 / math.sqrt(hd)
    out = CArray(None)
    _check(lib().sdq_flux_attention(ctypes.byref(out), qkv._raw, query_norm._raw, key_norm._raw, _h(qkv2),
                                    _h(query_norm2), _h(key_norm2), pe.cos._raw, pe.sin._raw, int(heads),
                                    float(scale), EPS, s._raw),
           "flux_attention")
    return Array(out)


def single_linear1_attention(x: Array, linear1: QuantizedArray, bias: Optional[Array], query_norm: Array,
                             key_norm: Array, pe: Rope, heads: int, s: Stream,
                             scale: Optional[float] = None) -> Array:
    """The single block from its modulated input to linear2's input
    (flux.rs:440-465): linear1, its q/k/v columns through the attention and
    its MLP columns through GELU, concatenated as [attention, gelu(mlp)].  One
    matmul launch writes the q/k/v columns to a buffer of their own and the
    GELU'd MLP columns straight into the result; the attention then fills the
    result's first heads * 128 columns."""
    if scale is None:
        scale = 1.0 / math.sqrt(128)
    out = CArray(None)
    _check(lib().sdq_flux_single_linear1_attention(
        ctypes.byref(out), x._raw, linear1.weight._raw, linear1.scales._raw, linear1.biases._raw, _h(bias),
        _some_int(linear1.group_size), _some_int(linear1.bits), linear1.QUANT_MODE, query_norm._raw,
        key_norm._raw, pe.cos._raw, pe.sin._raw, int(heads), float(scale), EPS, s._raw),
        "flux_single_linear1_attention")
    return Array(out)
