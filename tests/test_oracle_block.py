"""Pins the oracle's Flux block ops (oracle/sdq_oracle_block.c) with closed
forms, invariants and numpy's own routines, before the GPU kernels are
compared with it."""
from __future__ import annotations

import numpy as np
import pytest


def test_layer_norm_hand_worked_and_invariants(oracle):
    x = np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)
    got = oracle.layer_norm(x, 0.0)
    # mean 2.5, biased variance 1.25
    want = (np.array([-1.5, -0.5, 0.5, 1.5]) / np.sqrt(1.25)).astype(np.float32)
    assert np.allclose(got, want, rtol=0, atol=1e-7)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((16, 3072)).astype(np.float32) * 3 + 1
    y = oracle.layer_norm(x, 1e-6)
    assert np.allclose(y.mean(axis=1), 0, atol=1e-6)
    assert np.allclose(y.var(axis=1), 1, atol=1e-5)
    w = rng.standard_normal(3072).astype(np.float32)
    b = rng.standard_normal(3072).astype(np.float32)
    assert np.allclose(oracle.layer_norm(x, 1e-6, w, b), y * w + b, atol=1e-5)
    # eps enters under the square root: a constant row is 0, not NaN
    assert np.all(oracle.layer_norm(np.full((1, 8), 5.0, np.float32), 1e-6) == 0)


def test_rms_norm_hand_worked(oracle):
    got = oracle.rms_norm(np.array([[3.0, 4.0]], np.float32), 0.0)
    r = np.sqrt(12.5)
    assert np.allclose(got, [[3 / r, 4 / r]], atol=1e-7)
    w = np.array([2.0, -1.0], np.float32)
    assert np.allclose(oracle.rms_norm(np.array([[3.0, 4.0]], np.float32), 0.0, w), [[6 / r, -4 / r]], atol=1e-7)
    rng = np.random.default_rng(1)
    y = oracle.rms_norm(rng.standard_normal((8, 128)).astype(np.float32) * 7, 1e-6)
    assert np.allclose(np.sqrt((y.astype(np.float64) ** 2).mean(axis=1)), 1, atol=1e-5)


def test_norm_modulate_reduces_to_layer_norm(oracle):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((2, 5, 64)).astype(np.float32)
    z = np.zeros((2, 1, 64), np.float32)
    ln = oracle.layer_norm(x, 1e-6)
    assert np.array_equal(oracle.norm_modulate(x, z, z, 1e-6), ln)
    one = np.ones((2, 1, 64), np.float32)
    assert np.allclose(oracle.norm_modulate(x, z, one, 1e-6), 2 * ln, atol=1e-6)
    sh = rng.standard_normal((2, 1, 64)).astype(np.float32)
    assert np.allclose(oracle.norm_modulate(x, sh, z, 1e-6), ln + sh, atol=1e-6)


def test_rope_rotations(oracle):
    x = np.array([[1.0, 2.0, -3.0, 0.5]], np.float32)
    ident = oracle.rope(x, np.ones((1, 2), np.float32), np.zeros((1, 2), np.float32))
    assert np.array_equal(ident, x)
    quarter = oracle.rope(x, np.zeros((1, 2), np.float32), np.ones((1, 2), np.float32))
    # interleaved: (e, o) -> (-o, e) per pair
    assert np.array_equal(quarter, [[-2.0, 1.0, -0.5, -3.0]])
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 7, 16)).astype(np.float32)
    ang = rng.uniform(-4, 4, (7, 8))
    y = oracle.rope(x, np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32))
    pair_norm = lambda a: np.hypot(a[..., 0::2], a[..., 1::2])  # noqa: E731
    assert np.allclose(pair_norm(y), pair_norm(x), rtol=1e-5)
    # the rotation is by +angle: pair 0 of position n goes to angle + atan2
    assert np.allclose(np.arctan2(y[..., 1::2], y[..., 0::2]),
                       np.angle(np.exp(1j * (np.arctan2(x[..., 1::2], x[..., 0::2]) + ang))), atol=1e-4)


def test_embed_nd_tables(oracle):
    ids = np.array([[0, 0, 0], [0, 3, 5], [1, 2, 7]], np.float32)
    cs, sn = oracle.embed_nd(ids, [16, 56, 56], 10000.0)
    assert cs.shape == (3, 64)
    assert np.allclose(cs ** 2 + sn ** 2, 1, atol=1e-6)
    assert np.all(cs[0] == 1) and np.all(sn[0] == 0)
    # frequency 0 of each axis is 1 rad per unit position
    assert np.isclose(sn[1, 8], np.sin(3.0)) and np.isclose(sn[1, 36], np.sin(5.0))
    assert np.isclose(cs[2, 1], np.cos(1.0 / 10000.0 ** (2 / 16)))


def _np_sdpa(q, k, v, scale, mask=None, causal=False):
    s = np.einsum("bhqd,bhkd->bhqk", q.astype(np.float64), k.astype(np.float64)) * scale
    if mask is not None:
        s = s + mask
    if causal:
        nq, nk = s.shape[-2:]
        s = np.where(np.arange(nk)[None, :] > np.arange(nq)[:, None] + (nk - nq), -np.inf, s)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("bhqk,bhkd->bhqd", p, v.astype(np.float64))


def test_sdpa_closed_forms(oracle):
    rng = np.random.default_rng(4)
    k = rng.standard_normal((1, 2, 9, 8)).astype(np.float32)
    v = rng.standard_normal((1, 2, 9, 8)).astype(np.float32)
    # q = 0: every key equally weighted
    out = oracle.sdpa(np.zeros((1, 2, 3, 8), np.float32), k, v, 0.5)
    assert np.allclose(out, v.mean(axis=2, keepdims=True), atol=1e-6)
    # causal: the first query sees key 0 only
    q = rng.standard_normal((1, 2, 9, 8)).astype(np.float32)
    out = oracle.sdpa(q, k, v, 0.3, "causal")
    assert np.allclose(out[:, :, 0], v[:, :, 0], atol=1e-7)
    # a one-hot key wins: orthogonal keys, q a large multiple of key 5
    eye = np.eye(8, dtype=np.float32)[None, None].repeat(2, axis=1)
    out = oracle.sdpa(eye[:, :, 5:6] * 40, eye, v[:, :, :8], 1.0)
    assert np.allclose(out[:, :, 0], v[:, :, 5], atol=1e-6)
    # permuting keys and values together changes nothing
    perm = rng.permutation(9)
    a = oracle.sdpa(q, k, v, 0.3)
    b = oracle.sdpa(q, k[:, :, perm], v[:, :, perm], 0.3)
    assert np.allclose(a, b, atol=1e-6)
    # a mask of -inf everywhere but key 2 selects v[2]; a constant mask is a no-op
    m = np.full((9,), -np.inf, np.float32)
    m[2] = 0
    assert np.allclose(oracle.sdpa(q, k, v, 0.3, "array", m), v[:, :, 2:3], atol=1e-7)
    assert np.allclose(oracle.sdpa(q, k, v, 0.3, "array", np.full((9,), 7.0, np.float32)), a, atol=1e-6)


@pytest.mark.parametrize("mode", ["", "causal", "array"])
def test_sdpa_against_numpy(oracle, mode):
    rng = np.random.default_rng(5)
    q = rng.standard_normal((2, 4, 5, 16)).astype(np.float32)
    k = rng.standard_normal((2, 2, 7, 16)).astype(np.float32)   # grouped: 2 query heads per k/v head
    v = rng.standard_normal((2, 2, 7, 16)).astype(np.float32)
    mask = rng.standard_normal((1, 4, 5, 7)).astype(np.float32) if mode == "array" else None
    got = oracle.sdpa(q, k, v, 0.25, mode, mask)
    kk, vv = np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1)
    want = _np_sdpa(q, kk, vv, 0.25, mask, causal=mode == "causal")
    assert np.allclose(got, want, atol=1e-6)
