"""The Flux block ops on the GPU (norm.hip, attention.hip, through the C ABI)
against the oracle (oracle/sdq_oracle_block.c, pinned in
test_oracle_block.py) on the same seeded inputs.

Tolerances:
  layer/RMS norm, norm_modulate: f32 outputs within 2e-5 absolute of the f64
    oracle (outputs are O(1)); 16-bit outputs within one rounding of it.
  rope: bit-exact (the same separately rounded f32 operations).
  attention: the products run on bf16 MFMAs, so against the f64 oracle on the
    same inputs the north star's matmul bar applies -- max |err| / max |ref|
    <= 2e-2 and cosine >= 0.9999 -- and, when the inputs are already bf16,
    the tighter 1e-2 / 0.99999.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import cosine, max_rel_err

pytestmark = pytest.mark.gpu


def _bf16(a: np.ndarray) -> np.ndarray:
    """Round to bf16 and widen back (the values a bf16 tensor holds)."""
    import sdq

    return sdq.bf16_bits_to_f32(sdq.f32_to_bf16_bits(a)).reshape(a.shape)


def _dev(sdq, a: np.ndarray, dtype) -> "sdq.Array":
    if dtype == sdq.FLOAT16:
        return sdq.Array.from_numpy(a.astype(np.float16), sdq.FLOAT16)
    return sdq.Array.from_numpy(a.astype(np.float32), dtype)


def _host(sdq, arr) -> np.ndarray:
    out = arr.to_numpy()
    if arr.dtype == sdq.BFLOAT16:
        return sdq.bf16_bits_to_f32(out).reshape(out.shape)
    return out.astype(np.float32)


def _held(sdq, a: np.ndarray, dtype) -> np.ndarray:
    """The values a device array of `dtype` built from `a` holds."""
    if dtype == sdq.BFLOAT16:
        return _bf16(a)
    if dtype == sdq.FLOAT16:
        return a.astype(np.float16).astype(np.float32)
    return a.astype(np.float32)


def _round_to(sdq, a: np.ndarray, dtype) -> np.ndarray:
    return _held(sdq, a, dtype)


# ---- norms -----------------------------------------------------------------------


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,C", [(37, 3072), (5, 1000), (3, 64), (9, 4096), (2, 8192)])
@pytest.mark.parametrize("affine", [False, True])
def test_layer_norm(sdq, oracle, stream, dt, rows, C, affine):
    dtype = {"f32": sdq.FLOAT32, "bf16": sdq.BFLOAT16, "f16": sdq.FLOAT16}[dt]
    rng = np.random.default_rng(rows * C + affine)
    x = _held(sdq, (rng.standard_normal((rows, C)) * 2 + 0.5).astype(np.float32), dtype)
    w = _held(sdq, rng.standard_normal(C).astype(np.float32), dtype) if affine else None
    b = _held(sdq, rng.standard_normal(C).astype(np.float32), dtype) if affine else None
    print(f"layer_norm {dt} [{rows},{C}] affine={affine}", flush=True)
    got = _host(sdq, _dev(sdq, x, dtype).layer_norm(
        None if w is None else _dev(sdq, w, dtype), None if b is None else _dev(sdq, b, dtype), 1e-5, stream))
    want = oracle.layer_norm(x, 1e-5, w, b)
    tol = 2e-5 + (0 if dt == "f32" else np.abs(want) * (2 ** -8 if dt == "bf16" else 2 ** -11))
    assert np.all(np.abs(got - want) <= tol)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("rows,C", [(64, 128), (7, 4096), (4, 100)])
def test_rms_norm(sdq, oracle, stream, dt, rows, C):
    dtype = sdq.FLOAT32 if dt == "f32" else sdq.BFLOAT16
    rng = np.random.default_rng(rows + C)
    x = _held(sdq, (rng.standard_normal((rows, C)) * 3).astype(np.float32), dtype)
    w = _held(sdq, rng.standard_normal(C).astype(np.float32), dtype)
    print(f"rms_norm {dt} [{rows},{C}]", flush=True)
    got = _host(sdq, _dev(sdq, x, dtype).rms_norm(_dev(sdq, w, dtype), 1e-6, stream))
    want = oracle.rms_norm(x, 1e-6, w)
    tol = 2e-5 + (0 if dt == "f32" else np.abs(want) * 2 ** -8)
    assert np.all(np.abs(got - want) <= tol)
    nw = _host(sdq, _dev(sdq, x, dtype).rms_norm(None, 1e-6, stream))
    assert np.all(np.abs(nw - oracle.rms_norm(x, 1e-6)) <= 2e-5 + (0 if dt == "f32" else 2 ** -8 * 4))


@pytest.mark.parametrize("xdt,pdt,B,N", [("bf16", "bf16", 2, 333), ("bf16", "f32", 1, 4608), ("f32", "f32", 3, 17)])
def test_norm_modulate(sdq, oracle, stream, xdt, pdt, B, N):
    from sdq import flux

    C = 3072
    xd = sdq.BFLOAT16 if xdt == "bf16" else sdq.FLOAT32
    pd = sdq.BFLOAT16 if pdt == "bf16" else sdq.FLOAT32
    rng = np.random.default_rng(B * N)
    x = _held(sdq, rng.standard_normal((B, N, C)).astype(np.float32), xd)
    shift = _held(sdq, (rng.standard_normal((B, 1, C)) * 0.5).astype(np.float32), pd)
    scale = _held(sdq, (rng.standard_normal((B, 1, C)) * 0.5).astype(np.float32), pd)
    print(f"norm_modulate x={xdt} p={pdt} [{B},{N},{C}]", flush=True)
    got = _host(sdq, flux.norm_modulate(_dev(sdq, x, xd), _dev(sdq, shift, pd), _dev(sdq, scale, pd), stream))
    want = oracle.norm_modulate(x, shift, scale, 1e-6)
    tol = 3e-5 + (0 if xdt == "f32" else np.abs(want) * 2 ** -8)
    assert np.all(np.abs(got - want) <= tol)


# ---- rotary embedding ---------------------------------------------------------------


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_rope_bit_exact(sdq, oracle, stream, dt):
    from sdq import flux

    dtype = sdq.FLOAT32 if dt == "f32" else sdq.BFLOAT16
    B, H, N, D = 1, 3, 300, 128
    ids = np.stack([np.zeros(N), np.arange(N) // 20, np.arange(N) % 20], axis=1).astype(np.float32)
    pe = flux.embed_nd(ids, N, [16, 56, 56], 10000.0)
    cs, sn = oracle.embed_nd(ids, [16, 56, 56], 10000.0)
    assert np.array_equal(pe.cos.to_numpy().reshape(N, 64), cs) and np.array_equal(pe.sin.to_numpy().reshape(N, 64), sn)
    rng = np.random.default_rng(9)
    x = _held(sdq, rng.standard_normal((B, H, N, D)).astype(np.float32), dtype)
    got = _host(sdq, flux.rotate(_dev(sdq, x, dtype), pe, stream))
    want = _round_to(sdq, oracle.rope(x, cs, sn), dtype)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---- attention -------------------------------------------------------------------------


def _check_attention(got, want, inputs_bf16: bool):
    tol_err, tol_cos = (1e-2, 0.99999) if inputs_bf16 else (2e-2, 0.9999)
    err = max_rel_err(got, want)
    cos = cosine(got, want)
    assert err <= tol_err and cos >= tol_cos, f"max rel err {err:.3e}, cosine {cos:.7f}"


CASES = [
    # B, Hq, Hk, Nq, Nk, D, mode, dtype
    (1, 2, 2, 300, 300, 128, "", "bf16"),
    (1, 3, 3, 77, 77, 64, "causal", "f32"),      # CLIP's text tower
    (2, 4, 4, 129, 200, 128, "array", "bf16"),   # T5-style additive bias
    (1, 4, 2, 64, 64, 64, "", "f16"),            # grouped K/V heads
    (2, 2, 1, 50, 190, 128, "causal", "bf16"),   # causal with Nk > Nq
    (1, 1, 1, 1, 33, 128, "", "f32"),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c)))
def test_sdpa_matches_oracle(sdq, oracle, stream, case):
    B, Hq, Hk, Nq, Nk, D, mode, dt = case
    dtype = {"f32": sdq.FLOAT32, "bf16": sdq.BFLOAT16, "f16": sdq.FLOAT16}[dt]
    rng = np.random.default_rng(sum(case[:6]))
    q = _held(sdq, rng.standard_normal((B, Hq, Nq, D)).astype(np.float32), dtype)
    k = _held(sdq, rng.standard_normal((B, Hk, Nk, D)).astype(np.float32), dtype)
    v = _held(sdq, rng.standard_normal((B, Hk, Nk, D)).astype(np.float32), dtype)
    scale = 1.0 / math.sqrt(D)
    print(f"sdpa {case}", flush=True)
    qa, ka, va = _dev(sdq, q, dtype), _dev(sdq, k, dtype), _dev(sdq, v, dtype)
    if mode == "array":
        mask = (rng.standard_normal((1, Hq, Nq, Nk)) * 2).astype(np.float32)
        got = qa.sdpa_masked(ka, va, scale, sdq.Array.from_numpy(mask), stream)
    elif mode == "causal":
        mask = None
        got = qa.sdpa_causal(ka, va, scale, stream)
    else:
        mask = None
        got = qa.sdpa(ka, va, scale, stream)
    assert got.shape == [B, Hq, Nq, D] and got.dtype == dtype
    want = oracle.sdpa(q, k, v, scale, mode, mask)
    _check_attention(_host(sdq, got), want, dt == "bf16")


def test_sdpa_flux_size_sampled(sdq, oracle, stream):
    """Flux at 1024x1024: 24 heads over 4096 + 512 tokens, head_dim 128; 64
    sampled queries of three heads against the oracle."""
    B, H, N, D = 1, 24, 4608, 128
    rng = np.random.default_rng(46)
    q = _bf16(rng.standard_normal((B, H, N, D)).astype(np.float32))
    k = _bf16(rng.standard_normal((B, H, N, D)).astype(np.float32))
    v = _bf16(rng.standard_normal((B, H, N, D)).astype(np.float32))
    print("sdpa flux size", flush=True)
    got = _host(sdq, _dev(sdq, q, sdq.BFLOAT16).sdpa(_dev(sdq, k, sdq.BFLOAT16), _dev(sdq, v, sdq.BFLOAT16),
                                                    1 / math.sqrt(D), stream))
    idx = np.sort(rng.choice(N, 64, replace=False))
    for h in (0, 11, 23):
        want = oracle.sdpa(q[:, h:h + 1, idx], k[:, h:h + 1], v[:, h:h + 1], 1 / math.sqrt(D))
        _check_attention(got[:, h:h + 1, idx], want, True)


def _flux_ref(oracle, qkv_parts, norms, cs, sn, heads, scale):
    """The reference's composition on the host: split_qkv, qk_norm, concat
    along tokens, rotate, sdpa, merge_heads (flux.rs:300-381)."""
    qs, ks, vs = [], [], []
    for qkv, (qn, kn) in zip(qkv_parts, norms):
        B, n, _ = qkv.shape
        t = qkv[..., :3 * heads * 128].reshape(B, n, 3, heads, 128).transpose(2, 0, 3, 1, 4)
        qs.append(oracle.rms_norm(t[0], 1e-6, qn))
        ks.append(oracle.rms_norm(t[1], 1e-6, kn))
        vs.append(t[2])
    q = oracle.rope(np.concatenate(qs, axis=2), cs, sn)
    k = oracle.rope(np.concatenate(ks, axis=2), cs, sn)
    v = np.concatenate(vs, axis=2)
    o = oracle.sdpa(q, k, v, scale)
    B, H, N, D = o.shape
    return o.transpose(0, 2, 1, 3).reshape(B, N, H * D)


@pytest.mark.parametrize("kind", ["double", "single"])
def test_flux_attention_matches_composition(sdq, oracle, stream, kind):
    from sdq import flux

    rng = np.random.default_rng(7 if kind == "double" else 8)
    heads, hd = 4, 128
    ntxt, nimg = 40, 200
    N = ntxt + nimg
    ids = np.concatenate([np.zeros((ntxt, 3)), np.stack([np.zeros(nimg), np.arange(nimg) // 16,
                                                         np.arange(nimg) % 16], 1)]).astype(np.float32)
    pe = flux.embed_nd(ids, N, [16, 56, 56], 10000.0)
    cs, sn = oracle.embed_nd(ids, [16, 56, 56], 10000.0)
    norm = lambda: _bf16((1 + 0.2 * rng.standard_normal(hd)).astype(np.float32))  # noqa: E731
    scale = 1 / math.sqrt(hd)
    print(f"flux attention {kind}", flush=True)
    if kind == "double":
        txt = _bf16(rng.standard_normal((1, ntxt, 3 * heads * hd)).astype(np.float32))
        img = _bf16(rng.standard_normal((1, nimg, 3 * heads * hd)).astype(np.float32))
        nt, ni = (norm(), norm()), (norm(), norm())
        got = flux.attention(_dev(sdq, txt, sdq.BFLOAT16), _dev(sdq, nt[0], sdq.BFLOAT16),
                             _dev(sdq, nt[1], sdq.BFLOAT16), pe, heads, stream,
                             qkv2=_dev(sdq, img, sdq.BFLOAT16), query_norm2=_dev(sdq, ni[0], sdq.BFLOAT16),
                             key_norm2=_dev(sdq, ni[1], sdq.BFLOAT16))
        want = _flux_ref(oracle, [txt, img], [nt, ni], cs, sn, heads, scale)
    else:
        width = 3 * heads * hd + 4 * heads * hd  # linear1: qkv then the MLP columns
        x = _bf16(rng.standard_normal((1, N, width)).astype(np.float32))
        nq, nk = norm(), norm()
        got = flux.attention(_dev(sdq, x, sdq.BFLOAT16), _dev(sdq, nq, sdq.BFLOAT16), _dev(sdq, nk, sdq.BFLOAT16),
                             pe, heads, stream)
        want = _flux_ref(oracle, [x], [(nq, nk)], cs, sn, heads, scale)
    assert got.shape == [1, N, heads * hd] and got.dtype == sdq.BFLOAT16
    _check_attention(_host(sdq, got), want, False)


def test_flux_single_block_attention_full_size_sampled(sdq, oracle, stream):
    """A single block at 1024x1024: linear1's [1, 4608, 21504] output, 24
    heads; the kernel's output for 48 sampled tokens of every head against the
    composition computed for those tokens."""
    from sdq import flux

    heads, hd, N = 24, 128, 4608
    rng = np.random.default_rng(11)
    x = _bf16(rng.standard_normal((1, N, 21504)).astype(np.float32))
    nq = _bf16((1 + 0.2 * rng.standard_normal(hd)).astype(np.float32))
    nk = _bf16((1 + 0.2 * rng.standard_normal(hd)).astype(np.float32))
    ids = np.concatenate([np.zeros((512, 3)), np.stack([np.zeros(4096), np.arange(4096) // 64,
                                                        np.arange(4096) % 64], 1)]).astype(np.float32)
    pe = flux.embed_nd(ids, N, [16, 56, 56], 10000.0)
    cs, sn = oracle.embed_nd(ids, [16, 56, 56], 10000.0)
    print("flux attention single full size", flush=True)
    got = _host(sdq, flux.attention(_dev(sdq, x, sdq.BFLOAT16), _dev(sdq, nq, sdq.BFLOAT16),
                                    _dev(sdq, nk, sdq.BFLOAT16), pe, heads, stream))
    t = x[..., :3 * heads * hd].reshape(1, N, 3, heads, hd).transpose(2, 0, 3, 1, 4)
    q = oracle.rope(oracle.rms_norm(t[0], 1e-6, nq), cs, sn)
    k = oracle.rope(oracle.rms_norm(t[1], 1e-6, nk), cs, sn)
    idx = np.sort(rng.choice(N, 48, replace=False))
    o = oracle.sdpa(np.ascontiguousarray(q[:, :, idx]), k, np.ascontiguousarray(t[2]), 1 / math.sqrt(hd))
    want = o.transpose(0, 2, 1, 3).reshape(1, len(idx), heads * hd)
    _check_attention(got[:, idx], want, False)


def test_errors(sdq, stream):
    from sdq import flux

    a = sdq.Array.from_numpy(np.zeros((1, 2, 8, 96), np.float32))
    with pytest.raises(sdq.Error, match="head_dim 96 is not supported"):
        a.sdpa(a, a, 0.1, stream)
    q = sdq.Array.from_numpy(np.zeros((1, 2, 8, 64), np.float32))
    with pytest.raises(sdq.Error, match="mask_mode must be"):
        q._sdpa(q, q, 0.1, b"none", None, stream, "sdpa")
    with pytest.raises(sdq.Error, match="mask's last axis"):
        q.sdpa_masked(q, q, 0.1, sdq.Array.from_numpy(np.zeros((8, 7), np.float32)), stream)
    k3 = sdq.Array.from_numpy(np.zeros((1, 3, 8, 64), np.float32))
    with pytest.raises(sdq.Error, match="multiple of the key/value heads"):
        q.sdpa(k3, k3, 0.1, stream)
    x = sdq.Array.from_numpy(np.zeros((1, 4, 3072), np.float32))
    with pytest.raises(sdq.Error, match=r"shift and scale must hold"):
        flux.norm_modulate(x, sdq.Array.from_numpy(np.zeros((1, 1, 100), np.float32)),
                           sdq.Array.from_numpy(np.zeros((1, 1, 100), np.float32)), stream)
    with pytest.raises(sdq.Error, match="rows longer than 8192"):
        sdq.Array.from_numpy(np.zeros((1, 9000), np.float32)).layer_norm(None, None, 1e-5, stream)
