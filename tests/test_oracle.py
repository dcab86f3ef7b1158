"""Pins the CPU oracle (oracle/sdq_oracle.c) before anything is compared with
it.  The reference ships no golden vectors for this path (MLX is an external,
absent dependency), so every function is pinned here by published test
vectors, closed forms, special cases worked by hand, invariants, or brute
force -- each chosen so that a plausible slip (a wrong shift, sign, rounding
mode, nibble order, fused vs unfused op) fails at least one test.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import cosine, ramp_activation, ramp_weight

# ---- SeededRng (crates/sd-tensor/src/lib.rs:105-145) ---------------------------

# splitmix64 published test vector: seed 1234567 (Vigna, splitmix64.c).
SPLITMIX_1234567 = [
    6457827717110365317,
    3203168211198807973,
    9817491932198370423,
    4593380528125082431,
    16408922859458223821,
]


def test_splitmix64_matches_the_published_vector(oracle):
    r = oracle.Rng(1234567)
    assert [r.next_u64() for _ in range(5)] == SPLITMIX_1234567


def test_next_f64_is_53_bits_shifted_off_zero(oracle):
    r = oracle.Rng(1234567)
    for u in SPLITMIX_1234567:
        got = r.next_f64()
        assert got == ((u >> 11) + 1) / 2.0**53
        assert 0.0 < got <= 1.0


def test_normals_are_box_muller_cos_then_sin(oracle):
    # The pair structure: z0 = r cos(theta), z1 = r sin(theta) with
    # r = sqrt(-2 ln u1), theta = 2 pi u2 -- so z0^2 + z1^2 = -2 ln u1 and
    # atan2(z1, z0) = theta (mod 2 pi).  Swapping cos and sin, or u1 and u2,
    # breaks one of the two.
    seed = 99
    u = oracle.Rng(seed)
    z = oracle.Rng(seed).normals(2000)
    for i in range(0, 2000, 2):
        u1, u2 = u.next_f64(), u.next_f64()
        r2 = -2.0 * math.log(u1)
        assert abs(float(z[i]) ** 2 + float(z[i + 1]) ** 2 - r2) <= 1e-5 * max(1.0, r2)
        ang = math.atan2(float(z[i + 1]), float(z[i])) % (2 * math.pi)
        d = abs(ang - 2 * math.pi * u2)
        assert min(d, 2 * math.pi - d) < 1e-5 or r2 < 1e-8


def test_normals_odd_count_drops_the_last_sin(oracle):
    a = oracle.Rng(7).normals(5)
    b = oracle.Rng(7).normals(6)
    assert np.array_equal(a, b[:5])


def test_normals_are_standard_normal(oracle):
    from scipy import stats

    z = oracle.normals(2024, 400_000).astype(np.float64)
    assert abs(z.mean()) < 0.01
    assert abs(z.std() - 1.0) < 0.01
    assert stats.kstest(z, "norm").pvalue > 1e-4


# ---- 16-bit storage ------------------------------------------------------------------


def test_f16_conversion_matches_ieee_round_to_nearest_even(oracle):
    # numpy's float32 -> float16 cast is IEEE RNE, including subnormals,
    # overflow to inf and ties.
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 2.0**-25, 2.0**-24, 3 * 2.0**-26,
                  np.inf, -np.inf], dtype=np.float32),
    ]).astype(np.float32)
    for v in vals:
        want = int(np.float32(v).astype(np.float16).view(np.uint16))
        assert oracle.f16_from_f32(float(v)) == want, v
        back = oracle.f32_from_f16(want)
        assert np.float32(back) == np.float16(np.uint16(want).view(np.float16)).astype(np.float32)


def test_bf16_conversion_rounds_to_nearest_even(oracle):
    # Ties: 1 + 2^-8 is exactly half-way between 1 and 1 + 2^-7 -> even (1.0);
    # 1 + 3*2^-8 is half-way between 1 + 2^-7 and 1 + 2^-6 -> even (1 + 2^-6).
    assert oracle.f32_from_bf16(oracle.bf16_from_f32(1.0 + 2.0**-8)) == 1.0
    assert oracle.f32_from_bf16(oracle.bf16_from_f32(1.0 + 3 * 2.0**-8)) == 1.0 + 2.0**-6
    assert oracle.f32_from_bf16(oracle.bf16_from_f32(1.0 + 2.0**-8 + 2.0**-20)) == 1.0 + 2.0**-7
    # Truncation is always within half an ulp of the value.
    rng = np.random.default_rng(1)
    for v in rng.standard_normal(5000).astype(np.float32):
        r = oracle.f32_from_bf16(oracle.bf16_from_f32(float(v)))
        ulp = 2.0 ** (math.floor(math.log2(abs(float(v)))) - 7)
        assert abs(r - float(v)) <= ulp / 2


# ---- quantize: hand-worked known answers ---------------------------------------------


def test_ramp_codes_pack_first_element_in_the_low_bits(oracle):
    # w = 0..15 then 15s: w_min 0, w_max 15, |w_min| <= |w_max| -> scale = -1,
    # edge = 15, q0 = rint(15/-1) = -15 -> scale = 15/-15 = -1, bias = 15,
    # code = 15 - w.  Codes 15, 14, ..., 8 in the first word, LSB first.
    w = np.array([list(range(16)) + [15] * 48], dtype=np.float32)
    wq, s, b = oracle.quantize(w, 64, 4)
    assert wq[0, 0] == 0x89ABCDEF
    assert wq[0, 1] == 0x01234567
    assert np.all(wq[0, 2:] == 0)
    assert s[0, 0] == -1.0 and b[0, 0] == 15.0
    assert np.array_equal(oracle.dequantize(wq, s, b, 64, 4), w)


def test_negative_dominant_group_puts_the_bias_at_the_minimum(oracle):
    w = -np.array([list(range(16)) + [15] * 48], dtype=np.float32)
    wq, s, b = oracle.quantize(w, 64, 4)
    assert s[0, 0] == 1.0 and b[0, 0] == -15.0
    assert wq[0, 0] == 0x89ABCDEF  # code = w + 15
    assert np.array_equal(oracle.dequantize(wq, s, b, 64, 4), w)


def test_codes_round_half_to_even(oracle):
    # scale -1, bias 15 as above; (w - 15) / -1 = 15 - w lands on .5 exactly:
    # 0.5 -> 14.5 -> 14, 2.5 -> 12.5 -> 12, 13.5 -> 1.5 -> 2 (half away from
    # zero would give 15, 13, 2).
    row = [0.0, 15.0, 0.5, 2.5, 13.5] + [15.0] * 59
    wq, s, b = oracle.quantize(np.array([row], dtype=np.float32), 64, 4)
    codes = [(int(wq[0, 0]) >> (4 * e)) & 15 for e in range(5)]
    assert codes == [15, 0, 14, 12, 2]


def test_eight_bit_ramp(oracle):
    # w = 0..63: scale -> -(63/255) refit to 63/-255, bias 63; the code of w is
    # rint((63 - w) * 255 / 63), which never ties (85(63-w)/21 is never x.5).
    w = np.arange(64, dtype=np.float32)[None, :]
    wq, s, b = oracle.quantize(w, 64, 8)
    want = np.rint((63.0 - np.arange(64)) * 255.0 / 63.0).astype(np.uint32)
    got = np.array([(int(wq[0, k // 4]) >> (8 * (k % 4))) & 255 for k in range(64)], dtype=np.uint32)
    assert np.array_equal(got, want)
    assert got[0] == 255 and got[63] == 0
    assert b[0, 0] == 63.0
    assert np.float32(s[0, 0]) == np.float32(63.0) / np.float32(-255.0)


def test_two_bit_codes(oracle):
    w = np.tile(np.array([0.0, 1.0, 2.0, 3.0], dtype=np.float32), 16)[None, :]
    wq, s, b = oracle.quantize(w, 64, 2)
    assert np.all(wq == 0x1B1B1B1B)  # codes 3,2,1,0 repeating, LSB first
    assert np.array_equal(oracle.dequantize(wq, s, b, 64, 2), w)


def test_constant_and_zero_groups(oracle):
    # Constant c: the range clamps to 1e-7, q0 = rint(c / -1e-7) != 0, so the
    # bias is c itself and every code is 0: c comes back exactly.
    w = np.full((1, 64), 0.5, dtype=np.float32)
    wq, s, b = oracle.quantize(w, 64, 4)
    assert np.all(wq == 0) and b[0, 0] == 0.5
    assert np.array_equal(oracle.dequantize(wq, s, b, 64, 4), w)
    # All zero: q0 = 0, so bias = 0 and scale stays -1e-7.
    z = np.zeros((1, 64), dtype=np.float32)
    wq, s, b = oracle.quantize(z, 64, 4)
    assert np.all(wq == 0) and b[0, 0] == 0.0 and s[0, 0] == np.float32(-1e-7)
    assert np.all(oracle.dequantize(wq, s, b, 64, 4) == 0.0)


def test_group_sizes_are_independent_groups(oracle):
    # Quantizing [r, K] with group g is quantizing [r*K/g, g] with group g.
    w = oracle.normals(5, 8 * 512, 0.02).reshape(8, 512)
    for gs in (32, 64, 128):
        for bits in (2, 4, 8):
            a = oracle.quantize(w, gs, bits)
            c = oracle.quantize(w.reshape(-1, gs), gs, bits)
            assert np.array_equal(a[0].ravel(), c[0].ravel())
            assert np.array_equal(a[1].ravel(), c[1].ravel())
            assert np.array_equal(a[2].ravel(), c[2].ravel())


def test_invalid_layouts_are_rejected(oracle):
    with pytest.raises(ValueError):
        oracle.quantize(np.zeros((2, 100), np.float32), 64, 4)
    with pytest.raises(ValueError):
        oracle.quantize(np.zeros((2, 64), np.float32), 64, 3)
    with pytest.raises(ValueError):
        oracle.quantize(np.zeros((2, 64), np.float32), 48, 4)


# ---- quantize: invariants on random weights ------------------------------------------


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_every_value_lands_on_its_nearest_code(oracle, bits, gs):
    w = oracle.normals(11, 64 * 512, 0.02).reshape(64, 512)
    wq, s, b = oracle.quantize(w, gs, bits)
    deq = oracle.dequantize(wq, s, b, gs, bits)
    per = 32 // bits
    codes = ((wq[:, :, None] >> (np.arange(per, dtype=np.uint32) * bits)) & ((1 << bits) - 1)).reshape(64, 512)
    sc = np.repeat(s, gs, axis=1).astype(np.float64)
    bi = np.repeat(b, gs, axis=1).astype(np.float64)
    n_bins = (1 << bits) - 1
    # Brute force over every code: the chosen one is the nearest grid point,
    # up to f32 rounding of (w - bias) / scale, unless w lies beyond the grid.
    grid = sc[..., None] * np.arange(n_bins + 1) + bi[..., None]
    err = np.abs(w[..., None].astype(np.float64) - grid)
    best = err.min(axis=-1)
    chosen = np.take_along_axis(err, codes[..., None].astype(np.int64), axis=-1)[..., 0]
    assert np.all(chosen <= best + 1e-6 * np.abs(sc))
    inside = (codes > 0) & (codes < n_bins)
    assert np.all(np.abs(w - deq)[inside] <= 0.5 * np.abs(sc)[inside] * (1 + 1e-5) + 1e-12)


@pytest.mark.parametrize("bits", [4, 8])
def test_the_dominant_edge_reconstructs_exactly(oracle, bits):
    w = oracle.normals(12, 128 * 256, 0.02).reshape(128, 256)
    wq, s, b = oracle.quantize(w, 64, bits)
    deq = oracle.dequantize(wq, s, b, 64, bits)
    g = w.reshape(128, 4, 64)
    lo, hi = g.min(-1), g.max(-1)
    edge = np.where(np.abs(lo) > np.abs(hi), lo, hi)
    idx = np.argmax(g == edge[..., None], axis=-1)
    got = np.take_along_axis(deq.reshape(128, 4, 64), idx[..., None], axis=-1)[..., 0]
    assert np.array_equal(got, edge)
    assert np.array_equal(b, edge)


@pytest.mark.parametrize("store", [10, 12, 9])
def test_scales_are_stored_in_the_weights_dtype_after_coding(oracle, store):
    # Codes come from the f32 scale and bias; only the stored values are
    # rounded to the weight's dtype.
    w = oracle.normals(13, 16 * 256, 0.02).reshape(16, 256)
    q32, s32, b32 = oracle.quantize(w, 64, 4, 10)
    q, s, b = oracle.quantize(w, 64, 4, store)
    assert np.array_equal(q, q32)
    conv = oracle.bf16_from_f32 if store == 12 else (oracle.f16_from_f32 if store == 9 else None)
    if conv is None:
        assert np.array_equal(s, s32) and np.array_equal(b, b32)
    else:
        assert np.array_equal(s.ravel(), np.array([conv(float(v)) for v in s32.ravel()], np.uint16))
        assert np.array_equal(b.ravel(), np.array([conv(float(v)) for v in b32.ravel()], np.uint16))


# ---- dequantize ------------------------------------------------------------------------


def test_dequantize_is_an_unfused_multiply_then_add(oracle):
    # Every 4-bit code once per row, random f32 scale and bias per row.  The
    # result must be fl(fl(q*s) + b) -- and that differs from the fused
    # fl(q*s + b) somewhere, so the test would catch a contraction.
    rng = np.random.default_rng(3)
    rows = 4096
    codes = np.tile(np.arange(16, dtype=np.uint32), 4)  # 64 codes
    words = np.zeros(8, np.uint32)
    for k, c in enumerate(codes):
        words[k // 8] |= np.uint32(c) << np.uint32(4 * (k % 8))
    wq = np.tile(words, (rows, 1))
    s = (rng.standard_normal((rows, 1)) * 0.01).astype(np.float32)
    b = (rng.standard_normal((rows, 1)) * 0.05).astype(np.float32)
    deq = oracle.dequantize(wq, s, b, 64, 4)
    q = codes.astype(np.float32)[None, :]
    unfused = (q * s).astype(np.float32) + b
    assert np.array_equal(deq, unfused.astype(np.float32))
    fused = (q.astype(np.float64) * s.astype(np.float64) + b.astype(np.float64)).astype(np.float32)
    assert not np.array_equal(deq, fused)


def test_dequantize_rounds_each_op_to_bf16_scales(oracle):
    rng = np.random.default_rng(4)
    w = oracle.normals(14, 8 * 128, 0.02).reshape(8, 128)
    wq, s, b = oracle.quantize(w, 64, 4, 12)
    deq = oracle.dequantize(wq, s, b, 64, 4, 12)
    sf = np.array([oracle.f32_from_bf16(int(v)) for v in s.ravel()], np.float32).reshape(s.shape)
    bf = np.array([oracle.f32_from_bf16(int(v)) for v in b.ravel()], np.float32).reshape(b.shape)
    codes = ((wq[:, :, None] >> (np.arange(8, dtype=np.uint32) * 4)) & 15).reshape(8, 128).astype(np.float32)
    rb = lambda a: np.vectorize(lambda v: oracle.f32_from_bf16(oracle.bf16_from_f32(float(v))))(a).astype(np.float32)
    p = rb((codes * np.repeat(sf, 64, 1)).astype(np.float32))
    want = rb((p + np.repeat(bf, 64, 1)).astype(np.float32))
    assert np.array_equal(deq, want)
    del rng


# ---- quantized matmul ------------------------------------------------------------------


@pytest.mark.parametrize("bits", [4, 8])
def test_qmatmul_is_the_dense_product_of_the_dequantized_weight(oracle, bits):
    x = oracle.normals(21, 9 * 256).reshape(9, 256)
    w = oracle.normals(22, 40 * 256, 0.02).reshape(40, 256)
    wq, s, b = oracle.quantize(w, 64, bits)
    deq = oracle.dequantize(wq, s, b, 64, bits).astype(np.float64)
    want = x.astype(np.float64) @ deq.T
    y64 = oracle.qmatmul_f64(x, wq, s, b, 64, bits)
    assert np.allclose(y64, want, rtol=1e-12, atol=1e-12)
    y32 = oracle.qmatmul(x, wq, s, b, 64, bits)
    assert np.max(np.abs(y32 - want)) <= 1e-5 * np.max(np.abs(want))


def test_qmatmul_brute_force_single_output(oracle):
    x = oracle.normals(23, 64).reshape(1, 64)
    w = oracle.normals(24, 64, 0.02).reshape(1, 64)
    wq, s, b = oracle.quantize(w, 64, 4)
    acc32 = np.float32(0.0)
    acc64 = 0.0
    for k in range(64):
        q = (int(wq[0, k // 8]) >> (4 * (k % 8))) & 15
        wv = np.float32(np.float32(q) * s[0, 0]) + b[0, 0]
        acc32 = np.float32(acc32 + np.float32(x[0, k] * wv))
        acc64 += float(x[0, k]) * float(wv)
    assert oracle.qmatmul(x, wq, s, b)[0, 0] == acc32
    assert oracle.qmatmul_f64(x, wq, s, b)[0, 0] == acc64


@pytest.mark.parametrize("bits", [4, 8])
def test_blocked_parallel_qmatmul_is_bit_identical(oracle, bits):
    x = oracle.normals(31, 37 * 512).reshape(37, 512)
    w = oracle.normals(32, 70 * 512, 0.02).reshape(70, 512)
    wq, s, b = oracle.quantize(w, 64, bits)
    a = oracle.qmatmul(x, wq, s, b, 64, bits)
    c = oracle.qmatmul_omp(x, wq, s, b, 64, bits, threads=4)
    assert np.array_equal(a, c)


# ---- the reference's own thresholds, on its own inputs (mlx_quantized.rs) ---------


def test_round_trip_cost_is_what_the_bit_width_says(oracle):
    # mlx_quantized.rs:53-75
    w = ramp_weight(256, 512)
    prev = 0.0
    for bits in (4, 8):
        wq, s, b = oracle.quantize(w, 64, bits)
        c = cosine(w, oracle.dequantize(wq, s, b, 64, bits))
        assert c > 0.99
        assert c > prev
        prev = c


def test_quantized_matmul_agrees_with_the_dense_one(oracle):
    # mlx_quantized.rs:83-117
    w = ramp_weight(256, 512)
    x = ramp_activation(8, 512)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    for bits in (4, 8):
        wq, s, b = oracle.quantize(w, 64, bits)
        got = oracle.qmatmul(x, wq, s, b, 64, bits)
        assert got.shape == (8, 256)
        assert cosine(want, got) > 0.999


def test_resident_bytes_closed_forms(oracle):
    # mlx_quantized.rs:120-141; at group 64 with 4-byte scales the ratios are
    # (bits/32 + 2/64) / 1: 0.15625 and 0.28125.
    dense = 1024 * 1024 * 4
    assert oracle.resident_bytes(1024, 1024, 64, 4) / dense == 0.15625
    assert oracle.resident_bytes(1024, 1024, 64, 8) / dense == 0.28125


# ---- gelu_approx (mlx.rs:1041-1054) ------------------------------------------------------


def test_gelu_approx_identities_and_library_agreement(oracle):
    x = np.concatenate([np.linspace(-8, 8, 4001, dtype=np.float32), oracle.normals(41, 10000) * 3]).astype(np.float32)
    y = oracle.gelu_approx(x)
    assert oracle.gelu_approx(np.zeros(1, np.float32))[0] == 0.0
    # tanh-GELU(x) - tanh-GELU(-x) = x exactly in real arithmetic.
    yn = oracle.gelu_approx(-x)
    assert np.max(np.abs((y - yn) - x)) <= 4e-6 * np.maximum(1.0, np.abs(x)).max()
    # Against an independent f64 evaluation of the published formula ...
    xd = x.astype(np.float64)
    ref = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd**3)))
    assert np.max(np.abs(y - ref)) < 2e-6
    # ... and against torch's tanh-approximate GELU, where torch is present.
    torch = pytest.importorskip("torch")
    t = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    assert np.max(np.abs(y - t)) < 2e-6
