"""Pins the oracle's GGUF block decoders (oracle/sdq_oracle_gguf.c) before the
GPU path is compared with it.

- f16: every one of the 65536 patterns against numpy's float16 -> float32 and
  against the oracle's bit-construction decoder; NaN patterns give the
  reference's canonical NaN (mlx_gguf.rs:302-318, test at 464-475).
- bf16: the reference's own known answers (mlx_gguf.rs:504-540).
- each block type: a hand-worked block whose values are written out below,
  and random blocks built by the encoders in gguf_blocks.py (codes -> bytes,
  the inverse direction of the decoder).
"""
from __future__ import annotations

import numpy as np
import pytest

import gguf_blocks as gb


def _dec(oracle, raw: bytes, kind: int, n: int) -> np.ndarray:
    return oracle.gguf_dequantize(np.frombuffer(raw, dtype=np.uint8), kind, n)


def test_f16_every_pattern(oracle):
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = _dec(oracle, pats.tobytes(), gb.F16, 65536)
    want = pats.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # NaNs come out as the reference's f32::NAN, whatever their sign and payload.
    assert np.all(got[nan].view(np.uint32) == 0x7FC00000)
    # The smallest subnormal is where a factor-of-two slip first shows.
    assert oracle.gguf_f16(0x0001) == 2.0 ** -24
    bitwise = np.array([oracle.f32_from_f16(int(h)) for h in pats[::97]], dtype=np.float32)
    sub = got[::97]
    ok = ~np.isnan(bitwise)
    assert np.array_equal(sub[ok].view(np.uint32), bitwise[ok].view(np.uint32))


def test_bf16_known_answers(oracle):
    pats = np.array([0x3F80, 0x4900, 0x8000, 0x7F80, 0xFF80, 0x7FC0], dtype=np.uint16)
    got = _dec(oracle, pats.tobytes(), gb.BF16, pats.size)
    assert got[0] == 1.0 and got[1] == 524288.0
    assert got[2] == 0.0 and np.signbit(got[2])
    assert np.isposinf(got[3]) and np.isneginf(got[4]) and np.isnan(got[5])
    # Widening is exact: f32 values truncated to their top half round-trip.
    vals = np.array([0.0, 1.0, -1.0, 2.0, 0.5, -0.125, 3.0e38, -3.0e38, 1.0e38], dtype=np.float32)
    top = (vals.view(np.uint32) >> 16).astype(np.uint16)
    trunc = (vals.view(np.uint32) & 0xFFFF0000).view(np.float32)
    assert np.array_equal(_dec(oracle, top.tobytes(), gb.BF16, top.size), trunc)


def test_f32_is_copied(oracle):
    v = np.array([1.5, -0.0, np.inf, 3.0e-45], dtype=np.float32)
    assert np.array_equal(_dec(oracle, v.tobytes(), gb.F32, 4).view(np.uint32), v.view(np.uint32))


def test_q4_0_hand_worked(oracle):
    # d = 0.5; byte i holds code i (low) and 15 - i (high): values 0..15 are
    # 0.5*(i-8), values 16..31 are 0.5*(7-i).
    raw = bytes([0x00, 0x38]) + bytes((i | ((15 - i) << 4)) for i in range(16))
    got = _dec(oracle, raw, gb.Q4_0, 32)
    want = [-4.0, -3.5, -3.0, -2.5, -2.0, -1.5, -1.0, -0.5, 0.0, 0.5, 1.0, 1.5, 2.0, 2.5, 3.0, 3.5,
            3.5, 3.0, 2.5, 2.0, 1.5, 1.0, 0.5, 0.0, -0.5, -1.0, -1.5, -2.0, -2.5, -3.0, -3.5, -4.0]
    assert got.tolist() == want


def test_q8_0_hand_worked(oracle):
    q = [-128, -1, 0, 1, 127] + [2] * 27
    raw = bytes([0x00, 0x34]) + np.array(q, dtype=np.int8).tobytes()  # d = 0.25
    got = _dec(oracle, raw, gb.Q8_0, 32)
    assert got[:6].tolist() == [-32.0, -0.25, 0.0, 0.25, 31.75, 0.5]


SCALES_12 = bytes([0x41, 0x02, 0x03, 0x04, 0x45, 0x06, 0x07, 0x08, 0x21, 0x43, 0x65, 0x87])
# (scale, min) of sub-blocks 0..7 unpacked by hand from SCALES_12: 0-3 are the
# low six bits of bytes 0-3 and 4-7; 4-7 take a nibble of bytes 8-11 and the
# top two bits of bytes 0-7.
SCALE_MIN = [(1, 5), (2, 6), (3, 7), (4, 8), (17, 18), (3, 4), (5, 6), (7, 8)]


def test_scale_min_packing_matches_the_hand_unpacking():
    sc = [p[0] for p in SCALE_MIN]
    m = [p[1] for p in SCALE_MIN]
    assert gb.pack_scale_min_k4(sc, m) == SCALES_12


def test_q4_k_hand_worked(oracle):
    # d = 1, dmin = 0.5; every code byte 0x3A: even sub-blocks read 10, odd 3.
    raw = bytes([0x00, 0x3C, 0x00, 0x38]) + SCALES_12 + bytes([0x3A]) * 128
    got = _dec(oracle, raw, gb.Q4_K, 256).reshape(8, 32)
    want = [7.5, 3.0, 26.5, 8.0, 161.0, 7.0, 47.0, 17.0]
    assert np.array_equal(got, np.repeat(np.array(want, np.float32)[:, None], 32, axis=1))


def test_q5_k_hand_worked(oracle):
    # As above with qh = 0xA5 everywhere: bit j set for j in {0, 2, 5, 7}
    # adds 16 to those sub-blocks' codes.
    raw = bytes([0x00, 0x3C, 0x00, 0x38]) + SCALES_12 + bytes([0xA5]) * 32 + bytes([0x3A]) * 128
    got = _dec(oracle, raw, gb.Q5_K, 256).reshape(8, 32)
    want = [23.5, 3.0, 74.5, 8.0, 161.0, 55.0, 47.0, 129.0]
    assert np.array_equal(got, np.repeat(np.array(want, np.float32)[:, None], 32, axis=1))


def test_q6_k_hand_worked(oracle):
    # d = 0.5; ql bytes 0x21 (low 1, high 2); qh bytes 0xE4 (quarters r read
    # high bits 0, 1, 2, 3): codes -31, -15, 2, 18 for r = 0..3.
    sc = [1, -1, 2, -2, 3, -3, 4, -4, 5, -5, 6, -6, 7, -7, 8, -8]
    raw = bytes([0x21]) * 128 + bytes([0xE4]) * 64 + np.array(sc, np.int8).tobytes() + bytes([0x00, 0x38])
    got = _dec(oracle, raw, gb.Q6_K, 256).reshape(2, 4, 2, 16)
    want = np.array([
        [[-15.5, 15.5], [-15.0, 15.0], [3.0, -3.0], [36.0, -36.0]],
        [[-77.5, 77.5], [-45.0, 45.0], [7.0, -7.0], [72.0, -72.0]],
    ], dtype=np.float32)
    assert np.array_equal(got, np.repeat(want[..., None], 16, axis=3))


@pytest.mark.parametrize("kind", [gb.Q4_0, gb.Q8_0, gb.Q4_K, gb.Q5_K, gb.Q6_K])
def test_random_blocks_against_the_encoders(oracle, kind):
    rng = np.random.default_rng(7 + kind)
    raws, wants = [], []
    for _ in range(24):
        d = int(gb.random_finite_half(rng, 1e-3, 2.0))
        dm = int(gb.random_finite_half(rng, 1e-3, 2.0))
        if kind == gb.Q4_0:
            q = rng.integers(0, 16, 32)
            raws.append(gb.enc_q4_0(d, q))
            wants.append(gb.val_q4_0(d, q))
        elif kind == gb.Q8_0:
            q = rng.integers(-128, 128, 32)
            raws.append(gb.enc_q8_0(d, q))
            wants.append(gb.val_q8_0(d, q))
        elif kind in (gb.Q4_K, gb.Q5_K):
            sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
            q = rng.integers(0, 16 if kind == gb.Q4_K else 32, 256)
            enc = gb.enc_q4_k if kind == gb.Q4_K else gb.enc_q5_k
            raws.append(enc(d, dm, sc, m, q))
            wants.append(gb.val_qk(d, dm, sc, m, q))
        else:
            sc, q = rng.integers(-128, 128, 16), rng.integers(0, 64, 256)
            raws.append(gb.enc_q6_k(d, sc, q))
            wants.append(gb.val_q6_k(d, sc, q))
    per = gb.BLOCK[kind][0]
    got = _dec(oracle, b"".join(raws), kind, per * len(raws))
    want = np.concatenate(wants)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_rejects_bad_sizes_and_types(oracle):
    with pytest.raises(ValueError):
        oracle.gguf_dequantize(np.zeros(18, np.uint8), gb.Q4_0, 16)   # not a whole block
    with pytest.raises(ValueError):
        oracle.gguf_dequantize(np.zeros(17, np.uint8), gb.Q4_0, 32)   # bytes short
    with pytest.raises(ValueError):
        oracle.gguf_dequantize(np.zeros(4, np.uint8), 3, 1)           # Q4_1: unsupported
    assert oracle.gguf_block(gb.Q6_K) == (256, 210)


def test_block_nans_are_the_positive_quiet_nan(oracle):
    """inf * 0 (x86 would give its negative indefinite NaN) and a NaN min both
    decode to 0x7FC00000, the NaN of the reference's arm64 platform."""
    sc = [0, 1, 2, 3, 4, 5, 6, 7]
    raw_inf = gb.enc_q4_k(0x7C00, 0x3C00, sc, [0] * 8, np.zeros(256, np.uint8))   # d = +inf
    raw_nan = gb.enc_q4_k(0x3C00, 0xFE00, sc, [1] * 8, np.zeros(256, np.uint8))   # dmin = -NaN
    got = _dec(oracle, raw_inf + raw_nan, gb.Q4_K, 512).view(np.uint32)
    assert np.all(got[:32] == 0x7FC00000)          # sub-block 0: (inf * 0) * 0
    assert np.all(got[256:] == 0x7FC00000)         # every value minus a NaN
