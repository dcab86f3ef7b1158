"""Test helpers for the GGUF path: block encoders, random blocks and a GGUF
file writer.

The encoders go the other way from the decoders under test -- from integer
codes and scales to the llama.cpp block bytes (the layouts mlx_gguf.rs:27-40
names and its decoders at mlx_gguf.rs:324-438 read) -- so a transposed nibble
half, a wrong high-bit index or a mis-split scale byte in a decoder shows up as
a mismatch against values computed here from the codes.
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 8, 12, 13, 14, 30
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q8_0: (32, 34),
         Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}
ALL_TYPES = [F32, F16, BF16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K]


def f16_bits(v: float) -> int:
    return int(np.array([v], dtype=np.float16).view(np.uint16)[0])


def f16_val(bits: int) -> np.float32:
    return np.array([bits], dtype=np.uint16).view(np.float16).astype(np.float32)[0]


# ---- encoders (codes -> bytes) -------------------------------------------------


def enc_q4_0(d_bits: int, q: np.ndarray) -> bytes:
    """q: 32 codes in 0..15; value i is d * (q[i] - 8)."""
    q = np.asarray(q, dtype=np.uint8)
    body = (q[:16] & 15) | ((q[16:] & 15) << 4)
    return struct.pack("<H", d_bits) + body.astype(np.uint8).tobytes()


def enc_q8_0(d_bits: int, q: np.ndarray) -> bytes:
    """q: 32 signed codes; value i is d * q[i]."""
    return struct.pack("<H", d_bits) + np.asarray(q, dtype=np.int8).tobytes()


def pack_scale_min_k4(sc: np.ndarray, m: np.ndarray) -> bytes:
    """Eight 6-bit (scale, min) pairs into 12 bytes: pairs 0-3 in the low six
    bits of bytes 0-3 / 4-7, pairs 4-7 as low nibbles in bytes 8-11 and their
    top two bits in the top bits of bytes 0-3 / 4-7."""
    sc = [int(v) for v in sc]
    m = [int(v) for v in m]
    out = [0] * 12
    for j in range(4):
        out[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        out[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        out[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return bytes(out)


def _nibbles_k(q: np.ndarray) -> np.ndarray:
    """256 4-bit codes -> 128 bytes: sub-block j's 32 codes are the low (even
    j) or high (odd j) nibbles of 32-byte half j // 2."""
    q = np.asarray(q, dtype=np.uint8).reshape(8, 32)
    out = np.zeros((4, 32), dtype=np.uint8)
    for h in range(4):
        out[h] = (q[2 * h] & 15) | ((q[2 * h + 1] & 15) << 4)
    return out.reshape(-1)


def enc_q4_k(d_bits: int, dmin_bits: int, sc, m, q) -> bytes:
    """q: 256 codes 0..15; value j*32+i is d*sc[j]*q - dmin*m[j]."""
    return (struct.pack("<HH", d_bits, dmin_bits) + pack_scale_min_k4(sc, m)
            + _nibbles_k(q).tobytes())


def enc_q5_k(d_bits: int, dmin_bits: int, sc, m, q) -> bytes:
    """q: 256 codes 0..31; bit 4 of code j*32+i is bit j of qh[i]."""
    q = np.asarray(q, dtype=np.uint8).reshape(8, 32)
    qh = np.zeros(32, dtype=np.uint8)
    for j in range(8):
        qh |= (((q[j] >> 4) & 1) << j).astype(np.uint8)
    return (struct.pack("<HH", d_bits, dmin_bits) + pack_scale_min_k4(sc, m) + qh.tobytes()
            + _nibbles_k(q.reshape(-1) & 15).tobytes())


def enc_q6_k(d_bits: int, sc, q) -> bytes:
    """q: 256 codes 0..63 (value = d * sc * (q - 32)); sc: 16 signed scales,
    scale of value n*128 + r*32 + l being sc[n*8 + l//16 + 2r]."""
    q = np.asarray(q, dtype=np.uint8).reshape(2, 4, 32)
    ql = np.zeros((2, 64), dtype=np.uint8)
    qh = np.zeros((2, 32), dtype=np.uint8)
    for n in range(2):
        ql[n, :32] = (q[n, 0] & 15) | ((q[n, 2] & 15) << 4)
        ql[n, 32:] = (q[n, 1] & 15) | ((q[n, 3] & 15) << 4)
        qh[n] = (q[n, 0] >> 4) | ((q[n, 1] >> 4) << 2) | ((q[n, 2] >> 4) << 4) | ((q[n, 3] >> 4) << 6)
    return (ql.tobytes() + qh.tobytes() + np.asarray(sc, dtype=np.int8).tobytes()
            + struct.pack("<H", d_bits))


# ---- values of encoded blocks, in the reference's f32 operation order -----------


def val_q4_0(d_bits, q):
    d = f16_val(d_bits)
    return (d * (np.asarray(q, np.int32) - 8).astype(np.float32)).astype(np.float32)


def val_q8_0(d_bits, q):
    return (f16_val(d_bits) * np.asarray(q, np.int8).astype(np.float32)).astype(np.float32)


def val_qk(d_bits, dmin_bits, sc, m, q):
    d, dmin = f16_val(d_bits), f16_val(dmin_bits)
    sc = np.repeat(np.asarray(sc, np.float32), 32)
    m = np.repeat(np.asarray(m, np.float32), 32)
    d1 = (d * sc).astype(np.float32)
    m1 = (dmin * m).astype(np.float32)
    return ((d1 * np.asarray(q, np.float32)).astype(np.float32) - m1).astype(np.float32)


def val_q6_k(d_bits, sc, q):
    d = f16_val(d_bits)
    sc = np.asarray(sc, np.int8).astype(np.float32)
    idx = np.arange(256)
    n, r, l = idx // 128, (idx // 32) % 4, idx % 32
    s = sc[n * 8 + l // 16 + 2 * r]
    return ((d * s).astype(np.float32) * (np.asarray(q, np.int32) - 32).astype(np.float32)).astype(np.float32)


# ---- random tensors ---------------------------------------------------------------


def random_finite_half(rng, lo=1e-4, hi=4e-2, n=None):
    v = np.asarray(rng.uniform(lo, hi, size=n)).astype(np.float16)
    return v.view(np.uint16)


def random_tensor(kind: int, n: int, rng, finite: bool = True) -> bytes:
    """Raw bytes of an n-value tensor of GGML type `kind`.  finite=True keeps
    the block scales finite and positive (code bytes random); finite=False is
    random bytes throughout (NaN, infinite and subnormal scales included)."""
    per, nbytes = BLOCK[kind]
    blocks = n // per
    if not finite:
        return rng.integers(0, 256, size=blocks * nbytes, dtype=np.uint8).tobytes()
    if kind == F32:
        return rng.standard_normal(n).astype(np.float32).tobytes()
    if kind == F16:
        return rng.standard_normal(n).astype(np.float16).tobytes()
    if kind == BF16:
        f = rng.standard_normal(n).astype(np.float32).view(np.uint32)
        return (f >> 16).astype(np.uint16).tobytes()
    raw = np.frombuffer(rng.integers(0, 256, size=blocks * nbytes, dtype=np.uint8).tobytes(),
                        dtype=np.uint8).reshape(blocks, nbytes).copy()
    if kind in (Q4_0, Q8_0):
        raw[:, 0:2] = random_finite_half(rng, n=blocks).view(np.uint8).reshape(blocks, 2)
    elif kind in (Q4_K, Q5_K):
        raw[:, 0:2] = random_finite_half(rng, n=blocks).view(np.uint8).reshape(blocks, 2)
        raw[:, 2:4] = random_finite_half(rng, n=blocks).view(np.uint8).reshape(blocks, 2)
    elif kind == Q6_K:
        raw[:, 208:210] = random_finite_half(rng, n=blocks).view(np.uint8).reshape(blocks, 2)
    return raw.tobytes()


# ---- a GGUF file writer -------------------------------------------------------------


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _kv_value(kind: int, v) -> bytes:
    fmt = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?",
           10: "<Q", 11: "<q", 12: "<d"}
    if kind in fmt:
        return struct.pack(fmt[kind], v)
    if kind == 8:
        return _str(v)
    if kind == 9:
        inner, items = v
        return struct.pack("<IQ", inner, len(items)) + b"".join(_kv_value(inner, x) for x in items)
    raise ValueError(kind)


def write_gguf(path: Path, tensors, metadata=(), version: int = 3, align: int = 32) -> None:
    """tensors: (name, row-major shape, GGML type, raw bytes); metadata:
    (key, value type, value).  Each tensor's data starts at a multiple of
    `align` past the data start, which is the first multiple of `align`
    after the directory."""
    head = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(metadata))
    for key, kind, v in metadata:
        head += _str(key) + struct.pack("<I", kind) + _kv_value(kind, v)
    offset = 0
    blobs = []
    for name, shape, kind, raw in tensors:
        dims = list(reversed(list(shape)))
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", kind, offset)
        blobs.append((offset, raw))
        offset = (offset + len(raw) + align - 1) // align * align
    data_start = (len(head) + align - 1) // align * align
    body = bytearray(offset)
    for off, raw in blobs:
        body[off:off + len(raw)] = raw
    Path(path).write_bytes(head + b"\0" * (data_start - len(head)) + bytes(body))
