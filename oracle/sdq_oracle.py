"""numpy-facing wrapper of the CPU oracle (oracle/_build/libsdq_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product library never loads
it.  See sdq_oracle.h for what each function restates and where from.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libsdq_oracle.so"

UINT32, FLOAT16, FLOAT32, BFLOAT16 = 3, 9, 10, 12

_lib = None


def build() -> Path:
    """Compile the oracle with its Makefile (gcc; no GPU needed)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i64, c_int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.sdo_rng_next_u64.restype = ctypes.c_uint64
        L.sdo_rng_next_u64.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.sdo_rng_next_f64.restype = ctypes.c_double
        L.sdo_rng_next_f64.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.sdo_rng_normals.restype = None
        L.sdo_rng_normals.argtypes = [ctypes.POINTER(ctypes.c_uint64), vp, ctypes.c_size_t]
        L.sdo_quantize.restype = c_int
        L.sdo_quantize.argtypes = [vp, i64, i64, c_int, c_int, c_int, vp, vp, vp]
        L.sdo_dequantize.restype = c_int
        L.sdo_dequantize.argtypes = [vp, vp, vp, c_int, i64, i64, c_int, c_int, vp]
        L.sdo_qmatmul.restype = c_int
        L.sdo_qmatmul.argtypes = [vp, i64, i64, vp, vp, vp, i64, c_int, c_int, vp]
        L.sdo_qmatmul_f64.restype = c_int
        L.sdo_qmatmul_f64.argtypes = [vp, i64, i64, vp, vp, vp, i64, c_int, c_int, vp]
        L.sdo_qmatmul_omp.restype = c_int
        L.sdo_qmatmul_omp.argtypes = [vp, i64, i64, vp, vp, vp, i64, c_int, c_int, vp, c_int]
        L.sdo_resident_bytes.restype = ctypes.c_uint64
        L.sdo_resident_bytes.argtypes = [i64, i64, c_int, c_int]
        L.sdo_gelu_approx.restype = None
        L.sdo_gelu_approx.argtypes = [vp, vp, ctypes.c_size_t]
        fp = vp
        L.sdo_layer_norm.restype = None
        L.sdo_layer_norm.argtypes = [fp, i64, i64, ctypes.c_float, fp, fp, fp]
        L.sdo_rms_norm.restype = None
        L.sdo_rms_norm.argtypes = [fp, i64, i64, ctypes.c_float, fp, fp]
        L.sdo_norm_modulate.restype = None
        L.sdo_norm_modulate.argtypes = [fp, i64, i64, i64, ctypes.c_float, fp, fp, fp]
        L.sdo_rope.restype = None
        L.sdo_rope.argtypes = [fp, i64, i64, i64, fp, fp, fp]
        L.sdo_embed_nd.restype = c_int
        L.sdo_embed_nd.argtypes = [fp, i64, fp, i64, ctypes.c_float, fp, fp]
        L.sdo_sdpa.restype = c_int
        L.sdo_sdpa.argtypes = [fp, fp, fp, i64, i64, i64, i64, i64, i64, ctypes.c_float, c_int, i64, fp,
                               i64, i64, i64, fp]
        L.sdo_gguf_block.restype = c_int
        L.sdo_gguf_block.argtypes = [c_int, ctypes.POINTER(i64), ctypes.POINTER(i64)]
        L.sdo_gguf_f16.restype = ctypes.c_float
        L.sdo_gguf_f16.argtypes = [ctypes.c_uint16]
        L.sdo_gguf_dequantize.restype = c_int
        L.sdo_gguf_dequantize.argtypes = [vp, ctypes.c_size_t, c_int, i64, vp]
        for n in ("sdo_bf16_from_f32", "sdo_f16_from_f32"):
            getattr(L, n).restype = ctypes.c_uint16
            getattr(L, n).argtypes = [ctypes.c_float]
        for n in ("sdo_f32_from_bf16", "sdo_f32_from_f16"):
            getattr(L, n).restype = ctypes.c_float
            getattr(L, n).argtypes = [ctypes.c_uint16]
        _lib = L
    return _lib


def _p(a: np.ndarray) -> ctypes.c_void_p:
    return a.ctypes.data_as(ctypes.c_void_p)


class Rng:
    """SeededRng (crates/sd-tensor/src/lib.rs:105-145)."""

    def __init__(self, seed: int):
        self.state = ctypes.c_uint64(seed)

    def next_u64(self) -> int:
        return lib().sdo_rng_next_u64(ctypes.byref(self.state))

    def next_f64(self) -> float:
        return lib().sdo_rng_next_f64(ctypes.byref(self.state))

    def normals(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        lib().sdo_rng_normals(ctypes.byref(self.state), _p(out), n)
        return out


def normals(seed: int, n: int, scale: float = 1.0) -> np.ndarray:
    v = Rng(seed).normals(n)
    if scale != 1.0:
        v = (v * np.float32(scale)).astype(np.float32)
    return v


def _store_np(dtype: int):
    return np.float32 if dtype == FLOAT32 else np.uint16


def quantize(w: np.ndarray, group_size: int = 64, bits: int = 4, store_dtype: int = FLOAT32):
    """w [rows, cols] (f32 values) -> (wq uint32, scales, biases); scales and
    biases as f32 arrays, or raw uint16 bits for bf16/f16 storage."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    wq = np.zeros((rows, cols * bits // 32), dtype=np.uint32)
    sc = np.zeros((rows, cols // group_size), dtype=_store_np(store_dtype))
    bi = np.zeros_like(sc)
    rc = lib().sdo_quantize(_p(w), rows, cols, group_size, bits, store_dtype, _p(wq), _p(sc), _p(bi))
    if rc != 0:
        raise ValueError("oracle quantize rejected its arguments")
    return wq, sc, bi


def dequantize(wq, scales, biases, group_size=64, bits=4, scale_dtype: int = FLOAT32) -> np.ndarray:
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    sc = np.ascontiguousarray(scales, dtype=_store_np(scale_dtype))
    bi = np.ascontiguousarray(biases, dtype=_store_np(scale_dtype))
    rows = wq.shape[0]
    cols = wq.shape[1] * 32 // bits
    out = np.empty((rows, cols), dtype=np.float32)
    rc = lib().sdo_dequantize(_p(wq), _p(sc), _p(bi), scale_dtype, rows, cols, group_size, bits, _p(out))
    if rc != 0:
        raise ValueError("oracle dequantize rejected its arguments")
    return out


def _mm_args(x, wq, scales, biases, bits):
    x = np.ascontiguousarray(x, dtype=np.float32)
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    sc = np.ascontiguousarray(scales, dtype=np.float32)
    bi = np.ascontiguousarray(biases, dtype=np.float32)
    M, K = x.shape
    N = wq.shape[0]
    assert wq.shape[1] * 32 // bits == K
    return x, wq, sc, bi, M, N, K


def qmatmul(x, wq, scales, biases, group_size=64, bits=4) -> np.ndarray:
    x, wq, sc, bi, M, N, K = _mm_args(x, wq, scales, biases, bits)
    y = np.empty((M, N), dtype=np.float32)
    if lib().sdo_qmatmul(_p(x), M, K, _p(wq), _p(sc), _p(bi), N, group_size, bits, _p(y)) != 0:
        raise ValueError("oracle qmatmul rejected its arguments")
    return y


def qmatmul_f64(x, wq, scales, biases, group_size=64, bits=4) -> np.ndarray:
    x, wq, sc, bi, M, N, K = _mm_args(x, wq, scales, biases, bits)
    y = np.empty((M, N), dtype=np.float64)
    if lib().sdo_qmatmul_f64(_p(x), M, K, _p(wq), _p(sc), _p(bi), N, group_size, bits, _p(y)) != 0:
        raise ValueError("oracle qmatmul_f64 rejected its arguments")
    return y


def qmatmul_omp(x, wq, scales, biases, group_size=64, bits=4, threads: int = 0) -> np.ndarray:
    x, wq, sc, bi, M, N, K = _mm_args(x, wq, scales, biases, bits)
    y = np.empty((M, N), dtype=np.float32)
    t = threads or (os.cpu_count() or 1)
    if lib().sdo_qmatmul_omp(_p(x), M, K, _p(wq), _p(sc), _p(bi), N, group_size, bits, _p(y), t) != 0:
        raise ValueError("oracle qmatmul_omp rejected its arguments")
    return y


def resident_bytes(rows: int, cols: int, group_size: int = 64, bits: int = 4) -> int:
    return int(lib().sdo_resident_bytes(rows, cols, group_size, bits))


def gelu_approx(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().sdo_gelu_approx(_p(x), _p(y), x.size)
    return y


def bf16_from_f32(v: float) -> int:
    return lib().sdo_bf16_from_f32(v)


def f32_from_bf16(h: int) -> float:
    return lib().sdo_f32_from_bf16(h)


def f16_from_f32(v: float) -> int:
    return lib().sdo_f16_from_f32(v)


def f32_from_f16(h: int) -> float:
    return lib().sdo_f32_from_f16(h)


# ---- GGUF block decoding (sdq_oracle_gguf.c; mlx_gguf.rs:27-438) ----------

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0 = 0, 1, 2, 8
GGML_Q4_K, GGML_Q5_K, GGML_Q6_K, GGML_BF16 = 12, 13, 14, 30


def gguf_block(ggml_type: int) -> tuple[int, int]:
    """(values per block, bytes per block) of a GGML type."""
    v, b = ctypes.c_int64(), ctypes.c_int64()
    if lib().sdo_gguf_block(ggml_type, ctypes.byref(v), ctypes.byref(b)) != 0:
        raise ValueError(f"oracle: GGML type {ggml_type} is not supported")
    return v.value, b.value


def gguf_f16(h: int) -> float:
    return lib().sdo_gguf_f16(h)


def gguf_dequantize(raw, ggml_type: int, n: int) -> np.ndarray:
    """Decodes n values of a GGML tensor's raw bytes to f32 (Gguf::dequantize)."""
    raw = np.ascontiguousarray(np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw,
                               dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    if lib().sdo_gguf_dequantize(_p(raw), raw.size, ggml_type, n, _p(out)) != 0:
        raise ValueError("oracle gguf_dequantize rejected its arguments")
    return out


# ---- ops around the Flux block linears (sdq_oracle_block.c) ----------------


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _opt(a):
    return None if a is None else _f32(a)


def _pn(a):
    return None if a is None else _p(a)


def layer_norm(x, eps: float, w=None, b=None) -> np.ndarray:
    x, w, b = _f32(x), _opt(w), _opt(b)
    C = x.shape[-1]
    out = np.empty_like(x)
    lib().sdo_layer_norm(_p(x), x.size // C, C, eps, _pn(w), _pn(b), _p(out))
    return out


def rms_norm(x, eps: float, w=None) -> np.ndarray:
    x, w = _f32(x), _opt(w)
    C = x.shape[-1]
    out = np.empty_like(x)
    lib().sdo_rms_norm(_p(x), x.size // C, C, eps, _pn(w), _p(out))
    return out


def norm_modulate(x, shift, scale, eps: float) -> np.ndarray:
    """x [B, N, C]; shift, scale [B, 1, C] (flux.rs:255-275)."""
    x, shift, scale = _f32(x), _f32(shift), _f32(scale)
    B, N, C = x.shape
    out = np.empty_like(x)
    lib().sdo_norm_modulate(_p(x), B, N, C, eps, _p(shift), _p(scale), _p(out))
    return out


def rope(x, cos, sin) -> np.ndarray:
    """x [..., N, D]; cos, sin [N, D/2] (flux.rs:165-205)."""
    x, cos, sin = _f32(x), _f32(cos), _f32(sin)
    N, D = x.shape[-2], x.shape[-1]
    out = np.empty_like(x)
    lib().sdo_rope(_p(x), x.size // D, D, N, _p(cos), _p(sin), _p(out))
    return out


def embed_nd(ids, axes_dim, theta: float):
    """(cos, sin) [seq, sum(axes_dim)/2] for ids [seq, n_axes] (flux.rs:126-156)."""
    ids = _f32(ids)
    seq, n_axes = ids.shape
    dims = np.ascontiguousarray(axes_dim, dtype=np.int64)
    half = int(dims.sum()) // 2
    cs = np.empty((seq, half), np.float32)
    sn = np.empty((seq, half), np.float32)
    if lib().sdo_embed_nd(_p(ids), seq, _p(dims), n_axes, theta, _p(cs), _p(sn)) != 0:
        raise ValueError("oracle embed_nd rejected its arguments")
    return cs, sn


def sdpa(q, k, v, scale: float, mode: str = "", mask=None, causal_offset=None) -> np.ndarray:
    """softmax(scale q k^T + mask) v in f64; q [B,Hq,Nq,D], k, v [B,Hk,Nk,D];
    mask broadcastable to [B, Hq, Nq, Nk]; causal: key j is visible to query
    i when j <= i + causal_offset (default Nk - Nq)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, Hq, Nq, D = q.shape
    Hk, Nk = k.shape[1], k.shape[2]
    out = np.empty_like(q)
    m = {"": 0, "causal": 1, "array": 2}[mode]
    mp, sb, sh, sq = None, 0, 0, 0
    if m == 2:
        full = np.broadcast_to(_f32(mask), (B, Hq, Nq, Nk))
        mk = _f32(full)
        mp, sb, sh, sq = _p(mk), Hq * Nq * Nk, Nq * Nk, Nk
    off = Nk - Nq if causal_offset is None else causal_offset
    rc = lib().sdo_sdpa(_p(q), _p(k), _p(v), B, Hq, Hk, Nq, Nk, D, scale, m, off, mp, sb, sh, sq, _p(out))
    if rc != 0:
        raise ValueError("oracle sdpa rejected its arguments")
    return out
