"""sdq -- Python binding of libsdq, the MI355X backend of the MLX-affine
quantized linear.

The surface mirrors the reference's Rust seam (crates/sd-tensor/src/mlx.rs) so
that tests read like its own (crates/sd-models/tests/mlx_quantized.rs):

    Stream.gpu() / Stream.cpu()            mlx.rs:472-510
    Array.from_slice_f32, shape, to_vec_f32 mlx.rs:558-612, 1414-1445
    QuantizedArray.quantize / dequantize / matmul / resident_bytes
                                           mlx.rs:1834-1985
    eval(...)                              mlx.rs:1531-1544
    Error                                  crates/sd-tensor/src/error.rs:14-34

Every call goes through the C ABI in include/sdq.h (ctypes).  A failing call
raises Error("sdq: <op>: <message>"), the message delivered by the library's
error handler on the calling thread, exactly as the reference's trampoline
does for mlx-c (mlx.rs:419-470).  There is no fallback: if libsdq.so is
missing, importing works but the first call raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path
from typing import Iterable, Sequence

import numpy as np

__all__ = [
    "Error",
    "Stream",
    "Array",
    "QuantizedArray",
    "eval",
    "lib",
    "LIB_PATH",
    "FLOAT32",
    "BFLOAT16",
    "FLOAT16",
    "UINT32",
    "ACT_NONE",
    "ACT_GELU_APPROX",
    "COMBINE_NONE",
    "COMBINE_GATED_RESIDUAL",
    "COMBINE_PRODUCT",
    "f32_to_bf16_bits",
    "bf16_bits_to_f32",
    "gguf_dequantize",
    "pair_rows",
]

LIB_PATH = Path(__file__).with_name("libsdq.so")

# Positions of mlx_dtype (mlx.rs:100-104), shared by include/sdq.h.
BOOL, UINT8, UINT16, UINT32, UINT64 = 0, 1, 2, 3, 4
INT8, INT16, INT32, INT64 = 5, 6, 7, 8
FLOAT16, FLOAT32, FLOAT64, BFLOAT16, COMPLEX64 = 9, 10, 11, 12, 13

# sdq_activation and sdq_combine (include/sdq.h): the matmul epilogue.
ACT_NONE, ACT_GELU_APPROX = 0, 1
COMBINE_NONE, COMBINE_GATED_RESIDUAL, COMBINE_PRODUCT = 0, 1, 2

_NP_OF = {
    FLOAT32: np.float32,
    FLOAT16: np.float16,
    BFLOAT16: np.uint16,  # raw bf16 bit patterns
    UINT32: np.uint32,
    INT32: np.int32,
    UINT16: np.uint16,
    UINT8: np.uint8,
}
_NAMES = {FLOAT32: "float32", FLOAT16: "float16", BFLOAT16: "bfloat16", UINT32: "uint32"}


class Error(Exception):
    """A failed call: the status was non-zero; the text is the library's."""


# ---- ctypes declarations ---------------------------------------------------


class _Handle(ctypes.Structure):
    _fields_ = [("ctx", ctypes.c_void_p)]


class CArray(_Handle):
    pass


class CStream(_Handle):
    pass


class CVectorArray(_Handle):
    pass


class COptionalInt(ctypes.Structure):
    _fields_ = [("value", ctypes.c_int), ("has_value", ctypes.c_bool)]


class COptionalDtype(ctypes.Structure):
    _fields_ = [("value", ctypes.c_int), ("has_value", ctypes.c_bool)]


_HANDLER_T = ctypes.CFUNCTYPE(None, ctypes.c_char_p, ctypes.c_void_p)
_tls = threading.local()


@_HANDLER_T
def _error_handler(msg, _data):
    _tls.last = msg.decode("utf-8", "replace") if msg else ""


_lib = None
_lib_lock = threading.Lock()


def _declare(L: ctypes.CDLL) -> None:
    A, S, V = CArray, CStream, CVectorArray
    P = ctypes.POINTER
    c_int, c_size, c_bool, c_vp = ctypes.c_int, ctypes.c_size_t, ctypes.c_bool, ctypes.c_void_p
    sig = {
        "sdq_set_error_handler": (None, [_HANDLER_T, c_vp, c_vp]),
        "sdq_array_new": (A, []),
        "sdq_array_new_data": (A, [c_vp, P(c_int), c_int, c_int]),
        "sdq_array_new_float32": (A, [ctypes.c_float]),
        "sdq_array_free": (c_int, [A]),
        "sdq_array_size": (c_size, [A]),
        "sdq_array_ndim": (c_size, [A]),
        "sdq_array_shape": (P(c_int), [A]),
        "sdq_array_dtype": (c_int, [A]),
        "sdq_array_nbytes": (c_size, [A]),
        "sdq_array_eval": (c_int, [A]),
        "sdq_array_data_float32": (P(ctypes.c_float), [A]),
        "sdq_array_data_uint32": (P(ctypes.c_uint32), [A]),
        "sdq_array_data_bfloat16": (P(ctypes.c_uint16), [A]),
        "sdq_array_data_float16": (P(ctypes.c_uint16), [A]),
        "sdq_array_copy_to_host": (c_int, [c_vp, c_size, A]),
        "sdq_vector_array_new": (V, []),
        "sdq_vector_array_new_value": (V, [A]),
        "sdq_vector_array_append_value": (c_int, [V, A]),
        "sdq_vector_array_size": (c_size, [V]),
        "sdq_vector_array_get": (c_int, [P(A), V, c_size]),
        "sdq_vector_array_free": (c_int, [V]),
        "sdq_default_gpu_stream_new": (S, []),
        "sdq_default_cpu_stream_new": (S, []),
        "sdq_gpu_stream_new": (S, []),
        "sdq_stream_free": (c_int, [S]),
        "sdq_synchronize": (c_int, [S]),
        "sdq_stream_native": (c_vp, [S]),
        "sdq_eval": (c_int, [V]),
        "sdq_get_active_memory": (c_int, [P(c_size)]),
        "sdq_get_peak_memory": (c_int, [P(c_size)]),
        "sdq_get_cache_memory": (c_int, [P(c_size)]),
        "sdq_reset_peak_memory": (c_int, []),
        "sdq_set_cache_limit": (c_int, [P(c_size), c_size]),
        "sdq_clear_cache": (c_int, []),
        "sdq_quantize": (c_int, [P(V), A, COptionalInt, COptionalInt, ctypes.c_char_p, A, S]),
        "sdq_dequantize": (
            c_int,
            [P(A), A, A, A, COptionalInt, COptionalInt, ctypes.c_char_p, A, COptionalDtype, S],
        ),
        "sdq_quantized_matmul": (
            c_int,
            [P(A), A, A, A, A, c_bool, COptionalInt, COptionalInt, ctypes.c_char_p, S],
        ),
        "sdq_quantized_linear": (
            c_int,
            [P(A), A, A, A, A, A, c_int, COptionalInt, COptionalInt, ctypes.c_char_p, S],
        ),
        "sdq_quantized_linear_combine": (
            c_int,
            [P(A), A, A, A, A, A, c_int, A, A, c_int, COptionalInt, COptionalInt, ctypes.c_char_p, S],
        ),
        "sdq_add": (c_int, [P(A), A, A, S]),
        "sdq_multiply": (c_int, [P(A), A, A, S]),
        "sdq_astype": (c_int, [P(A), A, c_int, S]),
        "sdq_contiguous": (c_int, [P(A), A, c_bool, S]),
        "sdq_gelu_approx": (c_int, [P(A), A, S]),
        "sdq_matmul_nt": (c_int, [P(A), A, A, S]),
        "sdq_quantized_matmul_raw": (
            c_int,
            [c_vp, c_int, c_vp, c_int, ctypes.c_int64, c_vp, c_vp, c_vp, c_int,
             ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, c_int, c_int, c_vp],
        ),
        "sdq_quantized_matmul_epilogue_raw": (
            c_int,
            [c_vp, c_int, c_vp, c_int, ctypes.c_int64, c_vp, c_vp, c_vp, c_int,
             ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, c_int, c_int, c_vp, c_int, c_int, c_vp],
        ),
        "sdq_quantized_matmul_noalloc": (
            c_int,
            [c_vp, c_int, c_vp, c_int, ctypes.c_int64, c_vp, c_vp, c_vp, c_int,
             ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, c_int, c_int, c_vp, c_int, c_int, c_vp],
        ),
        "sdq_quantized_linear_split_raw": (
            c_int,
            [c_vp, ctypes.c_int64, c_int, c_vp, ctypes.c_int64, c_int, ctypes.c_int64, c_int, c_vp, c_int,
             ctypes.c_int64, c_vp, c_vp, c_vp, c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, c_int,
             c_int, c_vp, c_int, c_vp],
        ),
        "sdq_quantized_linear_gated_raw": (
            c_int,
            [c_vp, ctypes.c_int64, c_int, c_vp, c_int, ctypes.c_int64, c_vp, c_vp, c_vp, c_int,
             ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, c_int, c_int, c_vp, c_int, c_int, c_vp],
        ),
        "sdq_quantized_linear_gated": (
            c_int,
            [P(A), A, A, A, A, A, c_int, COptionalInt, COptionalInt, ctypes.c_char_p, S],
        ),
        "sdq_pair_rows": (c_int, [P(A), A, A, S]),
        "sdq_gelu_approx_raw": (c_int, [c_vp, c_vp, c_int, ctypes.c_int64, c_vp]),
        "sdq_gguf_dequantize": (c_int, [P(A), A, c_int, P(c_int), c_int, S]),
        "sdq_fast_layer_norm": (c_int, [P(A), A, A, A, ctypes.c_float, S]),
        "sdq_fast_rms_norm": (c_int, [P(A), A, A, ctypes.c_float, S]),
        "sdq_fast_scaled_dot_product_attention": (
            c_int, [P(A), A, A, A, ctypes.c_float, ctypes.c_char_p, A, A, S]),
        "sdq_flux_norm_modulate": (c_int, [P(A), A, A, A, ctypes.c_float, S]),
        "sdq_flux_rope": (c_int, [P(A), A, A, A, S]),
        "sdq_flux_attention": (
            c_int, [P(A), A, A, A, A, A, A, A, A, c_int, ctypes.c_float, ctypes.c_float, S]),
        "sdq_flux_single_linear1_attention": (
            c_int, [P(A), A, A, A, A, A, COptionalInt, COptionalInt, ctypes.c_char_p, A, A, A, A, c_int,
                    ctypes.c_float, ctypes.c_float, S]),
        "sdq_gguf_quantize": (c_int, [P(V), A, c_int, P(c_int), c_int, COptionalInt, COptionalInt, S]),
        "sdq_array_device_ptr": (c_vp, [A]),
        "sdq_version": (ctypes.c_char_p, []),
        "sdq_device_count": (c_int, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def lib() -> ctypes.CDLL:
    """The loaded libsdq.so, with the error handler installed once per process
    (mlx.rs:447-453)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise Error(
                    f"sdq: {LIB_PATH} is not built; run `python stable-diffusion.rs_amd/build.py` "
                    "(there is no fallback path)"
                )
            L = ctypes.CDLL(str(LIB_PATH))
            _declare(L)
            L.sdq_set_error_handler(_error_handler, None, None)
            _lib = L
    return _lib


def _take_last_error() -> str | None:
    msg = getattr(_tls, "last", None)
    _tls.last = None
    return msg


def _check(status: int, what: str) -> None:
    """mlx.rs:459-470: success clears a stale message; failure carries it."""
    if status == 0:
        _take_last_error()
        return
    msg = _take_last_error()
    if msg:
        raise Error(f"sdq: {what}: {msg}")
    raise Error(f"sdq: {what} failed with status {status}")


def _none_int() -> COptionalInt:
    return COptionalInt(0, False)


def _some_int(v: int | None) -> COptionalInt:
    return COptionalInt(0, False) if v is None else COptionalInt(int(v), True)


# ---- bf16 helpers (host side, for building inputs and reading results) ------


def f32_to_bf16_bits(a) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- streams --------------------------------------------------------------------


class Stream:
    """The stream ops are submitted to (mlx.rs:472-510)."""

    def __init__(self, raw: CStream):
        self._raw = raw

    @classmethod
    def gpu(cls) -> "Stream":
        return cls(lib().sdq_default_gpu_stream_new())

    @classmethod
    def cpu(cls) -> "Stream":
        return cls(lib().sdq_default_cpu_stream_new())

    @classmethod
    def new(cls) -> "Stream":
        raw = lib().sdq_gpu_stream_new()
        if not raw.ctx:
            _check(1, "gpu_stream_new")
        return cls(raw)

    @classmethod
    def for_device(cls, device: str) -> "Stream":
        d = device.lower()
        if d in ("gpu", "hip", "rocm"):
            return cls.gpu()
        if d == "cpu":
            return cls.cpu()
        raise Error(f"unknown device {device!r}; try `gpu` or `cpu`")

    def synchronize(self) -> None:
        _check(lib().sdq_synchronize(self._raw), "synchronize")

    @property
    def native(self) -> int:
        """The hipStream_t address (0 for the CPU stream)."""
        return lib().sdq_stream_native(self._raw) or 0

    def __del__(self):
        if getattr(self, "_raw", None) is not None and _lib is not None:
            _lib.sdq_stream_free(self._raw)
            self._raw = None


# ---- arrays ------------------------------------------------------------------------


class Array:
    """A device array (mlx.rs:558-612).  Holds one reference; freed on drop."""

    def __init__(self, raw: CArray):
        if not raw.ctx:
            raise Error("sdq: operation returned a null array")
        self._raw = raw

    # construction -------------------------------------------------------------
    @classmethod
    def from_numpy(cls, a: np.ndarray, dtype: int | None = None) -> "Array":
        """Copy a host array to the device.  dtype BFLOAT16 takes either raw
        uint16 bit patterns or floats, which are rounded to nearest even."""
        a = np.asarray(a)
        if dtype is None:
            for code, t in ((FLOAT32, np.float32), (FLOAT16, np.float16), (UINT32, np.uint32),
                            (INT32, np.int32)):
                if a.dtype == t:
                    dtype = code
                    break
            else:
                raise Error(f"sdq: no device dtype for numpy {a.dtype}; pass dtype=")
        if dtype == BFLOAT16 and a.dtype != np.uint16:
            a = f32_to_bf16_bits(a.astype(np.float32)).reshape(a.shape)
        host = np.ascontiguousarray(a, dtype=_NP_OF[dtype])
        shape = (ctypes.c_int * max(1, host.ndim))(*host.shape)
        raw = lib().sdq_array_new_data(host.ctypes.data_as(ctypes.c_void_p), shape, host.ndim, dtype)
        if not raw.ctx:
            _check(1, "array_new_data")
        return cls(raw)

    @classmethod
    def from_slice_f32(cls, data: Sequence[float] | np.ndarray, shape: Sequence[int]) -> "Array":
        """mlx.rs:582-599: copies; the element count must match the shape."""
        v = np.asarray(data, dtype=np.float32).reshape(-1)
        n = int(np.prod(shape)) if len(shape) else 1
        if n != v.size:
            raise Error(f"sdq: shape {list(shape)} needs {n} elements, got {v.size}")
        return cls.from_numpy(v.reshape(shape), FLOAT32)

    # inspection ----------------------------------------------------------------
    @property
    def shape(self) -> list[int]:
        L = lib()
        nd = L.sdq_array_ndim(self._raw)
        ptr = L.sdq_array_shape(self._raw)
        if nd == 0 or not ptr:
            return []
        return [ptr[i] for i in range(nd)]

    @property
    def dtype(self) -> int:
        return lib().sdq_array_dtype(self._raw)

    def elem_count(self) -> int:
        return lib().sdq_array_size(self._raw)

    @property
    def nbytes(self) -> int:
        return lib().sdq_array_nbytes(self._raw)

    def is_f32(self) -> bool:
        return self.dtype == FLOAT32

    @property
    def device_ptr(self) -> int:
        """Device address of the data (for the raw entry points)."""
        return lib().sdq_array_device_ptr(self._raw) or 0

    def eval(self) -> None:
        _check(lib().sdq_array_eval(self._raw), "eval")

    def to_numpy(self) -> np.ndarray:
        """Synchronise and copy out.  bf16 comes back as raw uint16 bits."""
        out = np.empty(self.shape, dtype=_NP_OF[self.dtype])
        _check(
            lib().sdq_array_copy_to_host(out.ctypes.data_as(ctypes.c_void_p), out.nbytes, self._raw),
            "array_copy_to_host",
        )
        return out

    def to_float32(self) -> np.ndarray:
        """The values widened to f32 on the host (exact for bf16/f16)."""
        a = self.to_numpy()
        if self.dtype == BFLOAT16:
            return bf16_bits_to_f32(a)
        return a.astype(np.float32)

    def to_vec_f32(self, stream: Stream | None = None) -> list[float]:
        """mlx.rs:1426-1445: contiguous, eval, then the f32 contents; refuses
        arrays that are not f32."""
        src = self.contiguous(stream) if stream is not None else self
        src.eval()
        if not src.is_f32():
            raise Error("sdq: to_vec_f32 on an array that is not f32; cast with astype first")
        L = lib()
        ptr = L.sdq_array_data_float32(src._raw)
        if not ptr:
            _check(1, "array_data_float32")
        n = src.elem_count()
        return np.ctypeslib.as_array(ptr, shape=(n,)).copy().tolist()

    # ops -------------------------------------------------------------------------
    def _unary(self, fn: str, what: str, stream: Stream, *extra) -> "Array":
        res = CArray(None)
        _check(getattr(lib(), fn)(ctypes.byref(res), self._raw, *extra, stream._raw), what)
        return Array(res)

    def _binary(self, fn: str, what: str, other: "Array", stream: Stream) -> "Array":
        res = CArray(None)
        _check(getattr(lib(), fn)(ctypes.byref(res), self._raw, other._raw, stream._raw), what)
        return Array(res)

    def astype(self, dtype: int, stream: Stream) -> "Array":
        return self._unary("sdq_astype", "astype", stream, dtype)

    def contiguous(self, stream: Stream) -> "Array":
        return self._unary("sdq_contiguous", "contiguous", stream, False)

    def add(self, rhs: "Array", stream: Stream) -> "Array":
        return self._binary("sdq_add", "add", rhs, stream)

    def mul(self, rhs: "Array", stream: Stream) -> "Array":
        return self._binary("sdq_multiply", "multiply", rhs, stream)

    def matmul_nt(self, w: "Array", stream: Stream) -> "Array":
        """self @ w.T, the dense linear of sd-models/src/mlx/mod.rs:181-189."""
        return self._binary("sdq_matmul_nt", "matmul", w, stream)

    def layer_norm(self, weight: "Array | None", bias: "Array | None", eps: float, stream: Stream) -> "Array":
        """Layer norm over the last axis (mlx.rs:1059-1085)."""
        out = CArray(None)
        _check(lib().sdq_fast_layer_norm(ctypes.byref(out), self._raw, _h(weight), _h(bias), eps, stream._raw),
               "layer_norm")
        return Array(out)

    def rms_norm(self, weight: "Array | None", eps: float, stream: Stream) -> "Array":
        """RMS norm over the last axis (mlx.rs:1095-1115)."""
        out = CArray(None)
        _check(lib().sdq_fast_rms_norm(ctypes.byref(out), self._raw, _h(weight), eps, stream._raw), "rms_norm")
        return Array(out)

    def _sdpa(self, keys: "Array", values: "Array", scale: float, mode: bytes, mask: "Array | None",
              stream: Stream, what: str) -> "Array":
        out = CArray(None)
        _check(lib().sdq_fast_scaled_dot_product_attention(ctypes.byref(out), self._raw, keys._raw, values._raw,
                                                           scale, mode, _h(mask), CArray(None), stream._raw), what)
        return Array(out)

    def sdpa(self, keys: "Array", values: "Array", scale: float, stream: Stream) -> "Array":
        """Unmasked attention over [batch, heads, seq, head_dim] (mlx.rs:1161-1163)."""
        return self._sdpa(keys, values, scale, b"", None, stream, "sdpa")

    def sdpa_causal(self, keys: "Array", values: "Array", scale: float, stream: Stream) -> "Array":
        """Causal attention, CLIP's text tower (mlx.rs:1151-1159)."""
        return self._sdpa(keys, values, scale, b"causal", None, stream, "sdpa_causal")

    def sdpa_masked(self, keys: "Array", values: "Array", scale: float, mask: "Array", stream: Stream) -> "Array":
        """Attention with an additive mask, T5's position bias (mlx.rs:1119-1148)."""
        return self._sdpa(keys, values, scale, b"array", mask, stream, "sdpa_masked")

    def gelu_approx(self, stream: Stream) -> "Array":
        return self._unary("sdq_gelu_approx", "gelu_approx", stream)

    def __repr__(self) -> str:
        return f"sdq::Array{self.shape} {_NAMES.get(self.dtype, self.dtype)}"

    def __del__(self):
        if getattr(self, "_raw", None) is not None and _lib is not None:
            _lib.sdq_array_free(self._raw)
            self._raw = None


def eval(arrays: Iterable[Array]) -> None:  # noqa: A001 - mirrors mlx.rs:1535
    """Evaluate `arrays` (mlx.rs:1531-1544): wait for the work producing each."""
    L = lib()
    for a in arrays:
        vec = L.sdq_vector_array_new_value(a._raw)
        try:
            _check(L.sdq_eval(vec), "eval")
        finally:
            L.sdq_vector_array_free(vec)


# ---- the quantized weight ------------------------------------------------------


class QuantizedArray:
    """A weight held quantized at rest (mlx.rs:1834-1985): packed uint32 codes,
    per-group scales and biases, and the group size and bit width that no
    tensor records."""

    QUANT_MODE = b"affine"  # mlx.rs:1830-1832

    def __init__(self, weight: Array, scales: Array, biases: Array, group_size: int, bits: int):
        self.weight = weight
        self.scales = scales
        self.biases = biases
        self.group_size = group_size
        self.bits = bits

    @classmethod
    def quantize(cls, w: Array, group_size: int, bits: int, stream: Stream) -> "QuantizedArray":
        """[out, in] in, packed [out, in*bits/32] out (mlx.rs:1856-1911)."""
        L = lib()
        out = CVectorArray(None)
        _check(
            L.sdq_quantize(ctypes.byref(out), w._raw, _some_int(group_size), _some_int(bits),
                           cls.QUANT_MODE, CArray(None), stream._raw),
            "quantize",
        )
        return cls._from_vector(out, "quantize", group_size, bits)

    @classmethod
    def _from_vector(cls, out: CVectorArray, what: str, group_size: int, bits: int) -> "QuantizedArray":
        """Takes the three arrays of a quantize result (mlx.rs:1884-1898)."""
        L = lib()
        try:
            n = L.sdq_vector_array_size(out)
            if n != 3:
                raise Error(f"sdq: {what} returned {n} arrays, expected weight, scales and biases")
            parts = []
            for i in range(3):
                a = CArray(None)
                _check(L.sdq_vector_array_get(ctypes.byref(a), out, i), f"{what} output {i}")
                parts.append(Array(a))
        finally:
            L.sdq_vector_array_free(out)
        return cls(parts[0], parts[1], parts[2], group_size, bits)

    @classmethod
    def from_gguf_blocks(cls, raw, ggml_type: int, shape: Sequence[int], group_size: int, bits: int,
                         stream: Stream) -> "QuantizedArray":
        """A GGUF tensor's raw blocks decoded and quantized on the device in one
        kernel: equal to quantize(gguf_dequantize(raw)) -- the loader's
        dequantize -> from_slice_f32 -> quantize (quantized.rs:190-196)."""
        L = lib()
        ra = _raw_bytes(raw)
        dims = (ctypes.c_int * max(1, len(shape)))(*[int(d) for d in shape])
        out = CVectorArray(None)
        _check(
            L.sdq_gguf_quantize(ctypes.byref(out), ra._raw, int(ggml_type), dims, len(shape),
                                _some_int(group_size), _some_int(bits), stream._raw),
            "gguf_quantize",
        )
        return cls._from_vector(out, "gguf_quantize", group_size, bits)

    def dequantize(self, stream: Stream, dtype: int | None = None) -> Array:
        """The dense array (mlx.rs:1913-1945) -- for tests, not the hot path."""
        res = CArray(None)
        od = COptionalDtype(0, False) if dtype is None else COptionalDtype(int(dtype), True)
        _check(
            lib().sdq_dequantize(ctypes.byref(res), self.weight._raw, self.scales._raw,
                                 self.biases._raw, _some_int(self.group_size),
                                 _some_int(self.bits), self.QUANT_MODE, CArray(None), od,
                                 stream._raw),
            "dequantize",
        )
        return Array(res)

    def matmul(self, x: Array, stream: Stream) -> Array:
        """x @ weight.T, dequantizing inside the kernel (mlx.rs:1947-1975)."""
        res = CArray(None)
        _check(
            lib().sdq_quantized_matmul(ctypes.byref(res), x._raw, self.weight._raw,
                                       self.scales._raw, self.biases._raw, True,
                                       _some_int(self.group_size), _some_int(self.bits),
                                       self.QUANT_MODE, stream._raw),
            "quantized_matmul",
        )
        return Array(res)

    def linear(self, x: Array, stream: Stream, bias: Array | None = None,
               activation: int = 0) -> Array:
        """act(x @ weight.T + bias) in one launch: quantized::linear's
        quantized branch with its bias add (quantized.rs:293-318) and an
        optional activation (ACT_GELU_APPROX, the Flux MLP's GELU,
        flux.rs:400-413), applied to the f32 accumulator before the output's
        one rounding."""
        res = CArray(None)
        _check(
            lib().sdq_quantized_linear(ctypes.byref(res), x._raw, self.weight._raw,
                                       self.scales._raw, self.biases._raw,
                                       bias._raw if bias is not None else CArray(None),
                                       int(activation), _some_int(self.group_size),
                                       _some_int(self.bits), self.QUANT_MODE, stream._raw),
            "quantized_linear",
        )
        return Array(res)

    def linear_combine(self, x: Array, stream: Stream, residual: Array, combine: int,
                       bias: Array | None = None, activation: int = 0,
                       gate: Array | None = None) -> Array:
        """`linear` followed by COMBINE_GATED_RESIDUAL (residual + gate * y,
        Flux's gated residual, flux.rs:389-398) or COMBINE_PRODUCT (y *
        residual, T5's gelu(wi_0 x) * (wi_1 x), t5.rs:209-214), one launch."""
        res = CArray(None)
        _check(
            lib().sdq_quantized_linear_combine(
                ctypes.byref(res), x._raw, self.weight._raw, self.scales._raw, self.biases._raw,
                bias._raw if bias is not None else CArray(None), int(activation), residual._raw,
                gate._raw if gate is not None else CArray(None), int(combine),
                _some_int(self.group_size), _some_int(self.bits), self.QUANT_MODE, stream._raw),
            "quantized_linear_combine",
        )
        return Array(res)

    @classmethod
    def pair(cls, gate: "QuantizedArray", up: "QuantizedArray", stream: Stream) -> "QuantizedArray":
        """The operand of `linear_gated`: gate's and up's rows interleaved in
        blocks of eight (packed weights, scales and biases alike), built once
        at load time from T5's wi_0 and wi_1 (t5.rs:209-214)."""
        if (gate.group_size, gate.bits) != (up.group_size, up.bits):
            raise Error("pair: gate and up must share group size and bits")
        return cls(pair_rows(gate.weight, up.weight, stream), pair_rows(gate.scales, up.scales, stream),
                   pair_rows(gate.biases, up.biases, stream), gate.group_size, gate.bits)

    def linear_gated(self, x: Array, stream: Stream, bias: Array | None = None,
                     activation: int = ACT_GELU_APPROX) -> Array:
        """act(x @ gate.T + bias_g) * (x @ up.T + bias_u) in one launch, this
        array being a `pair`: T5's gelu_new(wi_0 x) * (wi_1 x)
        (t5.rs:201-214).  bias: the two biases through `pair_rows`."""
        res = CArray(None)
        _check(
            lib().sdq_quantized_linear_gated(ctypes.byref(res), x._raw, self.weight._raw,
                                             self.scales._raw, self.biases._raw, _h(bias),
                                             int(activation), _some_int(self.group_size),
                                             _some_int(self.bits), self.QUANT_MODE, stream._raw),
            "quantized_linear_gated",
        )
        return Array(res)

    def resident_bytes(self) -> int:
        """Packed words at 4 bytes plus scales and biases at 4 bytes each, the
        reference's accounting (mlx.rs:1977-1985)."""
        packed = self.weight.elem_count() * 4
        scales = (self.scales.elem_count() + self.biases.elem_count()) * 4
        return packed + scales


# ---- memory accounting (mlx.rs:1732-1826) ---------------------------------------


def _h(a: "Array | None") -> CArray:
    """An optional array argument: the handle, or an empty one."""
    return CArray(None) if a is None else a._raw


def pair_rows(gate: Array, up: Array, stream: Stream) -> Array:
    """Rows of two equal-shaped arrays interleaved in blocks of eight (gate's
    block b at rows 16 b.., up's at 16 b + 8..): the layout `linear_gated`
    reads."""
    res = CArray(None)
    _check(lib().sdq_pair_rows(ctypes.byref(res), gate._raw, up._raw, stream._raw), "pair_rows")
    return Array(res)


def _raw_bytes(raw) -> Array:
    """A GGUF tensor's bytes as a device uint8 array (an Array passes through)."""
    if isinstance(raw, Array):
        return raw
    host = np.frombuffer(raw, dtype=np.uint8) if isinstance(raw, (bytes, bytearray, memoryview)) \
        else np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
    return Array.from_numpy(host, UINT8)


def gguf_dequantize(raw, ggml_type: int, shape: Sequence[int], stream: Stream) -> Array:
    """A GGUF tensor's raw blocks decoded to a float32 device array, as
    Gguf::dequantize + Array::from_slice_f32 (mlx_gguf.rs:235-276,
    quantized.rs:190-191)."""
    L = lib()
    ra = _raw_bytes(raw)
    dims = (ctypes.c_int * max(1, len(shape)))(*[int(d) for d in shape])
    out = CArray(None)
    _check(L.sdq_gguf_dequantize(ctypes.byref(out), ra._raw, int(ggml_type), dims, len(shape), stream._raw),
           "gguf_dequantize")
    return Array(out)


def _size_query(fn: str) -> int:
    v = ctypes.c_size_t(0)
    _check(getattr(lib(), fn)(ctypes.byref(v)), fn[4:])
    return v.value


def active_memory() -> int:
    return _size_query("sdq_get_active_memory")


def peak_memory() -> int:
    return _size_query("sdq_get_peak_memory")


def cache_memory() -> int:
    return _size_query("sdq_get_cache_memory")


def reset_peak_memory() -> None:
    _check(lib().sdq_reset_peak_memory(), "reset_peak_memory")


def clear_cache() -> None:
    _check(lib().sdq_clear_cache(), "clear_cache")


def device_count() -> int:
    return lib().sdq_device_count()


def version() -> str:
    return lib().sdq_version().decode()


# The policy layer (quantized.rs) builds on the classes above.
from . import quantized  # noqa: E402,F401
