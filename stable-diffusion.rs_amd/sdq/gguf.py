"""GGUF container reader for the quantized loader (crates/sd-tensor/src/mlx_gguf.rs).

The reference parses the container on the host and decodes every block on the
host too (mlx_gguf.rs:235-276).  Here the host parses only the directory; a
tensor's bytes go to the device as the file stores them and the libsdq
kernels decode them there (`sdq_gguf_dequantize`), or decode and quantize them
in one pass (`sdq_gguf_quantize`, used by quantized.from_gguf).

Format, as the reference reads it:
    magic "GGUF" (u32 0x46554747), version 2 or 3, tensor count u64,
    metadata count u64, metadata (key string, type u32, value; skipped),
    per tensor: name string, n_dims u32, dims u64 (fastest-varying first),
    type u32, offset u64; tensor data from the next 32-byte boundary.
Strings are a u64 length then UTF-8 bytes; everything is little-endian.
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import BinaryIO, Dict, List, Tuple

from . import Array, Error, QuantizedArray, Stream, gguf_dequantize

MAGIC = 0x46554747  # "GGUF", mlx_gguf.rs:25
ALIGN = 32          # mlx_gguf.rs:219-225

# GGML type ids (mlx_gguf.rs:61-79) -> (name, values per block, bytes per block)
# (mlx_gguf.rs:27-40, 81-92).
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 8, 12, 13, 14, 30
TYPES: Dict[int, Tuple[str, int, int]] = {
    F32: ("F32", 1, 4),
    F16: ("F16", 1, 2),
    BF16: ("BF16", 1, 2),
    Q4_0: ("Q4_0", 32, 18),
    Q8_0: ("Q8_0", 32, 34),
    Q4_K: ("Q4_K", 256, 144),
    Q5_K: ("Q5_K", 256, 176),
    Q6_K: ("Q6_K", 256, 210),
}


def block(kind: int) -> Tuple[int, int]:
    """(values per block, bytes per block) of a GGML type (mlx_gguf.rs:81-92)."""
    return TYPES[kind][1], TYPES[kind][2]


def _type_from_id(i: int) -> int:
    if i not in TYPES:
        raise Error(
            f"gguf: type {i} is not one this project's checkpoints use; "
            "the supported set is F32, F16, BF16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K"
        )
    return i


@dataclass
class TensorInfo:
    """One directory entry (mlx_gguf.rs:96-112).  `shape` is row-major: the
    file's dimensions reversed once at parse (mlx_gguf.rs:205-208)."""

    name: str
    shape: List[int]
    kind: int
    offset: int

    def elem_count(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n


class _Reader:
    def __init__(self, f: BinaryIO):
        self.f = f

    def _exact(self, n: int) -> bytes:
        b = self.f.read(n)
        if len(b) != n:
            raise Error("gguf: failed to fill whole buffer")
        return b

    def u32(self) -> int:
        return struct.unpack("<I", self._exact(4))[0]

    def u64(self) -> int:
        return struct.unpack("<Q", self._exact(8))[0]

    def string(self) -> str:
        n = self.u64()
        try:
            return self._exact(n).decode("utf-8")
        except UnicodeDecodeError as e:
            raise Error(f"gguf: bad utf8 in a name: {e}") from None

    def skip_value(self, kind: int) -> None:
        """mlx_gguf.rs:136-160: metadata is skipped, arrays element by element."""
        sizes = {0: 1, 1: 1, 7: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 10: 8, 11: 8, 12: 8}
        if kind in sizes:
            self.f.seek(sizes[kind], os.SEEK_CUR)
        elif kind == 8:
            self.f.seek(self.u64(), os.SEEK_CUR)
        elif kind == 9:
            inner = self.u32()
            for _ in range(self.u64()):
                self.skip_value(inner)
        else:
            raise Error(f"gguf: unknown metadata type {kind}")


class Gguf:
    """The tensor directory of a GGUF file and where its data starts
    (mlx_gguf.rs:166-231)."""

    def __init__(self, path: Path, f: BinaryIO, tensors: List[TensorInfo], data_start: int):
        self.path = path
        self._f = f
        self.tensors = tensors
        self.data_start = data_start

    @classmethod
    def open(cls, path) -> "Gguf":
        path = Path(path)
        try:
            f = open(path, "rb")
        except OSError as e:
            raise Error(f"gguf: {e}") from None
        r = _Reader(f)
        if r.u32() != MAGIC:
            f.close()
            raise Error(f"gguf: {path} is not a GGUF file")
        version = r.u32()
        if not 2 <= version <= 3:
            f.close()
            raise Error(f"gguf: version {version} is not supported")
        tensor_count = r.u64()
        kv_count = r.u64()
        for _ in range(kv_count):
            r.string()
            r.skip_value(r.u32())
        tensors = []
        for _ in range(tensor_count):
            name = r.string()
            n_dims = r.u32()
            shape = [r.u64() for _ in range(n_dims)]
            shape.reverse()
            kind = _type_from_id(r.u32())
            offset = r.u64()
            tensors.append(TensorInfo(name, shape, kind, offset))
        here = f.tell()
        data_start = (here + ALIGN - 1) // ALIGN * ALIGN
        return cls(path, f, tensors, data_start)

    def close(self) -> None:
        self._f.close()

    def __enter__(self) -> "Gguf":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def raw(self, info: TensorInfo) -> bytes:
        """The tensor's bytes as stored (mlx_gguf.rs:236-250)."""
        n = info.elem_count()
        per, nbytes = block(info.kind)
        if n % per != 0:
            raise Error(f"gguf: {info.name} has {n} elements, not a multiple of {per}")
        self._f.seek(self.data_start + info.offset)
        b = self._f.read(n // per * nbytes)
        if len(b) != n // per * nbytes:
            raise Error("gguf: failed to fill whole buffer")
        return b

    def dequantize(self, info: TensorInfo, stream: Stream) -> Array:
        """One tensor as a float32 device array: Gguf::dequantize followed by
        Array::from_slice_f32 (mlx_gguf.rs:235-276, quantized.rs:190-191),
        with the block decoding on the device."""
        return gguf_dequantize(self.raw(info), info.kind, info.shape, stream)

    def quantize(self, info: TensorInfo, group_size: int, bits: int, stream: Stream) -> QuantizedArray:
        """One tensor decoded and quantized on the device in one kernel
        (quantized.rs:190-196 without the f32 round trip)."""
        return QuantizedArray.from_gguf_blocks(self.raw(info), info.kind, info.shape, group_size, bits, stream)


def load(path, stream: Stream) -> Dict[str, Array]:
    """Every tensor of a GGUF file as float32 device arrays, keyed by name
    (mlx_gguf.rs:444-455)."""
    with Gguf.open(path) as g:
        return {info.name: g.dequantize(info, stream) for info in g.tensors}
