"""The C ABI without a GPU: the library loads, exports every entry point
include/sdq.h declares, keeps mlx-c's struct layouts and error contract, and
refuses the CPU stream loudly instead of falling back to host code."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "sdq.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(sdq_[a-z0-9_]+)\s*\(", text)
    return sorted(set(n for n in names if not n.endswith("_func")))


def test_header_declares_the_path(sdq):
    names = declared_functions()
    for must in ("sdq_quantize", "sdq_dequantize", "sdq_quantized_matmul", "sdq_eval",
                 "sdq_set_error_handler", "sdq_array_new_data", "sdq_array_free",
                 "sdq_default_gpu_stream_new", "sdq_vector_array_get"):
        assert must in names


def test_library_exports_every_declared_symbol(sdq):
    L = ctypes.CDLL(str(sdq.LIB_PATH))
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert missing == []


def test_binding_declares_every_symbol(sdq):
    # The ctypes binding sets a signature for every C entry point.
    L = sdq.lib()
    for n in declared_functions():
        assert getattr(L, n).argtypes is not None, n


def test_struct_layouts_match_mlx_c(sdq):
    # mlx.rs:38-80: {void*} handles; optional int/dtype are an int then a bool.
    assert ctypes.sizeof(sdq.CArray) == ctypes.sizeof(ctypes.c_void_p)
    assert ctypes.sizeof(sdq.COptionalInt) == 8
    assert sdq.COptionalInt.has_value.offset == 4
    assert sdq.COptionalDtype.has_value.offset == 4


def test_dtype_positions_are_mlx_dtype_positions(sdq):
    # mlx.rs:100-104 hard-codes INT32 = 7, FLOAT16 = 9, FLOAT32 = 10.
    assert (sdq.INT32, sdq.FLOAT16, sdq.FLOAT32) == (7, 9, 10)
    text = HEADER.read_text()
    assert "SDQ_INT32 = 7" in text and "SDQ_FLOAT16 = 9" in text and "SDQ_FLOAT32 = 10" in text


def test_version_and_device_count(sdq):
    assert sdq.version().startswith("sdq ")
    assert "gfx950" in sdq.version()
    assert sdq.device_count() >= 0


def test_cpu_stream_is_refused_with_a_message(sdq):
    s = sdq.Stream.cpu()
    assert s.native == 0
    # Any op on it fails with the reason, through the error handler.
    L = sdq.lib()
    out = sdq.CVectorArray(None)
    rc = L.sdq_quantize(ctypes.byref(out), sdq.CArray(None), sdq.COptionalInt(64, True),
                        sdq.COptionalInt(4, True), b"affine", sdq.CArray(None), s._raw)
    assert rc != 0
    with pytest.raises(sdq.Error, match="no CPU backend"):
        sdq._check(rc if rc else 1, "quantize")
    assert out.ctx is None
    with pytest.raises(sdq.Error, match="no CPU backend"):
        s.synchronize()


def test_error_handler_receives_the_message_synchronously(sdq):
    L = sdq.lib()
    seen = []
    HANDLER = ctypes.CFUNCTYPE(None, ctypes.c_char_p, ctypes.c_void_p)

    @HANDLER
    def handler(msg, data):
        seen.append(msg.decode())

    try:
        L.sdq_set_error_handler(handler, None, None)
        rc = L.sdq_synchronize(L.sdq_default_cpu_stream_new())
        assert rc != 0
        assert seen and seen[-1].startswith("[synchronize]")
    finally:
        L.sdq_set_error_handler(sdq._error_handler, None, None)


def test_empty_handles_are_errors_not_crashes(sdq):
    L = sdq.lib()
    res = sdq.CArray(None)
    rc = L.sdq_astype(ctypes.byref(res), sdq.CArray(None), sdq.FLOAT32, L.sdq_default_cpu_stream_new())
    assert rc != 0
    sdq._take_last_error()
    assert L.sdq_array_size(sdq.CArray(None)) == 0
    assert L.sdq_array_ndim(sdq.CArray(None)) == 0
    assert L.sdq_vector_array_size(sdq.CVectorArray(None)) == 0
    assert L.sdq_array_free(sdq.CArray(None)) == 0


def test_raw_entry_point_validates_before_touching_the_gpu(sdq):
    L = sdq.lib()
    rc = L.sdq_quantized_matmul_raw(None, sdq.FLOAT32, None, sdq.BFLOAT16, 64, None, None, None,
                                    sdq.FLOAT32, 4, 8, 100, 64, 4, None)
    assert rc != 0
    with pytest.raises(sdq.Error):
        sdq._check(rc, "quantized_matmul_raw")
    rc = L.sdq_quantized_matmul_raw(None, sdq.FLOAT32, None, sdq.BFLOAT16, 64, None, None, None,
                                    sdq.FLOAT32, 4, 8, 64, 64, 3, None)
    assert rc != 0
    sdq._take_last_error()


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    # The binding has no fallback: without the .so every call raises.
    import importlib.util
    import sys

    spec = importlib.util.spec_from_file_location(
        "sdq_copy", REPO / "stable-diffusion.rs_amd" / "sdq" / "__init__.py",
        submodule_search_locations=[str(REPO / "stable-diffusion.rs_amd" / "sdq")])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["sdq_copy"] = mod
    try:
        spec.loader.exec_module(mod)
        mod.LIB_PATH = tmp_path / "libsdq.so"
        mod._lib = None
        with pytest.raises(mod.Error, match="not built"):
            mod.lib()
    finally:
        sys.modules.pop("sdq_copy", None)
