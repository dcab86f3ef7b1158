"""The GGUF directory reader (sdq/gguf.py), mirroring mlx_gguf.rs:166-276, on
files written by tests/gguf_blocks.py.  Host logic only: no GPU needed."""
from __future__ import annotations

import struct

import numpy as np
import pytest

import gguf_blocks as gb

METADATA = [
    ("general.architecture", 8, "flux"),
    ("general.alignment", 4, 32),
    ("u8", 0, 7), ("i8", 1, -3), ("u16", 2, 9), ("i16", 3, -9), ("i32", 5, -1), ("f32", 6, 0.5),
    ("bool", 7, True), ("u64", 10, 1 << 40), ("i64", 11, -(1 << 40)), ("f64", 12, 2.5),
    ("tokens", 9, (8, ["a", "bc", ""])),
    ("nested", 9, (9, [(4, [1, 2]), (4, [3])])),
]


def _tensors(rng):
    return [
        ("double_blocks.0.img_mlp.0.weight", [64, 256], gb.Q4_K, gb.random_tensor(gb.Q4_K, 64 * 256, rng)),
        ("img_in.weight", [32, 64], gb.Q8_0, gb.random_tensor(gb.Q8_0, 32 * 64, rng)),
        ("final_layer.norm.bias", [3], gb.F32, gb.random_tensor(gb.F32, 3, rng)),
        ("txt_in.weight", [16, 128], gb.F16, gb.random_tensor(gb.F16, 16 * 128, rng)),
    ]


def test_directory_shapes_offsets_and_bytes(tmp_path):
    from sdq.gguf import Gguf

    rng = np.random.default_rng(1)
    ts = _tensors(rng)
    p = tmp_path / "m.gguf"
    gb.write_gguf(p, ts, METADATA)
    with Gguf.open(p) as g:
        assert [t.name for t in g.tensors] == [t[0] for t in ts]
        assert [t.shape for t in g.tensors] == [t[1] for t in ts]  # reversed back to row-major
        assert [t.kind for t in g.tensors] == [t[2] for t in ts]
        assert g.data_start % 32 == 0
        for info, (_, _, _, raw) in zip(g.tensors, ts):
            assert g.raw(info) == raw
            assert info.offset % 32 == 0


def test_version_2_reads_and_other_versions_do_not(tmp_path):
    from sdq import Error
    from sdq.gguf import Gguf

    rng = np.random.default_rng(2)
    gb.write_gguf(tmp_path / "v2.gguf", _tensors(rng)[:1], version=2)
    with Gguf.open(tmp_path / "v2.gguf") as g:
        assert len(g.tensors) == 1
    gb.write_gguf(tmp_path / "v4.gguf", _tensors(rng)[:1], version=4)
    with pytest.raises(Error, match="version 4 is not supported"):
        Gguf.open(tmp_path / "v4.gguf")


def test_not_a_gguf_file(tmp_path):
    from sdq import Error
    from sdq.gguf import Gguf

    p = tmp_path / "x.bin"
    p.write_bytes(b"GGML" + bytes(60))
    with pytest.raises(Error, match="is not a GGUF file"):
        Gguf.open(p)
    with pytest.raises(Error, match="gguf:"):
        Gguf.open(tmp_path / "missing.gguf")


def test_unsupported_type_is_named(tmp_path):
    from sdq import Error
    from sdq.gguf import Gguf

    p = tmp_path / "q41.gguf"
    gb.write_gguf(p, [("w", [32], 3, bytes(20))])  # 3 = Q4_1
    with pytest.raises(Error, match="type 3 is not one this project's checkpoints use"):
        Gguf.open(p)


def test_unknown_metadata_type_and_truncation(tmp_path):
    from sdq import Error
    from sdq.gguf import Gguf

    p = tmp_path / "kv.gguf"
    head = struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13)
    p.write_bytes(head)
    with pytest.raises(Error, match="unknown metadata type 13"):
        Gguf.open(p)
    p.write_bytes(struct.pack("<IIQ", 0x46554747, 3, 5))
    with pytest.raises(Error, match="failed to fill"):
        Gguf.open(p)


def test_element_count_not_a_block_multiple(tmp_path):
    from sdq import Error
    from sdq.gguf import Gguf

    p = tmp_path / "odd.gguf"
    gb.write_gguf(p, [("w", [3, 10], gb.Q4_0, bytes(18))])
    with Gguf.open(p) as g:
        with pytest.raises(Error, match="w has 30 elements, not a multiple of 32"):
            g.raw(g.tensors[0])
