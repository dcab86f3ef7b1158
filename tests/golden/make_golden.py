#!/usr/bin/env python3
"""Writes tests/golden/quantized_linear.npz: small input/output vectors of the
MLX-affine quantized linear, produced by the CPU oracle.

The reference holds no quantization fixtures (its tensor fixtures are git-
ignored and its quantization arithmetic lives in MLX, which is not vendored),
so these vectors are the oracle's own outputs, frozen: a later change to the
oracle or to the GPU kernels that moves a single bit shows up against them.
Inputs come from the reference's SeededRng (crates/sd-tensor/src/lib.rs:105-145)
with the seeds listed below, weights scaled by 0.02 as in
crates/sd-models/tests/mlx_quantized.rs:29-33.

Run:  python tests/golden/make_golden.py   (rewrites the .npz in place)
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent / "oracle"))

import sdq_oracle as oracle  # noqa: E402

OUT = HERE / "quantized_linear.npz"

ROWS, COLS = 6, 256          # weight [N, K]
M = 5                        # activation rows
STORE = {"f32": oracle.FLOAT32, "bf16": oracle.BFLOAT16, "f16": oracle.FLOAT16}


def values(a: np.ndarray, store: int) -> np.ndarray:
    """Stored scales/biases (f32, or raw uint16 bits) as f32 values."""
    if store == oracle.BFLOAT16:
        return (a.astype(np.uint32) << 16).view(np.float32)
    if store == oracle.FLOAT16:
        return a.view(np.float16).astype(np.float32)
    return a


def widen(w: np.ndarray, store: int) -> np.ndarray:
    """Weights as the device holds them in `store`, widened back to f32."""
    if store == oracle.BFLOAT16:
        return np.array([oracle.f32_from_bf16(oracle.bf16_from_f32(float(v))) for v in w.ravel()],
                        dtype=np.float32).reshape(w.shape)
    if store == oracle.FLOAT16:
        return w.astype(np.float16).astype(np.float32)
    return w


def make() -> dict:
    out = {}
    rng = oracle.Rng(1234567)
    out["rng_seed1234567_u64"] = np.array([rng.next_u64() for _ in range(8)], dtype=np.uint64)
    out["rng_seed42_normals"] = oracle.normals(42, 16)

    w = oracle.normals(7001, ROWS * COLS, 0.02).reshape(ROWS, COLS)
    x = oracle.normals(7002, M * COLS, 1.0).reshape(M, COLS)
    out["w"] = w
    out["x"] = x
    for sname, store in STORE.items():
        ws = widen(w, store)
        out[f"w_{sname}"] = ws
        for bits in (2, 4, 8):
            for gs in (32, 64, 128):
                key = f"{sname}_b{bits}_g{gs}"
                wq, s, b = oracle.quantize(ws, gs, bits, store)
                out[f"wq_{key}"] = wq
                out[f"scales_{key}"] = s
                out[f"biases_{key}"] = b
                out[f"deq_{key}"] = oracle.dequantize(wq, s, b, gs, bits, store)
                out[f"y_{key}"] = oracle.qmatmul(x, wq, values(s, store), values(b, store), gs, bits)
    return out


def main() -> int:
    data = make()
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(data)} arrays)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
