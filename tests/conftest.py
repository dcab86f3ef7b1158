"""Shared test setup.

Markers: `gpu` -- needs an MI355X (run on the GPU box with `-m gpu`).  GPU
tests call libsdq through its C ABI (include/sdq.h, via the ctypes binding in
stable-diffusion.rs_amd/sdq) and compare with the CPU oracle
(oracle/sdq_oracle.c) on the same seeded inputs.
"""
from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "stable-diffusion.rs_amd"
for p in (str(REPO), str(PKG), str(REPO / "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

HAS_GPU = os.path.exists("/dev/kfd")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X); run with -m gpu")


def pytest_collection_modifyitems(config, items):
    if HAS_GPU:
        return
    skip = pytest.mark.skip(reason="no AMD GPU in this container (/dev/kfd absent)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle():
    import sdq_oracle

    sdq_oracle.lib()
    return sdq_oracle


@pytest.fixture(scope="session")
def sdq():
    import sdq as mod

    mod.lib()  # raises if libsdq.so is not built: no silent fallback
    return mod


@pytest.fixture(scope="session")
def stream(sdq):
    s = sdq.Stream.gpu()
    yield s
    s.synchronize()


def cosine(a, b) -> float:
    """Accumulated in f64 (mlx_quantized.rs:41-49)."""
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def max_rel_err(got, want) -> float:
    """max |got - want| / max |want|: the BASELINE tolerance's definition."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def ramp_weight(out: int, inp: int) -> np.ndarray:
    """mlx_quantized.rs:27-32."""
    i = np.arange(out * inp)
    return (((i % 97).astype(np.float32) - 48.0) / 96.0).astype(np.float32).reshape(out, inp)


def ramp_activation(rows: int, inp: int) -> np.ndarray:
    """mlx_quantized.rs:34-39."""
    i = np.arange(rows * inp)
    return (((i % 31).astype(np.float32) - 15.0) / 15.0).astype(np.float32).reshape(rows, inp)
