"""bench.py's measurement arithmetic and command line, on the CPU (no GPU
call): the algorithmic bytes and the roofline choice follow the formulas
they state, the committed traffic summary parses, and a multi-GPU request is
refused with a message before anything touches a device."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO))

import bench  # noqa: E402


def test_algorithmic_bytes_closed_form():
    # 4-bit 3072 -> 12288 at M = 1: packed codes (K/2 bytes a row), f32 scale
    # and bias per 64-group, bf16 x and y.
    M, N, K = 1, 12288, 3072
    want = N * K // 2 + 2 * N * (K // 64) * 4 + M * K * 2 + M * N * 2
    assert bench.algorithmic_bytes(M, N, K, 4) == want
    # 8-bit doubles the code bytes only.
    assert bench.algorithmic_bytes(M, N, K, 8) - bench.algorithmic_bytes(M, N, K, 4) == N * K // 2


def test_roofline_side_follows_the_ridge():
    # Arithmetic intensity 2MNK / bytes: the small-M point is HBM-bound, the
    # prefill point MFMA-bound, with the fraction taken against that peak.
    lo = bench.roofline_point(1, 12288, 3072, 4, 0.010)
    hi = bench.roofline_point(4608, 12288, 3072, 4, 0.330)
    assert lo["bound"] == "hbm" and hi["bound"] == "mfma"
    assert lo["frac"] == pytest.approx(lo["GB/s"] / bench.PEAK_HBM_GBS, rel=1e-3)
    assert hi["frac"] == pytest.approx(hi["TFLOP/s"] / bench.PEAK_BF16_TFLOPS, rel=1e-3)
    assert hi["TFLOP/s"] == pytest.approx(2 * 4608 * 12288 * 3072 / 0.330e-3 / 1e12, rel=1e-3)


def test_committed_traffic_summary_parses():
    if not bench.TRAFFIC_FILE.exists():
        pytest.skip("no traffic summary committed")
    for label in ("fc1", "fc2"):
        traffic, kernel = bench.measured_traffic(label)
        assert traffic and traffic > bench.algorithmic_bytes(1536, 12288, 3072, 4) // 2
        assert kernel and "qmm_kernel" in kernel


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stderr
