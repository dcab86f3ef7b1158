"""Build libsdq.so (the gfx950 HIP library behind include/sdq.h) in-tree.

    python stable-diffusion.rs_amd/build.py [--verbose]

Objects go to stable-diffusion.rs_amd/_build/, the library to
stable-diffusion.rs_amd/sdq/libsdq.so, next to the Python binding that loads
it.  Every source is compiled on each call (hipcc cross-compiles gfx950 code
without a GPU).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "sdq" / "libsdq.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    f"-I{REPO / 'include'}",
    f"-I{CSRC}",
    "-Wall",
    "-Wno-unused-function",
    # Packed FP32 arithmetic is kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

# Sources and their extra flags.  quant.hip must round every operation once
# (bit-exact quantize/dequantize), so contraction into FMA is off there.
SOURCES = [
    (CSRC / "sdq_runtime.cpp", []),
    (CSRC / "sdq_ops.cpp", []),
    (CSRC / "kernels" / "quant.hip", ["-ffp-contract=off"]),
    (CSRC / "kernels" / "elementwise.hip", []),
    (CSRC / "kernels" / "dense.hip", []),
    (CSRC / "kernels" / "qmv.hip", []),
    (CSRC / "kernels" / "qmm.hip", []),
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(str(c) for c in cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # The host pass does not know the GPU-only feature flag; that warning is noise.
    lines = [
        ln
        for ln in proc.stdout.splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in ln
    ]
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(map(str, cmd))}\n" + "\n".join(lines))
    if verbose and lines:
        print("\n".join(lines), flush=True)


def _compile(src: Path, extra: list[str], verbose: bool) -> Path:
    obj = BUILD / (src.stem + src.suffix.replace(".", "_") + ".o")
    cmd = [HIPCC, *COMMON, *extra, "-c", str(src), "-o", str(obj)]
    _run(cmd, verbose)
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, src, extra, verbose) for src, extra in SOURCES]
        objs = [f.result() for f in futs]
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, LIB)
    return LIB


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    lib = build(verbose=args.verbose)
    print(lib)
    return 0


if __name__ == "__main__":
    sys.exit(main())
