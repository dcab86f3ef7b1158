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

# dtype codes (include/sdq.h) of the (activation, scales, output) combinations
# the matmul kernels are instantiated for; qmm.hip / qmv.hip dispatch over the
# same list, and a combination missing here is a link error.
F16, F32, BF16 = 9, 10, 12
MATMUL_COMBOS = [
    (BF16, F32, F32), (BF16, BF16, BF16), (F32, F32, F32), (BF16, F32, BF16), (F16, F16, F16),
    (F16, F32, F32), (F32, BF16, F32), (F32, F16, F32), (BF16, F16, F32), (F16, BF16, F32),
]


def _combo_flags(c):
    return [f"-DSDQ_XD={c[0]}", f"-DSDQ_SD={c[1]}", f"-DSDQ_OD={c[2]}"]


# Sources, their extra flags and object names.  quant.hip and gguf.hip must
# round every operation once (bit-exact quantize/dequantize and GGUF
# decoding), so contraction into FMA is off there.  The matmul kernels' instantiation units are compiled once per
# dtype combination.
SOURCES = [
    (CSRC / "sdq_runtime.cpp", [], None),
    (CSRC / "sdq_ops.cpp", [], None),
    (CSRC / "sdq_ops_block.cpp", [], None),
    (CSRC / "sdq_noalloc.hip", [], None),
    (CSRC / "kernels" / "quant.hip", ["-ffp-contract=off"], None),
    (CSRC / "kernels" / "gguf.hip", ["-ffp-contract=off"], None),
    (CSRC / "kernels" / "elementwise.hip", [], None),
    (CSRC / "kernels" / "dense.hip", [], None),
    (CSRC / "kernels" / "attention.hip", [], None),
    (CSRC / "kernels" / "norm.hip", ["-ffp-contract=off"], None),
    (CSRC / "kernels" / "qmv.hip", [], None),
    (CSRC / "kernels" / "qmm.hip", [], None),
] + [
    (CSRC / "kernels" / f"{k}_inst.hip", _combo_flags(c), f"{k}_inst_{c[0]}_{c[1]}_{c[2]}")
    for k in ("qmm", "qmv")
    for c in MATMUL_COMBOS
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


def _compile(src: Path, extra: list[str], name: str | None, verbose: bool) -> Path:
    obj = _obj(src, name)
    cmd = [HIPCC, *COMMON, *extra, "-c", str(src), "-o", str(obj)]
    _run(cmd, verbose)
    return obj


def _obj(src: Path, name: str | None) -> Path:
    return BUILD / ((name or src.stem + src.suffix.replace(".", "_")) + ".o")


def build(verbose: bool = False, jobs: int | None = None, only: list[str] | None = None) -> Path:
    """Compile every source (or, with `only`, the sources whose file names
    start with one of the given prefixes, reusing the other objects from an
    earlier full build) and link the library."""
    BUILD.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4, 16)
    # Longest compiles first, so the pool's tail is short.
    order = sorted(SOURCES, key=lambda s: 0 if s[0].name.startswith(("qmm", "qmv")) else 1)
    # A partial build also recompiles every object older than the newest
    # header: a changed struct seen two ways by two objects breaks at run time.
    newest_header = max(p.stat().st_mtime for p in [*CSRC.rglob("*.hpp"), REPO / "include" / "sdq.h"])

    def stale(src: Path, name: str | None) -> bool:
        obj = _obj(src, name)
        return not obj.exists() or obj.stat().st_mtime < newest_header

    todo = [s for s in order if only is None or s[0].name.startswith(tuple(only)) or stale(s[0], s[2])]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, src, extra, name, verbose) for src, extra, name in todo]
        for f in futs:
            f.result()
    objs = [_obj(src, name) for src, _, name in order]
    missing = [o.name for o in objs if not o.exists()]
    if missing:
        raise RuntimeError(f"objects missing (run a full build first): {', '.join(missing)}")
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, LIB)
    return LIB


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--only", nargs="+", metavar="PREFIX",
                    help="recompile only sources whose file name starts with PREFIX (others from the last build)")
    args = ap.parse_args()
    lib = build(verbose=args.verbose, only=args.only)
    print(lib)
    return 0


if __name__ == "__main__":
    sys.exit(main())
