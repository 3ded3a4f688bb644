"""Ahead-of-time build of libcc1d_amd.so for gfx950.

Each ``*.hip`` translation unit in this directory is compiled to an object
with hipcc (in parallel), then linked into
``causal_conv1d_amd/_lib/libcc1d_amd.so``. The library exposes only the
``extern "C"`` entry points of ``include/cc1d.h``. ``bench/cc1d_floor.hip``
(bandwidth floors that ``bench.py`` times beside the kernels; measurement
code, not part of the package) is linked on its own into
``libcc1d_floor.so`` beside ``bench.py`` at the repository root.

Usage: ``python causal-conv1d-mojo_amd/csrc/build.py [--jobs N] [--verbose]``.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG_ROOT = CSRC.parent
REPO = PKG_ROOT.parent
INCLUDE = REPO / "include"
OBJ_DIR = CSRC / "_build"
LIB_DIR = PKG_ROOT / "causal_conv1d_amd" / "_lib"
LIB_PATH = LIB_DIR / "libcc1d_amd.so"
# bandwidth floors for bench.py (measurement only: built beside bench.py, outside the package)
FLOOR_SRC = CSRC / "bench" / "cc1d_floor.hip"
FLOOR_PATH = REPO / "libcc1d_floor.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: keep the backend from forming v_pk_{add,mul,fma}_f32;
# every fp32 operation stays a scalar VALU instruction.
# -munsafe-fp-atomics: fp32 atomicAdd maps to the hardware
# global_atomic_add_f32 (the accumulators live in coarse-grained memory).
COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, verbose: bool) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    # the host pass warns that it does not know the packed-fp32 feature; drop that noise
    noise = ("packed-fp32-ops", "warning generated", "warnings generated")
    msgs = [ln for ln in res.stderr.splitlines() if ln.strip() and not any(n in ln for n in noise)]
    if msgs and verbose:
        print("\n".join(msgs), file=sys.stderr)
    return obj


def _link(objs: list[Path], out: Path, verbose: bool) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library (and the bench's
    floor library). Returns the product library's path."""
    if HIPCC is None or not Path(HIPCC).exists():
        raise RuntimeError("hipcc not found; set HIPCC or install ROCm")
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    srcs = _sources() + [FLOOR_SRC]
    jobs = jobs or min(len(srcs), max(1, os.cpu_count() or 1))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    _link(objs[:-1], LIB_PATH, verbose)
    _link(objs[-1:], FLOOR_PATH, verbose)
    return LIB_PATH


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    path = build(args.jobs, args.verbose)
    print(path)


if __name__ == "__main__":
    main()
