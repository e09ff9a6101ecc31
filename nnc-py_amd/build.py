"""Build libnnc_hip.so (gfx950) from csrc/*.hip with hipcc, in-tree.

    python nnc-py_amd/build.py            # build lib/libnnc_hip.so
    python nnc-py_amd/build.py --jobs 8

Objects go to _build/, the library to lib/. Every source is compiled for
gfx950 only, with packed-fp32 instructions disabled
(-target-feature -packed-fp32-ops): hipcc -O3 would otherwise emit
v_pk_*_f32 on its own.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libnnc_hip.so"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

CXXFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *CXXFLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the gfx feature flag and says so; drop
    # that line, keep everything else
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l).strip()
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err:
        print(err, file=sys.stderr)
    return obj


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    """Compile every csrc/*.hip and link lib/libnnc_hip.so. Always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 8)
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} ({LIB.stat().st_size / 1e6:.1f} MB, {len(objs)} objects)")
    build_costmodel(verbose)
    return LIB


COSTMODEL = LIBDIR / "libnnc_costmodel.so"


def build_costmodel(verbose: bool = True) -> Path:
    """lib/libnnc_costmodel.so: the cost-model runtime (host C++, no HIP)."""
    LIBDIR.mkdir(exist_ok=True)
    tmp = COSTMODEL.with_suffix(".so.tmp")
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall",
           f"-I{ROOT / 'include'}", f"-I{CSRC}", str(CSRC / "costmodel.cpp"), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"cost model build failed:\n{res.stderr}")
    os.replace(tmp, COSTMODEL)
    if verbose:
        print(f"built {COSTMODEL}")
    return COSTMODEL


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    build(args.jobs)
