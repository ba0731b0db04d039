"""Build libmolt_amd.so (hand-written HIP for gfx950) in-tree.

Usage: ``python -m molt_amd.build`` (or ``__graft_entry__.build()``).
Every translation unit is compiled for ``--offload-arch=gfx950`` only, with
packed-fp32 VALU instructions disabled on the device side.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_lib"
LIB = OUT_DIR / "libmolt_amd.so"
SOURCES = ["capi.cpp", "ce.hip", "codec.hip", "gemv.hip", "lora.hip", "nf4_gemm.hip", "rmsnorm.hip", "swiglu.hip"]
ARCH = "gfx950"

DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
                "-Wno-unused-variable", "-Wno-unused-but-set-variable"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the MI355X library needs ROCm's hipcc")


def _compile(src: str, build_dir: Path) -> Path:
    obj = build_dir / (src.rsplit(".", 1)[0] + ".o")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", *COMMON_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    if src.endswith(".hip"):
        cmd[2:2] = ["-x", "hip", *DEVICE_FLAGS]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every source and link the shared library; returns its path."""
    build_dir = PKG / "_build"
    build_dir.mkdir(exist_ok=True)
    OUT_DIR.mkdir(exist_ok=True)
    workers = min(len(SOURCES), max(1, int(os.environ.get("MAX_JOBS", "8"))))
    with cf.ThreadPoolExecutor(workers) as pool:
        objs = list(pool.map(lambda s: _compile(s, build_dir), SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
