"""Builds libttlhip.so (gfx950) from the HIP sources in this directory.

Every source is compiled with hipcc for gfx950 only, in parallel, then linked
into tt-lang_amd/ttlhip/libttlhip.so, where the Python runtime loads it.
Packed-fp32 instruction selection is disabled for all device code.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent
OUT_DIR = PKG / "ttlhip"
LIB = OUT_DIR / "libttlhip.so"
OBJ_DIR = CSRC / "_build"

SOURCES = ["runtime.hip", "eltwise.hip", "matmul.hip", "bfp8.hip", "sdpa.hip", "layout.hip"]

ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libttlhip.so)")


COMMON_FLAGS = [
    "-std=c++17",
    "-O3",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    "-I", str(PKG.parent / "include"),
]


# Per-source flags.  eltwise.hip: kernarg preloading of the first four
# arguments, so the flat kernel's operand bases and chunk count and the bf16
# row reduction's row base, stride and width arrive in SGPRs at wave start
# (the other kernels take one struct argument, which is never preloaded).
# layout.hip: all five arguments of the tilize / untilize kernel (4096^2 bf16
# tilize 10.6 -> 10.2 us).  Not bfp8.hip: its unpack kernel (44k waves at C4)
# measured 0.5% slower with its arguments preloaded.
EXTRA_FLAGS = {
    "eltwise.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=4"],
    "layout.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=5"],
}


def _compile(src: str) -> Path:
    obj = OBJ_DIR / (Path(src).stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    OBJ_DIR.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), 8)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
