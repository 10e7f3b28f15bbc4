"""Builds the oracle's C restatements (test infrastructure only).

oracle/bfp8_ref.c -> oracle/_build/liboraclebfp8.so (gcc, no dependencies).
The reference itself ships no C/C++ code on this path (its kernels are
Python run by the simulator, or MLIR-generated Tensix C++ that needs the
un-vendored tt-metal toolchain), so there is no oracle/_ref build.
"""

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "_build"
LIB = OUT / "liboraclebfp8.so"


def build() -> Path:
    OUT.mkdir(exist_ok=True)
    cmd = ["gcc", "-O2", "-std=c99", "-fPIC", "-shared", "-Wall", str(HERE / "bfp8_ref.c"),
           "-o", str(LIB)]
    subprocess.run(cmd, check=True)
    return LIB


if __name__ == "__main__":
    print(build())
