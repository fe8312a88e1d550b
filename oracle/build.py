"""Build recipe for the CPU oracle (test infrastructure only).

Compiles ``oracle/sq8_oracle.c`` with gcc into ``oracle/_ref/libsq8_oracle.so``. The reference
itself is not compiled: its path needs CUDA, cub, glog and armadillo, none of which exist here.
"""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
OUT_DIR = ORACLE_DIR / "_ref"
LIB_PATH = OUT_DIR / "libsq8_oracle.so"

# x86-64-v3 (AVX2 + FMA) instead of -march=native: the library is built here and runs on the GPU
# box's host, whose exact CPU model is not known at build time.
CFLAGS = ["-O3", "-march=x86-64-v3", "-fopenmp", "-fPIC", "-shared", "-std=c11", "-Wall"]


def build() -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [os.environ.get("CC", "gcc"), *CFLAGS, str(ORACLE_DIR / "sq8_oracle.c"), "-lm", "-o",
           str(tmp)]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build())
