"""Build recipe for the gfx950 INT8 group-quant matmul library (``libsq8.so``).

Compiles every ``csrc/*.hip`` with hipcc for gfx950 and links one shared library that exports the
C ABI declared in ``include/sq8.h``. Runs on a machine without a GPU (hipcc cross-compiles).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
OBJ_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libsq8.so"
CPP_DIR = PKG_DIR / "cpp"
OP_LIB_PATH = PKG_DIR / "libsq8_op.so"
CPP_TEST_NAMES = ("test_matmul_layer", "test_model_file")
ORACLE_LIB = REPO_DIR / "oracle" / "_ref" / "libsq8_oracle.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed fp32 VALU instructions (v_pk_*_f32) are disabled for every device compile.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall",
                "-Wno-unused-result", "-I", str(REPO_DIR / "include"), "-I", str(CSRC)]


def _compile(src: Path, extra=()) -> Path:
    obj = OBJ_DIR / (src.parent.name + "_" + src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *extra, *DEVICE_FLAGS, "-x", "hip", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that noise.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msgs = [ln for ln in res.stderr.splitlines() if ln.strip() and noise not in ln]
    if msgs:
        print("\n".join(msgs), file=sys.stderr)
    return obj


def _link(objs, out: Path, extra=()):
    tmp = out.with_suffix(out.suffix + ".tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", *map(str, objs), *extra, "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of {out.name} failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)


def build_op_layer(verbose: bool = False) -> Path:
    """Compile the C++ op API (Tensor, MatmulLayer, get_matmul_kernel_quant8) into libsq8_op.so,
    linked against libsq8.so."""
    srcs = sorted((CPP_DIR / "src").glob("*.cpp")) + sorted((CPP_DIR / "src").glob("*.hip"))
    inc = ["-I", str(CPP_DIR / "include")]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda p: _compile(p, inc), srcs))
    _link(objs, OP_LIB_PATH, ["-shared", "-fPIC", "-L", str(PKG_DIR), "-lsq8",
                              "-Wl,-rpath,$ORIGIN"])
    if verbose:
        print(f"built {OP_LIB_PATH}")
    return OP_LIB_PATH


def build_cpp_tests(verbose: bool = False) -> list:
    """Compile the C++ test programs (link libsq8_op.so, libsq8.so and the oracle as checker)."""
    if not ORACLE_LIB.exists():
        raise RuntimeError(f"oracle library missing: {ORACLE_LIB}")
    inc = ["-I", str(CPP_DIR / "include"), "-I", str(REPO_DIR / "tests" / "cpp")]
    out = []
    for name in CPP_TEST_NAMES:
        obj = _compile(REPO_DIR / "tests" / "cpp" / f"{name}.cpp", inc)
        binary = OBJ_DIR / name
        _link([obj], binary, ["-L", str(PKG_DIR), "-lsq8_op", "-lsq8", "-L",
                              str(ORACLE_LIB.parent), "-lsq8_oracle",
                              "-Wl,-rpath,$ORIGIN/..", "-Wl,-rpath,$ORIGIN/../../oracle/_ref"])
        if verbose:
            print(f"built {binary}")
        out.append(binary)
    return out


def build(verbose: bool = False) -> Path:
    """Compile all HIP sources and link ``libsq8.so``; returns the library path."""
    OBJ_DIR.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    _link(objs, LIB_PATH, ["-shared", "-fPIC"])
    if verbose:
        print(f"built {LIB_PATH}")
    build_op_layer(verbose)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
