"""Host-side checks of the C ABI (no GPU work): the library loads, exports every function that
include/sq8.h declares, and rejects bad arguments with the documented status codes before it
touches the device."""
import re
from pathlib import Path

import pytest

from conftest import REPO

HEADER = REPO / "include" / "sq8.h"
HEADERS = sorted((REPO / "include").glob("*.h"))


def declared_functions(headers=(HEADER,)):
    names = set()
    for h in headers:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(sq8_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_expected(sq8):
    assert declared_functions() == sorted(sq8.EXPORTED_SYMBOLS)
    assert declared_functions(HEADERS) == sorted(sq8.EXPORTED_SYMBOLS + sq8.DECODE_SYMBOLS +
                                                 sq8.BATCH_SYMBOLS + sq8.PROBE_SYMBOLS)


def test_library_exports_every_declared_symbol(sq8):
    lib = sq8.lib()
    for name in declared_functions(HEADERS):
        assert hasattr(lib, name), name


def test_status_codes_match_header(sq8):
    text = HEADER.read_text()
    for name in ("SQ8_OK", "SQ8_ERR_NULL", "SQ8_ERR_DIMS", "SQ8_ERR_GROUP", "SQ8_ERR_WORKSPACE",
                 "SQ8_ERR_LAUNCH", "SQ8_ERR_DEVICE"):
        m = re.search(rf"{name}\s*=\s*(-?\d+)", text)
        assert m and int(m.group(1)) == getattr(sq8, name), name
        assert sq8.status_string(getattr(sq8, name)) != "unknown status"


FAKE = 0x1000  # never dereferenced: validation fails first


@pytest.mark.parametrize("args,code", [
    ((0, FAKE, FAKE, FAKE, 1, 8, 64, 64), -1),       # null x
    ((FAKE, FAKE, 0, FAKE, 1, 8, 64, 64), -1),       # null scales
    ((FAKE, FAKE, FAKE, FAKE, 0, 8, 64, 64), -2),    # empty batch (reference CHECKs non-empty)
    ((FAKE, FAKE, FAKE, FAKE, 1, 0, 64, 64), -2),
    ((FAKE, FAKE, FAKE, FAKE, 1, 8, 66, 2), -2),     # K % 4 != 0 (matmul_kernel.cu:185)
    ((FAKE, FAKE, FAKE, FAKE, 1, 8, 64, 0), -3),     # group size 0
    ((FAKE, FAKE, FAKE, FAKE, 1, 3, 100, 64), -3),   # N*K not a multiple of gs (layer.cpp:210)
])
def test_argument_errors(sq8, args, code):
    assert sq8.matmul_raw(*args) == code


def test_workspace_too_small_is_rejected(sq8):
    for M, N, K in ((64, 4096, 4096), (2048, 4096, 4096)):
        need = sq8.workspace_bytes(M, N, K, 64)
        if need:
            assert sq8.matmul_raw(FAKE, FAKE, FAKE, FAKE, M, N, K, 64, FAKE, need - 1) == -4


def test_path_selection(sq8):
    assert sq8.path_name(1, 4096, 4096, 64) == "gemv"
    assert sq8.path_name(2, 4096, 4096, 64) == "gemv"
    assert sq8.path_name(4, 4096, 4096, 64) == "gemv"      # 4 token rows still fit the LDS stage
    assert sq8.path_name(3, 4096, 14336, 64) == "mfma"
    assert sq8.path_name(2048, 4096, 4096, 64) == "mfma"
    assert sq8.path_name(8, 4096, 4096, 32) == "gemv"      # MFMA steps are whole 64-wide groups
    assert sq8.path_name(1, 4096, 100, 4) == "generic"   # gs not a multiple of 16
    assert sq8.path_name(1, 16, 100, 64) == "generic"    # K not a multiple of gs
    assert sq8.path_name(0, 16, 64, 64) == "invalid"


def test_workspace_sizes(sq8):
    assert sq8.workspace_bytes(1, 4096, 4096, 64) == 0
    # MFMA paths: split-K tickets and partials; the GEMM path adds f16 hi/lo copies of x (4*M*K B)
    for M in (8, 64, 2048):
        assert sq8.workspace_bytes(M, 4096, 4096, 64) > 0
    assert sq8.workspace_bytes(2048, 4096, 4096, 64) >= 4 * 2048 * 4096
    assert sq8.workspace_bytes(0, 4096, 4096, 64) == 0


def epi_raw(sq8, x, w, s, y, M, N, K, gs, epi, res, ws=0, wsb=0):
    return int(sq8.lib().sq8_matmul_epilogue(x or None, w or None, s or None, y or None, M, N, K,
                                             gs, epi, res or None, ws or None, wsb, None))


@pytest.mark.parametrize("M,N,K,epi,res,code", [
    (128, 512, 1024, 1, 0, -1),        # residual epilogue without a residual
    (128, 511, 1024, 2, 0, -2),        # SwiGLU needs the even N of a [w1; w3] weight
    (128, 512, 1024, 7, 0, -2),        # unknown epilogue
    (128, 512, 66, 2, 0, -2),          # the ordinary shape checks still apply
    (128, 512, 1024, 2, 0, -4),        # no workspace
    (4, 512, 1024, 1, FAKE, -4),       # unfused path: the product buffer is workspace too
])
def test_epilogue_argument_errors(sq8, M, N, K, epi, res, code):
    assert epi_raw(sq8, FAKE, FAKE, FAKE, FAKE, M, N, K, 64, epi, res) == code


def test_epilogue_fusion_and_workspace(sq8):
    # the prefill GEMM fuses; decode paths run the product into the workspace first
    assert sq8.epilogue_fused(2048, 28672, 4096)
    assert sq8.epilogue_fused(64, 4096, 14336)
    assert not sq8.epilogue_fused(1, 28672, 4096)
    assert not sq8.epilogue_fused(16, 28672, 4096)
    assert sq8.epilogue_fused(48, 28672, 4096)      # the decode GEMM (wide outputs, 33-64 rows)
    assert not sq8.epilogue_fused(48, 6144, 4096)   # the tile kernel
    L = sq8.lib()
    for M, N, K in ((1, 8192, 4096), (16, 8192, 4096), (2048, 8192, 4096)):
        base = sq8.workspace_bytes(M, N, K, 64)
        assert L.sq8_epilogue_workspace_bytes(M, N, K, 64, 0) == base
        for e in (1, 2):
            extra = L.sq8_epilogue_workspace_bytes(M, N, K, 64, e) - base
            # the product never lands in the 64 KiB ticket area of MFMA workspaces
            off = (max(base, 65536) + 255) // 256 * 256
            assert extra == (0 if sq8.epilogue_fused(M, N, K) else off + M * N * 4 - base)


def test_op_library_exports_its_c_interfaces(sq8):
    """libsq8_op.so exports every function of the scheduler and model C interfaces
    (llm-steadyinfer_amd/cpp/include/scheduler/scheduler_c.h, model/batch_model_c.h), and the
    Python binding binds exactly those."""
    import importlib
    nat = importlib.import_module("llm_steadyinfer_amd.native_scheduler")
    inc = REPO / "llm-steadyinfer_amd" / "cpp" / "include"
    sched_h, model_h = inc / "scheduler" / "scheduler_c.h", inc / "model" / "batch_model_c.h"
    assert declared_functions((sched_h,)) == sorted(nat.SCHED_SYMBOLS)
    assert declared_functions((model_h,)) == sorted(nat.MODEL_SYMBOLS)
    lib = nat.op_lib()
    for name in declared_functions((sched_h, model_h)):
        assert hasattr(lib, name), name


def test_c_headers_compile_as_c(tmp_path):
    """Every C interface header (include/*.h, the scheduler's and the models') is valid C99, as
    an FFI host (cgo, a C program) would include it."""
    import shutil
    import subprocess
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    inc = REPO / "llm-steadyinfer_amd" / "cpp" / "include"
    headers = HEADERS + [inc / "scheduler" / "scheduler_c.h", inc / "model" / "batch_model_c.h"]
    src = tmp_path / "all.c"
    src.write_text("".join(f'#include "{h}"\n' for h in headers) + "int main(void) { return 0; }\n")
    res = subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror",
                          "-fsyntax-only", str(src)], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, res.stderr[-3000:]
