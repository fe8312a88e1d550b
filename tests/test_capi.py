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
                                                 sq8.BATCH_SYMBOLS)


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
