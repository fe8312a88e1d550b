"""The C++ op API (MatmulLayer over get_matmul_kernel_quant8) through its own test program
(tests/cpp/test_matmul_layer.cpp, built by __graft_entry__.build())."""
import subprocess

import pytest

from conftest import REPO

BIN = REPO / "llm-steadyinfer_amd" / "_build" / "test_matmul_layer"


def _run(mode, timeout):
    if not BIN.exists():
        pytest.fail(f"{BIN} not built (run __graft_entry__.build())")
    res = subprocess.run([str(BIN), mode], capture_output=True, text=True, timeout=timeout)
    print(res.stdout)
    print(res.stderr[-2000:])
    assert res.returncode == 0, res.stdout[-2000:]
    assert f"{mode}: 0 failure(s)" in res.stdout


def test_op_layer_host_logic():
    """Weight/scale binding, shape checks and tensor basics; no GPU calls."""
    _run("host", 60)


@pytest.mark.gpu
def test_op_layer_forward_on_gpu():
    """MatmulLayer::forward on the HIP device against the CPU oracle, incl. bias and 1-D input."""
    _run("gpu", 110)
