"""CPU replay of the MFMA and packed-GEMV kernels' address arithmetic (no GPU).

``tests/cpp/test_index_replay.cpp`` compiles the plan and index header the kernels use
(``csrc/sq8_plan.h``) with g++ and walks every weight, scale, activation, partial and ticket
address of each launch for the Llama-3-8B and Qwen2-1.5B projection and LM-head shapes, fused
gate/up weights with N/2 % 16 != 0, and N = 1..64: loads in bounds and aligned, each weight load
decoded through the packed (or row-major) layout to the row and K range its lane multiplies, and
every (row, group) read once. It also checks that two known-bad variants are caught: the packed
GEMV's unclamped scale float4 at 8 groups per step, and a packed address that takes the row's
place in its tile from the lane.
"""
import shutil
import subprocess

import pytest

from conftest import REPO


def test_kernel_index_replay(tmp_path):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "test_index_replay"
    src = REPO / "tests" / "cpp" / "test_index_replay.cpp"
    res = subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-Werror", "-pthread", "-I",
                          str(REPO / "llm-steadyinfer_amd" / "csrc"), str(src), "-o", str(exe)],
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-3000:]
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    print(run.stdout[-2000:])
    assert run.returncode == 0, run.stdout[-3000:] + run.stderr[-2000:]
    assert "0 failures, 0 mutations missed" in run.stdout
