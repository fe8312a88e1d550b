"""op::MatmulLayer's opt-in packed upload on the host (no GPU): tests/cpp/test_packed_layer_host.cpp
built with g++ under ASan/UBSan against host stand-ins of HIP and libsq8 and a recording kernel
table. The uploaded bytes must be the packed layout (checked against its formula), forward() must
call the packed kernel with them (the row-major one without the opt-in), and pack_weights() must
refuse a host weight, an fp32 layer and K % 64 != 0."""
import shutil
import subprocess

import pytest

from conftest import REPO


def test_packed_matmul_layer_upload_on_host(tmp_path):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    cpp, t = REPO / "llm-steadyinfer_amd" / "cpp", REPO / "tests" / "cpp"
    exe = tmp_path / "test_packed_layer_host"
    srcs = [str(cpp / "src" / f"{f}.cpp") for f in ("alloc", "buffer", "tensor", "layer", "matmul",
                                                    "hip_config")]
    res = subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
                          "-fno-sanitize-recover=undefined", "-I", str(t / "mock_hip"), "-I",
                          str(cpp / "include"), "-I", str(t), str(t / "test_packed_layer_host.cpp"),
                          str(t / "mock_sq8.cpp")] + srcs + ["-o", str(exe)],
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-3000:]
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(run.stdout)
    assert run.returncode == 0, run.stdout[-2000:] + run.stderr[-3000:]
    assert "packed layer host: 0 failure(s)" in run.stdout
