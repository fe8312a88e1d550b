"""bench.py's command-line contract that needs no GPU: this build measures one GPU only, so any
other GPU count exits with status 2 and says so (before touching torch or the device)."""
import subprocess
import sys

from conftest import REPO


def test_multi_gpu_request_exits_with_message():
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""
