"""DeviceOpenCollector's host rules on the CPU (tests/cpp/test_open_collector.cpp,
`cpu` mode): handles, generations, the pending budget, empty and ready."""
import os
import subprocess

import pytest

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "_build",
                   "test_open_collector")


def test_open_collector_host_rules():
    if not os.path.exists(EXE):
        pytest.skip("C++ test driver not built: run python -m suf_amd.build")
    r = subprocess.run([EXE, "cpu"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "passed" in r.stdout


@pytest.mark.gpu
def test_open_collector_flushes_on_gpu():
    assert os.path.exists(EXE), "C++ test driver not built: run python -m suf_amd.build"
    r = subprocess.run([EXE, "gpu"], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stderr
    assert "passed" in r.stdout
