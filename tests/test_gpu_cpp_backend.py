"""Runs the C++ two-party test of HipPfssBackend (tests/cpp/test_hip_backend.cpp,
built by `python -m suf_amd.build`) on the GPU: the proto-interface backend,
a dealer instance plus one instance per party thread, reconstructing DCF,
interval-LUT and packed-compare outputs against their closed forms."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "_build", "test_hip_backend")


def test_cpp_two_party_backend():
    assert os.path.exists(EXE), "C++ test driver not built: run python -m suf_amd.build"
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stderr
    assert "two-party test passed" in r.stdout
