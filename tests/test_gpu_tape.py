"""Keys streamed from a tape file into device buffers (tests/cpp/test_tape.cpp,
`gpu` mode): DCF keys and truncation-gate keys come back byte-equal through
DeviceKeyArray's pinned staging, and evaluate as the originals do."""
import os
import subprocess
import tempfile

import pytest

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "_build", "test_tape")


def test_tape_keys_to_device():
    assert os.path.exists(EXE), "C++ test driver not built: run python -m suf_amd.build"
    with tempfile.TemporaryDirectory() as d:
        r = subprocess.run([EXE, "gpu", d], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stderr
    assert "passed" in r.stdout
