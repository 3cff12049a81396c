"""Tape formats on the CPU (tests/cpp/test_tape.cpp, `cpu` mode): records
byte-equal to the reference TapeWriter's (tests/golden/tape_records.bin,
written by tests/golden/make_tape.py), composite party-key tapes, key
arrays."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
EXE = os.path.join(HERE, "cpp", "_build", "test_tape")


def test_tape_formats_cpu():
    if not os.path.exists(EXE):
        pytest.skip("C++ test driver not built: run python -m suf_amd.build")
    r = subprocess.run([EXE, "cpu", os.path.join(HERE, "golden", "tape_records.bin")],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert "passed" in r.stdout
