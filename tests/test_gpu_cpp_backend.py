"""Runs the C++ two-party test of HipPfssBackend (tests/cpp/test_hip_backend.cpp,
built by `python -m suf_amd.build`) on the GPU: the proto-interface backend,
a dealer instance plus one instance per party thread, reconstructing DCF,
interval-LUT and packed-compare outputs against their closed forms and SUF's
AddU64 truncation route (composite_gen_trunc_gate's queries, the host bool
plan, launch_trunc_postproc_kernel on last_device_bools()) against x >> f;
and the reference's own XOR-group keys evaluated byte-equal to its shares."""
import json
import os
import subprocess
import tempfile

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


def test_cpp_backend_evaluates_reference_xor_keys():
    """Keys the reference's myl7 adapter made in the XOR group (1-, 8- and
    16-byte payloads, tests/golden/dcf_myl7.json) evaluate byte-equal to the
    reference's shares on an instance with xor_payloads."""
    assert os.path.exists(EXE), "C++ test driver not built: run python -m suf_amd.build"
    here = os.path.dirname(os.path.abspath(__file__))
    g = json.load(open(os.path.join(here, "golden", "dcf_myl7.json")))
    lines = ["prg %s" % g["prg_state"]]
    for c in g["cases"]:
        if c["group"] != "xor":
            continue
        plen = len(c["payload"]) // 2
        lines.append("case %d %d %s %s %d" % (c["in_bits"], plen, c["key0"], c["key1"], len(c["xs"])))
        for x, o0, o1 in zip(c["xs"], c["out0"]["full"], c["out1"]["full"]):
            lines.append("x %d %s %s" % (int(x), o0, o1))
    with tempfile.NamedTemporaryFile("w", suffix=".txt", delete=False) as f:
        f.write("\n".join(lines) + "\n")
        path = f.name
    try:
        r = subprocess.run([EXE, "golden", path], capture_output=True, text=True, timeout=110)
    finally:
        os.unlink(path)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stderr
    assert "golden xor keys" in r.stdout


def test_cpp_trunc_route_timings():
    """Times SUF's AddU64 truncation route through the backend (host bool
    plan, then the postproc launcher), its device-kept form and the fused
    truncation gate, both parties, GapARS f = 12 at 2^16 and 2^20 points;
    the shares of these routes are checked by test_cpp_two_party_backend."""
    assert os.path.exists(EXE), "C++ test driver not built: run python -m suf_amd.build"
    r = subprocess.run([EXE, "time-trunc"], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stderr
    assert r.stdout.count("trunc routes GapARS") == 2
