"""Composite party-key tapes on the CPU: the Python host side's
write_composite_tape / read_composite_tape (suf_amd/tape.py) against the C++
host side's (include/suf_hip/tape.hpp, through tests/cpp/test_tape.cpp):
a tape either side writes is read and written back byte-equal by the other,
and every truncated tape is refused.  Both restate
gates::write_composite_tape / read_composite_tape
(include/gates/composite_fss.hpp:2458-2641); the C++ side's field sizes are
checked against that layout in tests/cpp/test_tape.cpp."""
import os
import subprocess
import tempfile

import numpy as np
import pytest

from suf_amd import tape

HERE = os.path.dirname(os.path.abspath(__file__))
EXE = os.path.join(HERE, "cpp", "_build", "test_tape")


def _random_key(seed, triples=11, bit_triples=7):
    rng = np.random.default_rng(seed)
    w = lambda n: rng.integers(0, 2**64, n, dtype=np.uint64)  # noqa: E731
    k = tape.empty_key()
    k.update({"r_in_share": int(w(1)[0]), "r_in_share_vec": w(2), "r_out_share": w(3),
              "wrap_share": w(4), "r_hi_share": int(w(1)[0]), "wrap_sign_share": int(w(1)[0]),
              "extra_params": w(1), "pred_meta": (0, 0, 1), "cut_pred_meta": (1, 0, 1),
              "coeff_meta": (0, 1),
              "pred_keys": [rng.integers(0, 256, 40 + 9 * i, dtype=np.uint8).tobytes()
                            for i in range(3)],
              "cut_pred_keys": [b"\x05" * 17],
              "coeff_keys": [rng.integers(0, 256, 64, dtype=np.uint8).tobytes()],
              "base_coeff_share": w(2), "total_delta_share": w(2),
              "triples": w(3 * triples).reshape(triples, 3),
              "bit_triples": rng.integers(0, 2, (bit_triples, 3), dtype=np.uint8)})
    return k


def _run(*args):
    assert os.path.exists(EXE), "C++ test driver not built: run python -m suf_amd.build"
    r = subprocess.run([EXE] + list(args), capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr


def test_python_tape_round_trips_through_cpp():
    t = tape.write_composite_tape(_random_key(1))
    with tempfile.TemporaryDirectory() as d:
        src, dst = os.path.join(d, "py.tape"), os.path.join(d, "cpp.tape")
        with open(src, "wb") as f:
            f.write(t)
        _run("composite-rw", src, dst)
        with open(dst, "rb") as f:
            assert f.read() == t


def test_cpp_tape_round_trips_through_python():
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "cpp.tape")
        _run("composite-write", path)
        with open(path, "rb") as f:
            t = f.read()
    k = tape.read_composite_tape(t)
    assert tape.write_composite_tape(k) == t
    assert len(k["pred_keys"]) == 3 and [len(b) for b in k["pred_keys"]] == [100, 137, 174]
    assert k["triples"].shape == (7, 3) and k["bit_triples"].shape == (9, 3)
    assert k["pred_meta"] == (1, 2, 8) and k["coeff_meta"] == (1, 2)


def test_layout_of_the_head():
    k = _random_key(2)
    t = tape.write_composite_tape(k)
    assert int.from_bytes(t[0:8], "little") == k["r_in_share"]
    assert int.from_bytes(t[8:12], "little") == 2  # r_in_share_vec length
    assert int.from_bytes(t[12:20], "little") == int(k["r_in_share_vec"][0])
    # tail: [u32 bit-triple count][a b c] x 7
    assert int.from_bytes(t[-(4 + 21):-21], "little") == 7
    assert t[-21:] == k["bit_triples"].tobytes()


def test_every_truncation_is_refused():
    t = tape.write_composite_tape(_random_key(3, triples=2, bit_triples=2))
    for ln in range(len(t)):
        with pytest.raises(ValueError, match="truncated"):
            tape.read_composite_tape(t[:ln])
