"""Writes tests/golden/tape_records.bin: a tape written by the reference's own
proto::TapeWriter (include/proto/tape.hpp) through oracle/_ref/ref_tape
(oracle/ref_tape.cpp, built by oracle/build_ref.sh in this container).

Run from the repository root:  python tests/golden/make_tape.py
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
EXE = os.path.join(ROOT, "oracle", "_ref", "ref_tape")


def main():
    if not os.path.exists(EXE):
        raise SystemExit("oracle/_ref/ref_tape not built: run sh oracle/build_ref.sh first")
    out = os.path.join(HERE, "tape_records.bin")
    subprocess.run([EXE, out], check=True)
    print("wrote", out, os.path.getsize(out), "bytes")


if __name__ == "__main__":
    main()
