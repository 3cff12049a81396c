"""Writes tests/golden/suf_ref_eval.json: the reference's own eval_suf_ref
(include/suf/ref_eval.hpp:58-78) on the MIXED and DRELU gates of
tests/composite_specs.py at boundary and random points, from
oracle/_ref/ref_suf_eval (oracle/ref_suf_eval.cpp, built by
oracle/build_ref.sh in this container).

Run from the repository root:  python tests/golden/make_suf_ref.py
"""
import json
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
EXE = os.path.join(ROOT, "oracle", "_ref", "ref_suf_eval")


def main():
    if not os.path.exists(EXE):
        raise SystemExit("oracle/_ref/ref_suf_eval not built: run sh oracle/build_ref.sh first")
    data = json.loads(subprocess.run([EXE], check=True, capture_output=True, text=True).stdout)
    data["source"] = "eval_suf_ref of the reference (oracle/ref_suf_eval.cpp)"
    with open(os.path.join(HERE, "suf_ref_eval.json"), "w") as f:
        json.dump(data, f, indent=0)
    print("wrote", os.path.join(HERE, "suf_ref_eval.json"))


if __name__ == "__main__":
    main()
