"""Writes tests/golden/tables_f12.json: the GeLU, nExp and reciprocal tables
(piece boundaries and coefficient words, f = 12) and the rsqrt affine-init
intervals, as the reference's own header-only builders produce them.  The
values come from oracle/_ref/ref_tables (oracle/ref_tables.cpp over
include/gates/tables/*.hpp and include/suf/suf_silu_builders.hpp, built by
oracle/build_ref.sh in this container).

Run from the repository root:  python tests/golden/make_tables.py
"""
import json
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
EXE = os.path.join(ROOT, "oracle", "_ref", "ref_tables")


def main():
    if not os.path.exists(EXE):
        raise SystemExit("oracle/_ref/ref_tables not built: run sh oracle/build_ref.sh first")
    out = subprocess.run([EXE], check=True, capture_output=True, text=True).stdout
    data = json.loads(out)
    data["source"] = ("reference builders (gelu_spline_table.hpp, nexp_piecewise_table.hpp, "
                      "recip_piecewise_affine_init.hpp through build_silu_suf_from_piecewise; "
                      "rsqrt_piecewise_affine_init.hpp intervals) via oracle/ref_tables.cpp")
    with open(os.path.join(HERE, "tables_f12.json"), "w") as f:
        json.dump(data, f, indent=1)
    print("wrote", os.path.join(HERE, "tables_f12.json"))


if __name__ == "__main__":
    main()
