"""oracle/suf_ref.py (the plaintext SUF evaluation the composite gates must
reconstruct to) against the reference's own eval_suf_ref: every point of
tests/golden/suf_ref_eval.json (tests/golden/make_suf_ref.py), for the
MIXED and DRELU gates of tests/composite_specs.py."""
import json
import os

import numpy as np
import pytest

import composite_specs as cs
import suf_ref

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def golden():
    with open(os.path.join(HERE, "golden", "suf_ref_eval.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("name,spec", [("mixed", cs.MIXED), ("drelu", cs.DRELU)])
def test_suf_ref_matches_reference(golden, name, spec):
    rows = golden[name]
    x = np.array([int(r["x"]) for r in rows], dtype=np.uint64)
    arith, bools, piece = suf_ref.eval_suf(spec, x)
    assert [int(v) for v in piece] == [r["piece"] for r in rows]
    assert [int(v) for v in arith[:, 0]] == [int(r["arith"]) for r in rows]
    assert bools.astype(int).tolist() == [r["bools"] for r in rows]
