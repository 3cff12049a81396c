"""suf_amd/tables.py against the reference's own table builders (CPU).

tests/golden/tables_f12.json holds, at f = 12, the tables the reference's
header-only builders produce (tests/golden/make_tables.py over
oracle/ref_tables.cpp): make_gelu_spline_spec, make_nexp_piecewise_spec and
make_recip_affine_init_spec each through build_silu_suf_from_piecewise
(piece boundaries ending at the ~0 surrogate of 2^64, four coefficient
words per piece), and make_rsqrt_affine_init_spec's raw intervals.  The
restated builders must give the same boundaries and words exactly.  For
rsqrt the fixture holds the spec; the words of build_rsqrt_affine_eval_suf
(src/nn/transformer_layer.cpp:193-252) are the integer step
adj = a0 - floor(a1 * offset / 2^f), a1 applied here to the reference's
intervals (an exact integer formula, checked by hand below)."""
import json
import os

import pytest

from suf_amd import tables

HERE = os.path.dirname(os.path.abspath(__file__))
M64 = (1 << 64) - 1
F = 12


@pytest.fixture(scope="module")
def ref():
    with open(os.path.join(HERE, "golden", "tables_f12.json")) as f:
        d = json.load(f)
    assert d["frac_bits"] == F
    return d


@pytest.mark.parametrize("name,fn,words", [("gelu", tables.gelu_table, 4),
                                           ("nexp", tables.nexp_table, 4),
                                           ("recip", tables.recip_table, 2)])
def test_silu_style_tables_match_reference(ref, name, fn, words):
    alpha, coeffs = fn(F)
    ra = [int(v) for v in ref[name]["alpha"]]
    rc = [[int(v) for v in row] for row in ref[name]["coeffs"]]
    # Boundaries: the reference lists the piece starts plus the last end (~0).
    assert ra[-1] == M64
    assert [int(v) for v in alpha] == ra[:-1]
    assert len(coeffs) == len(rc)
    for i, row in enumerate(rc):
        assert [int(v) for v in coeffs[i]] == row[:words], (name, i)
        assert not any(row[words:]), (name, i)  # the words the gate does not read are 0


def test_rsqrt_table_matches_reference_intervals(ref):
    spec = ref["rsqrt_spec"]
    f = spec["frac_bits_in"]
    ivs = sorted(spec["intervals"], key=lambda v: int(v["start"]))
    want_alpha, want = [], []
    if int(ivs[0]["start"]) != 0:
        want_alpha.append(0)
        want.append([0, 0])
    for iv in ivs:
        a = [int(c) for c in iv["coeffs"]] + [0, 0]
        off = int(iv["offset"])
        adj = a[0] - ((a[1] * off) >> f)
        want_alpha.append(int(iv["start"]))
        want.append([adj, a[1]])
    ends = [int(iv["end"]) for iv in ivs]
    assert ends[-1] == M64
    assert ends[:-1] == [int(iv["start"]) for iv in ivs[1:]]  # contiguous pieces
    alpha, coeffs = tables.rsqrt_table(F)
    assert [int(v) for v in alpha] == want_alpha
    assert [[int(v) for v in row] for row in coeffs] == want


def test_rsqrt_adjustment_is_a_floor_shift():
    # adj = a0 - (a1 * offset >> f) with the arithmetic (floor) shift of the
    # reference's __int128: a negative product rounds down.
    a0, a1, off = 32768, -45, 5
    assert a0 - ((a1 * off) >> F) == 32768 - (-1)
    assert a0 - ((-a1 * off) >> F) == 32768
