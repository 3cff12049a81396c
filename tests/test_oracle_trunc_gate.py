"""Oracle truncation gate (composite_gen_trunc_gate + AddU64 eval + postproc)
pinned by its two-party reconstruction: x >> f for FaithfulTR, the arithmetic
shift for FaithfulARS, and the arithmetic shift under the gap |x| < 2^62 for
GapARS (include/gates/composite_fss.hpp:645-833,1385-1638,
include/gates/postproc_hooks.hpp:172-373)."""
import numpy as np
import pytest

import oracle_lib as ol

PRG = ol.Prg(ol.mt64_bytes(3, 128).tobytes())
M64 = (1 << 64) - 1


def signed(v):
    v = int(v) & M64
    return v - (1 << 64) if v >> 63 else v


def expected(kind, f, x):
    if kind == ol.TRUNC_TR:
        return (int(x) & M64) >> f
    return (signed(x) >> f) & M64


def x_cases(kind, f, rng, n_rand):
    lim = 1 << 62
    edge = [0, 1, -1, (1 << f) - 1, -(1 << f), (1 << f), -(1 << f) - 1, lim - 1, -lim,
            12345 << f, -(777 << f) + 3]
    if kind != ol.TRUNC_GAPARS:
        edge += [(1 << 63) - 1, -(1 << 63), M64, 1 << 63]
        rnd = [int(v) for v in rng.integers(0, 1 << 63, n_rand, dtype=np.uint64)]
        rnd = [v if i % 2 else v | (1 << 63) for i, v in enumerate(rnd)]
    else:
        edge = [v for v in edge if -lim <= v < lim]
        rnd = [int(v) - lim for v in rng.integers(0, 1 << 63, n_rand, dtype=np.uint64)]
    return [v & M64 for v in edge + rnd]


def r_cases(f, rng):
    lo = (1 << f) - 1
    base = [int(v) for v in rng.integers(0, 1 << 63, 4, dtype=np.uint64)]
    return [base[0], base[1] | (1 << 63), base[2] & ~lo,            # r_low == 0
            (base[3] & ~lo) | (1 << 63), 0, M64, 1 << 63, lo]


def run_gate(kind, f, r, xs, rng):
    rnd = rng.integers(0, 1 << 64, ol.TRUNC_RAND_WORDS, dtype=np.uint64)
    rnd[0] = np.uint64(r)
    k0, k1 = ol.trunc_gen(PRG, kind, f, rnd)
    xhat = np.array([(x + r) & M64 for x in xs], dtype=np.uint64)
    y0 = ol.trunc_eval(PRG, kind, f, k0, xhat)
    y1 = ol.trunc_eval(PRG, kind, f, k1, xhat)
    return k0, k1, y0, y1


@pytest.mark.parametrize("kind,f,n_rand", [
    (ol.TRUNC_GAPARS, 12, 200), (ol.TRUNC_GAPARS, 24, 60), (ol.TRUNC_GAPARS, 1, 40),
    (ol.TRUNC_GAPARS, 62, 20), (ol.TRUNC_TR, 12, 12), (ol.TRUNC_TR, 24, 6),
    (ol.TRUNC_ARS, 12, 12), (ol.TRUNC_ARS, 7, 6)])
def test_reconstruction_closed_form(kind, f, n_rand):
    rng = np.random.default_rng(1000 * kind + f)
    for r in r_cases(f, rng):
        xs = x_cases(kind, f, rng, n_rand)
        _, _, y0, y1 = run_gate(kind, f, r, xs, rng)
        got = [(int(a) + int(b)) & M64 for a, b in zip(y0, y1)]
        want = [expected(kind, f, x) for x in xs]
        bad = [(hex(x), hex(g), hex(w)) for x, g, w in zip(xs, got, want) if g != w]
        assert not bad, (kind, f, hex(r), bad[:4])


def test_gapars_fails_outside_gap():
    # The gap condition is real: for x = 2^63 - 2^f (outside [-2^62, 2^62))
    # and a mask r = 2^63 - 1, x + 2^62 + r wraps while MSB(r) = 0, so the
    # GapARS correction is missing and the result is off by 2^(64-f) -- the
    # closed-form checks above can tell GapARS from a faithful shift.
    rng = np.random.default_rng(7)
    f = 12
    x = (1 << 63) - (1 << f)
    _, _, y0, y1 = run_gate(ol.TRUNC_GAPARS, f, (1 << 63) - 1, [x], rng)
    got = (int(y0[0]) + int(y1[0])) & M64
    assert (got - expected(ol.TRUNC_GAPARS, f, x)) & M64 == (1 << 64) - (1 << (64 - f))


def test_blob_layout_and_shares():
    rng = np.random.default_rng(3)
    f = 12
    for kind in (ol.TRUNC_TR, ol.TRUNC_ARS, ol.TRUNC_GAPARS):
        r = int(rng.integers(1, 1 << 63)) | 1  # r_low != 0
        rnd = rng.integers(0, 1 << 64, ol.TRUNC_RAND_WORDS, dtype=np.uint64)
        rnd[0] = np.uint64(r)
        k0, k1 = ol.trunc_gen(PRG, kind, f, rnd)
        kb = ol.trunc_key_bytes(kind, f)
        assert k0.size == kb and kb % 8 == 0
        w0 = k0[:64].view(np.uint64)
        w1 = k1[:64].view(np.uint64)
        assert bytes(k0[:4]) == b"STG1" and k0[4] == kind and k0[5] == f
        assert k0[6] == 0 and k1[6] == 1
        flags = 1 | (2 if kind != ol.TRUNC_GAPARS else 0) | (4 if kind == ol.TRUNC_ARS else 0)
        assert k0[7] == flags == k1[7]
        add = lambda i: (int(w0[i]) + int(w1[i])) & M64
        assert add(1) == r                      # r_in
        assert add(2) == r >> f                 # r_hi
        assert add(3) == 0                      # r_out is zero-sum
        assert add(4) == 1                      # carry rotation wrap bit
        if kind == ol.TRUNC_ARS:
            assert add(5) == (1 if r < (1 << 63) else 0)
        if kind == ol.TRUNC_GAPARS:
            assert add(6) == ((1 << (64 - f)) if r >> 63 else 0)
        # The carry DCF key (f bits, alpha = r_low) reconstructs 1[x < r_low].
        ckb = ol.myl7_key_bytes(f, 8)
        for x in (0, (r & 0xfff) - 1, r & 0xfff, 0xfff):
            if x < 0:
                continue
            s0 = ol.myl7_eval(PRG, ol.GROUP_ADD, f, k0[64:64 + ckb], x, 8).view(np.uint64)[0]
            s1 = ol.myl7_eval(PRG, ol.GROUP_ADD, f, k1[64:64 + ckb], x, 8).view(np.uint64)[0]
            assert (int(s0) + int(s1)) & M64 == int(x < (r & 0xfff))


def test_no_carry_key_when_low_bits_of_mask_are_zero():
    rng = np.random.default_rng(5)
    f = 12
    r = int(rng.integers(0, 1 << 52)) << f
    k0, k1, y0, y1 = run_gate(ol.TRUNC_GAPARS, f, r, [5, -5 & M64], rng)
    assert k0[7] & 1 == 0 and not k0[64:].any()
    assert [(int(a) + int(b)) & M64 for a, b in zip(y0, y1)] == [0, (-1) & M64]
