"""GPU truncation gate (sufhip_trunc_gen / sufhip_trunc_eval) against the
oracle restatement of composite_gen_trunc_gate + the AddU64 evaluation +
postproc (byte-equal keys, equal shares) and against the closed forms of the
two-party reconstruction.  Cases cover every evaluation path: no frontier
(small batches), a partial prefix frontier, the full-domain table, the
64-bit wrap / sign keys of FaithfulTR / FaithfulARS, and masks whose low f
bits are zero (no carry key)."""
import numpy as np
import pytest
import torch

import oracle_lib as ol
from gpu_util import dev, host, say, u64
from suf_amd import native, pfss

pytestmark = pytest.mark.gpu

M64 = (1 << 64) - 1
STATE = ol.mt64_bytes(3, ol.PRG_STATE_BYTES).tobytes()
PRG = ol.Prg(STATE)


@pytest.fixture(scope="module", autouse=True)
def _init():
    native.call("sufhip_init", 0)


def _signed(v):
    v = int(v) & M64
    return v - (1 << 64) if v >> 63 else v


def _expected(kind, f, xs):
    if kind == ol.TRUNC_TR:
        return np.array([int(x) >> f for x in xs], dtype=np.uint64)
    return np.array([(_signed(x) >> f) & M64 for x in xs], dtype=np.uint64)


def _inputs(kind, f, n, rng):
    if kind == ol.TRUNC_GAPARS:
        lim = 1 << 62
        xs = [int(v) - lim for v in rng.integers(0, 1 << 63, n, dtype=np.uint64)]
        edge = [0, 1, -1, (1 << f) - 1, -(1 << f), lim - 1, -lim]
    else:
        xs = [int(v) for v in rng.integers(0, 1 << 64, n, dtype=np.uint64)]
        edge = [0, 1, M64, (1 << 63) - 1, 1 << 63]
    xs[:len(edge)] = edge[:n]
    # Small magnitudes around the fixed-point range most gates see.
    xs[len(edge):len(edge) + n // 4] = [int(v) for v in rng.integers(-(1 << 20), 1 << 20, n // 4)]
    return np.array([x & M64 for x in xs[:n]], dtype=np.uint64)


def _run(kind, f, n, r, seed, oracle_sample):
    rng = np.random.default_rng(seed)
    rnd = rng.integers(0, 1 << 64, ol.TRUNC_RAND_WORDS, dtype=np.uint64)
    rnd[0] = np.uint64(r)
    say("trunc kind=%d f=%d n=%d r=%#x frontier_bytes=%d" %
        (kind, f, n, r, native.load().sufhip_trunc_work_bytes(f, n)))
    k0, k1 = pfss.trunc_gen(kind, f, STATE, rnd)
    ok0, ok1 = ol.trunc_gen(PRG, kind, f, rnd)
    assert host(k0).tobytes() == ok0.tobytes()
    assert host(k1).tobytes() == ok1.tobytes()
    xs = _inputs(kind, f, n, rng)
    xhat = np.array([(int(x) + r) & M64 for x in xs], dtype=np.uint64)
    xd = dev(xhat)
    y0 = u64(pfss.trunc_eval(kind, f, STATE, k0, xd))
    y1 = u64(pfss.trunc_eval(kind, f, STATE, k1, xd))
    torch.cuda.synchronize()
    rec = (y0 + y1).astype(np.uint64)
    assert np.array_equal(rec, _expected(kind, f, xs)), (kind, f, n, hex(r))
    idx = np.unique(np.concatenate([np.arange(min(n, 16)),
                                    rng.integers(0, n, min(n, oracle_sample))]))
    o0 = ol.trunc_eval(PRG, kind, f, ok0, xhat[idx])
    o1 = ol.trunc_eval(PRG, kind, f, ok1, xhat[idx])
    assert np.array_equal(y0[idx], o0) and np.array_equal(y1[idx], o1)


@pytest.mark.parametrize("kind,f,n", [
    (ol.TRUNC_GAPARS, 12, 1 << 16),   # full-domain table, walked (d = f = 12)
    (ol.TRUNC_GAPARS, 24, 1 << 16),   # d = 15: walk 12 + 3 expanded levels, 9 per element
    (ol.TRUNC_GAPARS, 24, 1 << 15),   # d = 14: an even number of expanded levels
    (ol.TRUNC_GAPARS, 14, 1 << 16),   # d = f = 14: the last expanded level is final
    (ol.TRUNC_GAPARS, 12, 20),        # no frontier (d = 0)
    (ol.TRUNC_GAPARS, 30, 3000),      # d = 10, walked only
    (ol.TRUNC_GAPARS, 1, 1000),       # f = 1: table of 2 entries
    (ol.TRUNC_TR, 12, 2000),          # carry frontier + 64-bit wrap key
    (ol.TRUNC_ARS, 7, 300),           # carry, wrap and sign keys
    (ol.TRUNC_ARS, 24, 40),
])
def test_gate_matches_oracle_and_closed_form(kind, f, n):
    rng = np.random.default_rng(f * 131 + kind)
    lo = (1 << f) - 1
    for i, r in enumerate([int(rng.integers(0, 1 << 63)) | 1,
                           int(rng.integers(0, 1 << 63)) | (1 << 63),
                           int(rng.integers(0, 1 << 63)) & ~lo]):  # last: no carry key
        _run(kind, f, n, r & M64, 10 * f + i, 64 if kind == ol.TRUNC_GAPARS else 12)


def test_full_size_gapars_reconstructs():
    # 2^20 elements, f = 12 and 2f = 24 (the spline gate's two truncations).
    n = 1 << 20
    x = pfss.host_normal_fixed(5, 3.0, 8.0, 12, n)
    x3 = (x.astype(np.int64) * np.int64(4093) * np.int64(-37)).astype(np.uint64)  # Q36-ish
    for f, vals in ((12, x), (24, x3)):
        rnd = ol.mt64(100 + f, ol.TRUNC_RAND_WORDS)
        r = int(rnd[0])
        say("trunc full size f=%d" % f)
        k0, k1 = pfss.trunc_gen(native.TRUNC_GAPARS, f, STATE, rnd)
        xd = dev((vals + np.uint64(r)).astype(np.uint64))
        y0 = pfss.trunc_eval(native.TRUNC_GAPARS, f, STATE, k0, xd)
        y1 = pfss.trunc_eval(native.TRUNC_GAPARS, f, STATE, k1, xd)
        rec = u64(y0 + y1)
        assert np.array_equal(rec, (vals.view(np.int64) >> f).view(np.uint64))


def test_errors():
    rnd = np.zeros(ol.TRUNC_RAND_WORDS, dtype=np.uint64)
    with pytest.raises(native.SufHipError):
        pfss.trunc_gen(7, 12, STATE, rnd)
    with pytest.raises(native.SufHipError):
        pfss.trunc_gen(native.TRUNC_GAPARS, 63, STATE, rnd)
    k0, _ = pfss.trunc_gen(native.TRUNC_GAPARS, 12, STATE, rnd)
    xd = dev(np.arange(1 << 12, dtype=np.uint64))
    with pytest.raises(native.SufHipError):  # wrong kind for this key size
        pfss.trunc_eval(native.TRUNC_TR, 12, STATE, k0, xd)
    with pytest.raises(native.SufHipError):  # workspace too small
        pfss.trunc_eval(native.TRUNC_GAPARS, 12, STATE, k0, xd,
                        work=torch.empty(1, dtype=torch.int64, device="cuda"))
    out = pfss.trunc_eval(native.TRUNC_GAPARS, 12, STATE, k0, xd[:0])
    assert out.numel() == 0


def test_batched_prepare_matches_single_gate_path():
    # sufhip_trunc_prepare_batch (8 lanes per walk, local expansion of the
    # table gates' last levels, up to 96 jobs per walk launch) against the
    # one-gate prepare of sufhip_trunc_eval: equal shares for every gate.
    # 52 gates = 104 jobs, so the batch takes two walk launches; the shapes
    # cover tables (f <= 14, including f below the local expansion depth),
    # walked prefixes with expansion launches (f = 24, n = 2^16) and
    # walked-only prefixes.
    from suf_amd import tasks
    shapes = [(native.TRUNC_GAPARS, 12, 3000), (native.TRUNC_GAPARS, 13, 500),
              (native.TRUNC_GAPARS, 14, 700), (native.TRUNC_GAPARS, 2, 100),
              (native.TRUNC_GAPARS, 5, 64), (native.TRUNC_GAPARS, 24, 1 << 16),
              (native.TRUNC_GAPARS, 30, 3000), (native.TRUNC_TR, 12, 2000),
              (native.TRUNC_ARS, 7, 300), (native.TRUNC_ARS, 24, 40)]
    dealer = tasks.Dealer(77)
    gates = [tasks.Trunc(dealer, f, n, STATE, kind=kind)
             for i in range(52) for kind, f, n in [shapes[i % len(shapes)]]]
    say("batched prepare: %d gates" % len(gates))
    tasks.prepare_batch(gates)
    rng = np.random.default_rng(5)
    for i, g in enumerate(gates):
        xhat = rng.integers(0, 1 << 64, g.n, dtype=np.uint64)
        xd = dev(xhat)
        out = (torch.empty(g.n, dtype=torch.int64, device="cuda"),
               torch.empty(g.n, dtype=torch.int64, device="cuda"))
        g.finish(xd, out)
        for p in (0, 1):
            want = u64(pfss.trunc_eval(g.kind, g.f, STATE, g.keys[p], xd))
            assert np.array_equal(u64(out[p]), want), (i, g.kind, g.f, g.n, p)


@pytest.mark.parametrize("gates", [2, 4, 8, 16, 40])
def test_batched_prepare_every_local_depth(gates):
    """One walk launch expands E local levels, the fewest whose walks take
    less than three quarters of one full workgroup per CU: with f = 12 tables
    (two per gate) and 256 CUs, 2 / 4 / 8 / 16 / 40 gates give E = 0 / 1 / 2
    / 3 / 4.  Every gate's shares equal the one-gate path's."""
    from suf_amd import tasks
    dealer = tasks.Dealer(100 + gates)
    gs = [tasks.Trunc(dealer, 12, 256, STATE) for _ in range(gates)]
    say("batched prepare, %d gates (f = 12)" % gates)
    tasks.prepare_batch(gs)
    rng = np.random.default_rng(gates)
    for i, g in enumerate(gs):
        xd = dev(rng.integers(0, 1 << 64, g.n, dtype=np.uint64))
        out = (torch.empty(g.n, dtype=torch.int64, device="cuda"),
               torch.empty(g.n, dtype=torch.int64, device="cuda"))
        g.finish(xd, out)
        for p in (0, 1):
            want = u64(pfss.trunc_eval(g.kind, g.f, STATE, g.keys[p], xd))
            assert np.array_equal(u64(out[p]), want), (gates, i, p)
