"""Softmax block (RowMaxDiff + nExp + row sum + Recip + normalise) and
LayerNorm (mean, variance, Rsqrt, normalise) for two parties on one GPU.

Share level: each stage's shares equal the composition of the CPU oracle's
protocol steps (interval LUT, Beaver, truncation gate) on the same dealer
material (tests/twoparty_oracle.py).  Reconstruction: equals the fixed-point
closed forms of oracle/fixed_point.py, at small shapes and at the full
config shapes (12 x 128 causal score rows; 128 x 768).
"""
import os
import sys

import numpy as np
import pytest
import torch

import oracle_lib as ol
import twoparty_oracle as tp
from gpu_util import dev, say, u64
from suf_amd import layernorm, native, pfss, softmax, tables

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "oracle"))
import fixed_point as fp  # noqa: E402

pytestmark = pytest.mark.gpu

STATE = ol.mt64_bytes(3, ol.PRG_STATE_BYTES).tobytes()
F = 12


@pytest.fixture(scope="module", autouse=True)
def _init():
    native.call("sufhip_init", 0)


def _share(x, seed):
    x = np.asarray(x).astype(np.uint64)
    x0 = pfss.host_mt19937_64(seed, x.size)
    return x0, (x - x0).astype(np.uint64)


def _pair_dev(x0, x1):
    return dev(x0), dev(x1)


def _scores(offsets, seed, sigma=2.0):
    return pfss.host_normal_fixed(seed, sigma, 0.0, F, int(offsets[-1]))


def _recon(p):
    return (u64(p[0]) + u64(p[1])).astype(np.uint64)


def test_max_tree_plan_covers_rows():
    offs = np.array([0, 1, 4, 11, 11 + 64], dtype=np.int64)
    rounds, max_pos = softmax.max_tree_plan(offs)
    assert len(rounds) == 6 and len(max_pos) == 4


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("offsets", [
    np.array([0, 1, 3, 6, 13, 13 + 128, 13 + 128 + 65, 13 + 128 + 65 + 1000], dtype=np.int64),
    softmax.causal_offsets(2, 16),
    # Longest rows 300 and 512: two rows and one row per workgroup in the
    # one-launch tree; 7 rows leave a partial group.
    np.cumsum([0, 1, 2, 3, 300, 5, 64, 7]).astype(np.int64),
    np.cumsum([0, 512, 1, 33]).astype(np.int64),
])
def test_row_max_diff_shares(offsets, fused):
    x = _scores(offsets, 21)
    x[0] = np.uint64(1 << 63)  # most negative value in its own row
    x0, x1 = _share(x, 22)
    say("row max diff n=%d rows=%d" % (offsets[-1], len(offsets) - 1))
    rm = softmax.RowMaxDiff(offsets, softmax.Dealer(5))
    delta = tuple(torch.empty(int(offsets[-1]), dtype=torch.int64, device="cuda")
                  for _ in range(2))
    rm.eval2(_pair_dev(x0, x1), delta, fused=fused)
    g = [u64(delta[0]), u64(delta[1])]
    o = tp.relu_rounds2(rm, [x0, x1])
    assert np.array_equal(g[0], o[0]) and np.array_equal(g[1], o[1])
    want = fp.row_max_diff(x, offsets).view(np.uint64)
    assert np.array_equal((g[0] + g[1]).astype(np.uint64), want)


@pytest.mark.parametrize("fused", [True, False])
def test_row_max_diff_per_party_keystreams(fused):
    """Party 1's round keys with another keystream nonce (one bit flipped in
    its blob, on the host and the device copy): the kernels find the two
    blobs different and run one keystream per party; each party's shares
    still equal the oracle's evaluation of its own blob.  (The two shares no
    longer reconstruct the row maximum, as with any two unrelated blobs.)"""
    offsets = np.cumsum([0, 1, 2, 3, 300, 5, 64, 7, 128, 17]).astype(np.int64)
    x = _scores(offsets, 23)
    x0, x1 = _share(x, 24)
    say("row max diff, one keystream per party, n=%d fused=%s" % (offsets[-1], fused))
    rm = softmax.RowMaxDiff(offsets, softmax.Dealer(6))
    for rd in rm.rounds:
        lut = rd["lut"]
        lut.blobs[1] = lut.blobs[1].copy()
        lut.blobs[1][16] ^= 1
        lut.keys[1][16] ^= 1
    delta = tuple(torch.empty(int(offsets[-1]), dtype=torch.int64, device="cuda")
                  for _ in range(2))
    rm.eval2(_pair_dev(x0, x1), delta, fused=fused)
    g = [u64(delta[0]), u64(delta[1])]
    o = tp.relu_rounds2(rm, [x0, x1])
    assert np.array_equal(g[0], o[0]) and np.array_equal(g[1], o[1])


def test_recip_shares_and_closed_form():
    n = 300
    s = (np.arange(n, dtype=np.int64) * 1499 + 4096) % (200 << F)
    s[:5] = [0, 1, 4096, (64 << F) - 1, 1024 << F]
    s = s.astype(np.uint64)
    s0, s1 = _share(s, 31)
    say("recip n=%d" % n)
    d = softmax.Dealer(9)
    rc = softmax.Recip(n, d, STATE, F)
    t = torch.cuda.current_stream()
    for tr in rc.truncs():
        tr.prepare()
    shat = dev((s + np.uint64(rc.lut.mask)).astype(np.uint64))
    out = rc.eval2(_pair_dev(s0, s1), shat)
    t.synchronize()
    g = [u64(out[0]), u64(out[1])]
    prg = ol.Prg(STATE)
    o = tp.recip2(prg, rc, [s0, s1], u64(shat))
    assert np.array_equal(g[0], o[0]) and np.array_equal(g[1], o[1])
    want = fp.recip_task(rc.table[0], rc.table[1], s, F).view(np.uint64)
    assert np.array_equal((g[0] + g[1]).astype(np.uint64), want)


@pytest.mark.parametrize("fused", [True, False])
def test_recip_chain_fused_and_by_rounds(fused):
    """The one-launch chain and the round-by-round path (LUT opened in its
    own launch) give the oracle's shares."""
    n = 257
    s = ((np.arange(n, dtype=np.int64) * 7919 + 4096) % (300 << F)).astype(np.uint64)
    s0, s1 = _share(s, 32)
    say("recip chain fused=%s n=%d" % (fused, n))
    rc = softmax.Recip(n, softmax.Dealer(19), STATE, F)
    for tr in rc.truncs():
        tr.prepare()
    out = rc.eval2(_pair_dev(s0, s1), None, fused=fused)
    g = [u64(out[0]), u64(out[1])]
    shat = (s + np.uint64(rc.lut.mask)).astype(np.uint64)
    o = tp.recip2(ol.Prg(STATE), rc, [s0, s1], shat)
    assert np.array_equal(g[0], o[0]) and np.array_equal(g[1], o[1])


@pytest.mark.parametrize("fused", [True, False])
def test_rsqrt_chain_fused_and_by_rounds(fused):
    from suf_amd.tasks import operand, term
    n = 300
    v = ((np.arange(n, dtype=np.int64) * 613 + 3) % (17 << F)).astype(np.uint64)
    v0, v1 = _share(v, 42)
    say("rsqrt chain fused=%s n=%d" % (fused, n))
    rs = layernorm.Rsqrt(n, softmax.Dealer(20), STATE, F)
    for tr in rs.truncs():
        tr.prepare()
    eps = 4
    vp = _pair_dev(v0, v1)
    out = rs.eval2(operand(term(vp), const=eps), None, fused=fused)
    g = [u64(out[0]), u64(out[1])]
    ve = [(v0 + np.uint64(eps)).astype(np.uint64), v1]
    o = tp.rsqrt2(ol.Prg(STATE), rs, ve, tp.open2(ve, rs.lut.mask))
    assert np.array_equal(g[0], o[0]) and np.array_equal(g[1], o[1])
    want = fp.rsqrt_task(rs.table[0], rs.table[1], (v + np.uint64(eps)).astype(np.uint64), F)
    assert np.array_equal((g[0] + g[1]).astype(np.uint64), want.view(np.uint64))


def test_rsqrt_shares_and_closed_form():
    n = 200
    v = (np.arange(n, dtype=np.int64) * 331 + 1) % (20 << F)
    v[:4] = [0, 3, 4, 16 << F]
    v = v.astype(np.uint64)
    v0, v1 = _share(v, 41)
    say("rsqrt n=%d" % n)
    rs = layernorm.Rsqrt(n, softmax.Dealer(10), STATE, F)
    for tr in rs.truncs():
        tr.prepare()
    vp = _pair_dev(v0, v1)
    vhat = dev((v + np.uint64(rs.lut.mask)).astype(np.uint64))
    from suf_amd.tasks import operand, term
    out = rs.eval2(operand(term(vp)), vhat)
    g = [u64(out[0]), u64(out[1])]
    prg = ol.Prg(STATE)
    o = tp.rsqrt2(prg, rs, [v0, v1], u64(vhat))
    assert np.array_equal(g[0], o[0]) and np.array_equal(g[1], o[1])
    want = fp.rsqrt_task(rs.table[0], rs.table[1], v, F).view(np.uint64)
    assert np.array_equal((g[0] + g[1]).astype(np.uint64), want)


@pytest.mark.parametrize("heads,seq", [(1, 8), (2, 33)])
@pytest.mark.parametrize("fused", [True, False])
def test_softmax_block_small(heads, seq, fused):
    offs = softmax.causal_offsets(heads, seq)
    n = int(offs[-1])
    x = _scores(offs, 50 + seq)
    x0, x1 = _share(x, 51)
    say("softmax block heads=%d seq=%d n=%d fused=%s" % (heads, seq, n, fused))
    sm = softmax.SoftmaxBlock(offs, STATE, F, seed=13)
    out = tuple(torch.empty(n, dtype=torch.int64, device="cuda") for _ in range(2))
    sm.eval2(_pair_dev(x0, x1), out, fused=fused)
    prob, st = fp.softmax_block(x, offs, sm.nexp_table, sm.recip.table, F)
    if not fused:  # the one-launch block keeps its intermediates on chip
        assert np.array_equal(_recon(sm.delta), st["delta"].view(np.uint64))
        assert np.array_equal(_recon(sm.e), st["exp"].view(np.uint64))
        assert np.array_equal(_recon(sm.s), st["sum"].view(np.uint64))
    assert np.array_equal(_recon(out), prob.view(np.uint64))
    # Share level: the whole chain on the oracle.
    o, st2 = tp.softmax2(ol.Prg(STATE), sm, [x0, x1])
    if not fused:
        for k, dv in (("delta", sm.delta), ("exp", sm.e), ("sum", sm.s)):
            assert np.array_equal(u64(dv[0]), st2[k][0]) and np.array_equal(u64(dv[1]),
                                                                            st2[k][1])
    g = [u64(out[0]), u64(out[1])]
    assert np.array_equal(g[0], o[0]) and np.array_equal(g[1], o[1])


@pytest.mark.parametrize("lens", [[1, 2, 3, 300, 5, 64, 7], [200, 1, 33], [512, 2]])
def test_softmax_block_ragged_rows_fused(lens):
    """Ragged rows through the one-launch block (rows up to 300 / 200 / 512:
    one, two or four rows per workgroup, 8 or 4 elements per lane): shares
    equal the launch-by-launch path's and the oracle's."""
    offs = np.cumsum([0] + lens).astype(np.int64)
    n = int(offs[-1])
    x = _scores(offs, 70 + len(lens))
    x0, x1 = _share(x, 71)
    say("softmax block ragged rows %s" % (lens,))
    sm = softmax.SoftmaxBlock(offs, STATE, F, seed=17)
    outs = []
    for fused in (True, False):
        out = tuple(torch.empty(n, dtype=torch.int64, device="cuda") for _ in range(2))
        sm.eval2(_pair_dev(x0, x1), out, fused=fused)
        outs.append((u64(out[0]), u64(out[1])))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    prob, _ = fp.softmax_block(x, offs, sm.nexp_table, sm.recip.table, F)
    assert np.array_equal((outs[0][0] + outs[0][1]).astype(np.uint64), prob.view(np.uint64))


def test_softmax_block_config_shape_twice():
    offs = softmax.causal_offsets(12, 128)
    n = int(offs[-1])
    assert n == 99072
    x = _scores(offs, 11)
    x0, x1 = _share(x, 111)
    say("softmax block config shape n=%d" % n)
    sm = softmax.SoftmaxBlock(offs, STATE, F, seed=11)
    prob, st = fp.softmax_block(x, offs, sm.nexp_table, sm.recip.table, F)
    xin = _pair_dev(x0, x1)
    out = tuple(torch.empty(n, dtype=torch.int64, device="cuda") for _ in range(2))
    for _ in range(2):  # scratch and keys are reused across calls
        sm.eval2(xin, out)
        assert np.array_equal(_recon(out), prob.view(np.uint64))


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("rows,cols", [(4, 96), (3, 1100)])
def test_layernorm_small_shares(rows, cols, fused):
    """The one-launch block and the launch-per-step path give the oracle's
    shares (cols 1100: five elements per thread, a partial last one)."""
    x = pfss.host_normal_fixed(60, 1.0, 0.0, F, rows * cols)
    x[:cols] = x[:cols] * np.uint64(3)  # a wider row
    x0, x1 = _share(x, 61)
    say("layernorm %dx%d fused=%s" % (rows, cols, fused))
    ln = layernorm.LayerNormBlock(rows, cols, STATE, F, seed=14)
    out = tuple(torch.empty(rows * cols, dtype=torch.int64, device="cuda") for _ in range(2))
    ln.eval2(_pair_dev(x0, x1), out, fused=fused)
    y, st = fp.layernorm(x, rows, cols, F, ln.inv_len, ln.eps_q, ln.rsqrt.table)
    if not fused:  # the block launch keeps its intermediates in registers
        assert np.array_equal(_recon(ln.mu), st["mu"].view(np.uint64))
        assert np.array_equal(_recon(ln.var), st["var"].view(np.uint64))
    assert np.array_equal(_recon(out), y.view(np.uint64))
    # Share level: the whole chain on the oracle.
    o = tp.layernorm2(ol.Prg(STATE), ln, [x0, x1])
    g = [u64(out[0]), u64(out[1])]
    assert np.array_equal(g[0], o[0]) and np.array_equal(g[1], o[1])


def test_layernorm_config_shape_twice():
    rows, cols = 128, 768
    x = pfss.host_normal_fixed(12, 1.0, 0.0, F, rows * cols)
    x0, x1 = _share(x, 121)
    say("layernorm config shape %dx%d" % (rows, cols))
    ln = layernorm.LayerNormBlock(rows, cols, STATE, F, seed=12)
    y, _ = fp.layernorm(x, rows, cols, F, ln.inv_len, ln.eps_q, ln.rsqrt.table)
    xin = _pair_dev(x0, x1)
    out = tuple(torch.empty(rows * cols, dtype=torch.int64, device="cuda") for _ in range(2))
    shares = []
    for fused in (True, True, False):
        ln.eval2(xin, out, fused=fused)
        assert np.array_equal(_recon(out), y.view(np.uint64))
        shares.append((u64(out[0]), u64(out[1])))
    for g in shares[1:]:
        assert np.array_equal(g[0], shares[0][0]) and np.array_equal(g[1], shares[0][1])


def test_layernorm_block_rejects_wide_rows():
    ln = layernorm.LayerNormBlock(2, 8, STATE, F, seed=15)
    x = tuple(torch.zeros(16, dtype=torch.int64, device="cuda") for _ in range(2))
    out = tuple(torch.empty(16, dtype=torch.int64, device="cuda") for _ in range(2))
    a = ln.block_args(x, out)
    a.cols = 4096
    with pytest.raises(native.SufHipError):
        native.call("sufhip_layernorm2", native.ctypes.byref(a), None)
    a.cols, a.rsqrt.kind = 8, native.CHAIN_RECIP
    with pytest.raises(native.SufHipError):
        native.call("sufhip_layernorm2", native.ctypes.byref(a), None)


def test_lin2_and_row_sum2_bounds():
    """Row-indexed terms clamp their index; invalid operand descriptions are
    rejected on the host."""
    from suf_amd.tasks import lin2, operand, term
    n = 64
    a = (dev(np.arange(n, dtype=np.int64)), dev(np.arange(n, dtype=np.int64) * 2))
    idx = dev(np.array([0, 1, 2, 1000, -5] + [3] * (n - 5), dtype=np.int32))
    rowv = (dev(np.array([10, 20, 30, 40], dtype=np.int64)),
            dev(np.array([1, 2, 3, 4], dtype=np.int64)))
    out = tuple(torch.empty(n, dtype=torch.int64, device="cuda") for _ in range(2))
    say("lin2 clamp")
    lin2(operand(term(a), term(rowv, index=idx, shift=1, neg=True), const=7), n, out=out)
    g0 = u64(out[0]).astype(np.int64)
    ii = np.clip(np.array([0, 1, 2, 1000, -5] + [3] * (n - 5)), 0, 3)
    assert np.array_equal(g0, np.arange(n) - 2 * np.array([10, 20, 30, 40])[ii] + 7)
    bad = term(a)
    bad.len = n - 1
    with pytest.raises(native.SufHipError):
        lin2(operand(bad), n, out=out)
    with pytest.raises(native.SufHipError):
        lin2(operand(term(a, stride=2, off=2)), n, out=out)


def test_softmax_block_rejects_indexed_nexp_triples():
    """The one-launch block reads the nExp triples through plain pointers;
    a triple share with a row index (or a shift, multiplier, negation or a
    stride other than 1 or 3) is refused on the host before any launch."""
    offs = softmax.causal_offsets(1, 8)
    n = int(offs[-1])
    sm = softmax.SoftmaxBlock(offs, STATE, F, seed=13)
    for tr in sm.truncs():
        tr.prepare()
    x = _pair_dev(*_share(_scores(offs, 5), 6))
    out = tuple(torch.empty(n, dtype=torch.int64, device="cuda") for _ in range(2))
    a = sm.block_args(softmax.operand(softmax.term(x)), out)
    idx = torch.zeros(n, dtype=torch.int32, device="cuda")
    a.nexp.a[0].index = idx.data_ptr()
    with pytest.raises(native.SufHipError, match="plain arrays"):
        native.call("sufhip_softmax2", native.ctypes.byref(a), 0)


@pytest.mark.parametrize("kind", ["recip", "rsqrt"])
def test_chain_wide_form_matches_oracle(kind):
    """Batches of at least two passes of 1024-lane workgroups over every CU
    take the chain kernel's four-table form (one workgroup per CU); the
    shares equal the oracle's, with a partial last pass, under either
    keystream policy."""
    from suf_amd.tasks import operand, term
    n = 2 * 256 * 1024 + 333
    v = ((np.arange(n, dtype=np.int64) * 613 + 3) % (17 << F)).astype(np.uint64)
    v0, v1 = _share(v, 43)
    say("%s chain, wide form, n=%d" % (kind, n))
    if kind == "recip":
        g = softmax.Recip(n, softmax.Dealer(21), STATE, F)
    else:
        g = layernorm.Rsqrt(n, softmax.Dealer(22), STATE, F)
    for tr in g.truncs():
        tr.prepare()
    vp = _pair_dev(v0, v1)
    outs = []
    for per_party in (False, True):
        with pfss.keystream_per_party(per_party):
            if kind == "recip":
                out = g.eval2(vp, None, fused=True)
            else:
                out = g.eval2(operand(term(vp)), None, fused=True)
        outs.append([u64(out[0]), u64(out[1])])
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    if kind == "recip":
        o = tp.recip2(ol.Prg(STATE), g, [v0, v1], (v + np.uint64(g.lut.mask)).astype(np.uint64))
    else:
        o = tp.rsqrt2(ol.Prg(STATE), g, [v0, v1], tp.open2([v0, v1], g.lut.mask))
    assert np.array_equal(outs[0][0], o[0]) and np.array_equal(outs[0][1], o[1])
