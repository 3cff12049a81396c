"""GPU parity of the ring postprocessing / Beaver / row-reduction / packing
kernels (libsuf_hip.so, called through the C ABI) with the oracle."""
import numpy as np
import pytest
import torch

import oracle_lib as ol
from gpu_util import Pins, dev, say, u64
from suf_amd import native

pytestmark = pytest.mark.gpu

M64 = (1 << 64) - 1


@pytest.fixture(scope="module", autouse=True)
def _init():
    native.call("sufhip_init", 0)


def S():
    return torch.cuda.current_stream().cuda_stream


def rng_u64(rng, n):
    return rng.integers(0, 2**63, size=n, dtype=np.uint64) * np.uint64(2) + \
        rng.integers(0, 2, size=n, dtype=np.uint64)


def empty(n):
    return torch.empty(max(n, 1), dtype=torch.int64, device="cuda")


@pytest.mark.parametrize("n", [1, 255, 100003])
@pytest.mark.parametrize("party", [0, 1])
def test_beaver_mul(n, party):
    P = Pins()
    say("beaver_mul n=%d party=%d" % (n, party))
    rng = np.random.default_rng(n + party)
    a, b, c, d, e = (rng_u64(rng, n) for _ in range(5))
    out = empty(n)
    native.call("sufhip_beaver_mul", party, None, None, *[P(v) for v in (a, b, c, d, e)],
                out.data_ptr(), n, S())
    assert np.array_equal(u64(out)[:n], ol.beaver_mul(party, a, b, c, d, e))
    trip = np.stack([a, b, c], axis=1).ravel()
    out2 = empty(n)
    native.call("sufhip_beaver_mul_aos", party, P(trip), P(d),
                P(e), out2.data_ptr(), n, S())
    assert np.array_equal(u64(out2)[:n], ol.beaver_mul(party, a, b, c, d, e))


@pytest.mark.parametrize("f", [0, 1, 12, 24, 63, 64])
def test_trunc_shift(f):
    P = Pins()
    rng = np.random.default_rng(f)
    x = rng_u64(rng, 5000)
    out = empty(5000)
    native.call("sufhip_trunc_shift", P(x), out.data_ptr(), f, 5000, S())
    exp = x >> np.uint64(f) if 0 < f < 64 else (x if f <= 0 else np.zeros_like(x))
    assert np.array_equal(u64(out), exp)


@pytest.mark.parametrize("gapars", [0, 1])
@pytest.mark.parametrize("f", [0, 8, 12, 24, 62, 63])
@pytest.mark.parametrize("party", [0, 1])
def test_trunc_postproc_matches_oracle(gapars, f, party):
    P = Pins()
    say("trunc_postproc gapars=%d f=%d party=%d" % (gapars, f, party))
    rng = np.random.default_rng(100 * gapars + f + 7 * party)
    n = 3001
    hatx = rng_u64(rng, n)
    ar_stride, ar_idx = 3, 2
    arith = rng_u64(rng, n * ar_stride)
    b_stride = 4
    bools = rng.integers(0, 2, size=n * b_stride).astype(np.uint64)
    r_hi, m = int(rng_u64(rng, 1)[0]), int(rng_u64(rng, 1)[0])
    for (ci, si, wi) in ((0, 1, 2), (3, -1, 1), (-1, -1, -1), (5, 0, 9)):
        out = empty(n)
        native.call("sufhip_trunc_postproc", party, gapars, f, r_hi, m, P(hatx),
                    P(arith), ar_stride, ar_idx, P(bools), b_stride, ci,
                    si, wi, out.data_ptr(), n, S())
        exp = ol.trunc_postproc(party, gapars, f, r_hi, m, hatx, arith, ar_stride, ar_idx, bools,
                                b_stride, ci, si, wi, n)
        assert np.array_equal(u64(out), exp), (ci, si, wi)
    # no bools at all
    out = empty(n)
    native.call("sufhip_trunc_postproc", party, gapars, f, r_hi, m, P(hatx),
                P(arith), ar_stride, ar_idx, None, 0, 0, 1, 2, out.data_ptr(), n, S())
    exp = ol.trunc_postproc(party, gapars, f, r_hi, m, hatx, arith, ar_stride, ar_idx, None, 0,
                            0, 1, 2, n)
    assert np.array_equal(u64(out), exp)


def test_trunc_gapars_full_size_reconstruction():
    """2^20 elements, both parties, GapARS f=12: reconstructs v >> 12."""
    P = Pins()
    say("trunc gapars full size")
    rng = np.random.default_rng(12)
    n, f = 1 << 20, 12
    mag = rng.integers(0, 2**61, size=n, dtype=np.int64)
    v = np.where(rng.integers(0, 2, size=n) == 1, -mag, mag)
    r = int(rng_u64(rng, 1)[0]) | (1 << 63)
    xb = v.view(np.uint64) + np.uint64(1 << 62)
    hatx = v.view(np.uint64) + np.uint64(r)
    lm = np.uint64((1 << f) - 1)
    carry = (((xb & lm) + (np.uint64(r) & lm)) >> np.uint64(f)).astype(np.uint64)
    c0 = rng_u64(rng, n)
    c1 = carry - c0
    b0 = rng_u64(rng, n)
    b1 = np.zeros(n, np.uint64) - b0
    rh0 = int(rng_u64(rng, 1)[0])
    rh1 = ((r >> f) - rh0) & M64
    m = 1 << (64 - f)
    m0 = int(rng_u64(rng, 1)[0])
    m1 = (m - m0) & M64
    outs = []
    hd = dev(hatx)
    for p, (b, c, rh, mm) in enumerate(((b0, c0, rh0, m0), (b1, c1, rh1, m1))):
        o = empty(n)
        native.call("sufhip_trunc_postproc", p, 1, f, rh, mm, hd.data_ptr(), P(b), 1,
                    0, P(c), 1, 0, -1, -1, o.data_ptr(), n, S())
        outs.append(u64(o))
    assert np.array_equal((outs[0] + outs[1]).view(np.int64), v >> f)


def test_horner():
    P = Pins()
    rng = np.random.default_rng(2024)
    n = 70001
    vals = [rng_u64(rng, n) for _ in range(5)]
    out = empty(n)
    native.call("sufhip_horner_cubic", *[P(v) for v in vals], out.data_ptr(), n, S())
    assert np.array_equal(u64(out), ol.horner(*vals))


@pytest.mark.parametrize("out_words,rw", [(4, 4), (5, 3), (1, 1), (16, 16), (8, 8)])
def test_add_rout(out_words, rw):
    P = Pins()
    rng = np.random.default_rng(out_words)
    elems = 9999
    base = rng_u64(rng, elems * out_words)
    r = rng_u64(rng, rw)
    t = dev(base)
    rbuf = np.ascontiguousarray(r)
    native.call("sufhip_add_rout_aos", t.data_ptr(), elems, out_words, rbuf.ctypes.data, rw, S())
    assert np.array_equal(u64(t), ol.add_rout_aos(base, elems, out_words, r))


@pytest.mark.parametrize("rows,cols,ragged", [(1536, 128, True), (128, 768, False), (3, 1, True)])
def test_row_ops(rows, cols, ragged):
    P = Pins()
    say("row ops %dx%d ragged=%s" % (rows, cols, ragged))
    rng = np.random.default_rng(rows + cols)
    n = rows * cols
    mat = rng_u64(rng, n)
    lens = (np.arange(rows) % cols + 1).astype(np.int32) if ragged else None
    dl = P(lens) if ragged else None
    dm = dev(mat)
    outs = {}
    for name in ("sufhip_row_sum", "sufhip_row_mean"):
        o = empty(rows)
        native.call(name, dm.data_ptr(), rows, cols, dl, o.data_ptr(), S())
        outs[name] = u64(o)[:rows]
    assert np.array_equal(outs["sufhip_row_sum"], ol.row_sum(mat, rows, cols, lens))
    mu = ol.row_mean(mat, rows, cols, lens)
    assert np.array_equal(outs["sufhip_row_mean"], mu)
    o = empty(rows)
    native.call("sufhip_row_variance", dm.data_ptr(), P(mu), rows, cols, dl,
                o.data_ptr(), S())
    assert np.array_equal(u64(o)[:rows], ol.row_variance(mat, mu, rows, cols, lens))
    # row-broadcast Beaver
    A, C, d = (rng_u64(rng, n) for _ in range(3))
    B, e = rng_u64(rng, rows), rng_u64(rng, rows)
    for party in (0, 1):
        o = empty(n)
        native.call("sufhip_row_broadcast_mul", party, P(A), P(B),
                    P(C), P(d), P(e), rows, cols, dl,
                    o.data_ptr(), n, S())
        assert np.array_equal(u64(o)[:n], ol.row_broadcast_mul(party, A, B, C, d, e, rows, cols,
                                                               lens))
    # ragged packed rows (softmax layout: row r holds r % cols + 1 values)
    if ragged:
        offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        vals = rng_u64(rng, int(offs[-1]))
        o = empty(rows)
        native.call("sufhip_row_sum_ragged", P(vals), P(offs), rows,
                    o.data_ptr(), S())
        assert np.array_equal(u64(o)[:rows], ol.row_sum_ragged(vals, offs))


@pytest.mark.parametrize("eff_bits", [1, 5, 12, 17, 37, 50, 63, 64])
@pytest.mark.parametrize("n", [1, 64, 1000, 65537])
def test_pack_unpack(eff_bits, n):
    P = Pins()
    rng = np.random.default_rng(eff_bits * 1000 + n)
    vals = rng_u64(rng, n)
    words = (n * eff_bits + 63) // 64
    packed = empty(words)
    native.call("sufhip_pack_eff_bits", P(vals), eff_bits, packed.data_ptr(), n, S())
    assert np.array_equal(u64(packed)[:words], ol.pack_eff_bits(vals, eff_bits))
    back = empty(n)
    native.call("sufhip_unpack_eff_bits", packed.data_ptr(), eff_bits, back.data_ptr(), n, S())
    mask = np.uint64((1 << eff_bits) - 1) if eff_bits < 64 else np.uint64(M64)
    assert np.array_equal(u64(back)[:n], vals & mask)


@pytest.mark.parametrize("ring_bits", [37, 50, 64])
@pytest.mark.parametrize("eff_bits", [37, 50, 64])
def test_open_add(ring_bits, eff_bits):
    P = Pins()
    rng = np.random.default_rng(ring_bits + 3 * eff_bits)
    n = 20001
    local = rng_u64(rng, n)
    remote = rng_u64(rng, n)
    if eff_bits < 64:
        remote &= np.uint64((1 << eff_bits) - 1)
    packed = ol.pack_eff_bits(remote, eff_bits) if eff_bits < 64 else remote
    rmask = (1 << ring_bits) - 1 if ring_bits < 64 else M64
    dlo, dpk = dev(local), dev(packed)
    o = empty(n)
    native.call("sufhip_unpack_add_to_signed", dlo.data_ptr(), dpk.data_ptr(), eff_bits,
                o.data_ptr(), n, ring_bits, rmask, S())
    assert np.array_equal(u64(o), ol.open_add(local, packed, eff_bits, n, ring_bits, rmask, 1))
    native.call("sufhip_unpack_add_mod", dlo.data_ptr(), dpk.data_ptr(), eff_bits, o.data_ptr(),
                n, ring_bits, rmask, S())
    assert np.array_equal(u64(o), ol.open_add(local, packed, eff_bits, n, ring_bits, rmask, 0))
    if eff_bits == 64:
        native.call("sufhip_open_add_to_signed", dlo.data_ptr(), dpk.data_ptr(), o.data_ptr(), n,
                    ring_bits, rmask, S())
        assert np.array_equal(u64(o), ol.open_add(local, remote, 64, n, ring_bits, rmask, 1))


def test_zero_length_calls_are_noops():
    P = Pins()
    for name, args in (("sufhip_beaver_mul", (0, None, None, None, None, None, None, None, None, 0,
                                              None)),
                       ("sufhip_horner_cubic", (None,) * 6 + (0, None)),
                       ("sufhip_row_sum", (None, 0, 5, None, None, None)),
                       ("sufhip_pack_eff_bits", (None, 12, None, 0, None))):
        native.call(name, *args)
