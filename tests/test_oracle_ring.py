"""Pins the oracle's ring postprocessing against closed forms (CPU only).

Truncation is checked as the two-party protocol it serves: shares of
r_hi / carry / wrap / sign / m computed in the clear and split additively,
each party's postproc output summed, and the sum compared with x >> f
(faithful TR), the arithmetic shift (ARS) and the GapARS arithmetic shift
for |v| < 2^62 -- the closed forms of src/demo/test_truncation.cpp and
test_cuda_trunc_postproc.cpp:82-140.  Beaver products are checked by
reconstruction (z0 + z1 == x * y mod 2^64).
"""
import numpy as np
import pytest

import oracle_lib as ol

M64 = (1 << 64) - 1


def rng_u64(rng, n):
    return rng.integers(0, 2**63, size=n, dtype=np.uint64) * np.uint64(2) + \
        rng.integers(0, 2, size=n, dtype=np.uint64)


def split(rng, v):
    s0 = rng_u64(rng, len(v))
    return s0, (np.asarray(v, dtype=np.uint64) - s0)


@pytest.mark.parametrize("f", [1, 8, 12, 24, 63])
def test_faithful_trunc_and_ars_reconstruct(f):
    rng = np.random.default_rng(2025 + f)
    n = 4000
    x = rng_u64(rng, n)
    r = int(rng_u64(rng, 1)[0])
    xhat = x + np.uint64(r)
    lowmask = (1 << f) - 1
    carry = np.array([((int(a) & lowmask) + (r & lowmask)) >> f for a in x], dtype=np.uint64)
    wrap = (xhat < np.uint64(r)).astype(np.uint64)
    sign = (x >> np.uint64(63)).astype(np.uint64)
    r_hi = r >> f
    c0, c1 = split(rng, carry)
    w0, w1 = split(rng, wrap)
    s0, s1 = split(rng, sign)
    b0, b1 = split(rng, np.zeros(n, dtype=np.uint64))
    rh0 = int(rng_u64(rng, 1)[0])
    rh1 = (r_hi - rh0) & M64
    for ars in (0, 1):
        outs = []
        for p, (c, w, s, b, rh) in enumerate(((c0, w0, s0, b0, rh0), (c1, w1, s1, b1, rh1))):
            bools = np.stack([c, s, w], axis=1).ravel()
            outs.append(ol.trunc_postproc(p, 0, f, rh, 0, xhat, b, 1, 0, bools, 3, 0,
                                          1 if ars else -1, 2, n))
        got = outs[0] + outs[1]
        if ars:
            exp = (x.view(np.int64) >> np.int64(f)).view(np.uint64)
        else:
            exp = x >> np.uint64(f)
        assert np.array_equal(got, exp), (f, ars)


@pytest.mark.parametrize("f", [8, 12, 24])
def test_gapars_reconstructs_arithmetic_shift(f):
    rng = np.random.default_rng(77 + f)
    n = 4000
    mag = rng.integers(0, 2**61, size=n, dtype=np.int64)
    v = np.where(rng.integers(0, 2, size=n) == 1, -mag, mag)
    for r_msb in (0, 1):
        r = int(rng_u64(rng, 1)[0]) & ((1 << 63) - 1) | (r_msb << 63)
        xb = (v.view(np.uint64) + np.uint64(1 << 62))  # x = v + 2^62 in [0, 2^63)
        xhat = v.view(np.uint64) + np.uint64(r)
        lowmask = (1 << f) - 1
        carry = np.array([((int(a) & lowmask) + (r & lowmask)) >> f for a in xb], dtype=np.uint64)
        m = (1 << (64 - f)) if r_msb else 0
        c0, c1 = split(rng, carry)
        b0, b1 = split(rng, np.zeros(n, dtype=np.uint64))
        rh0 = int(rng_u64(rng, 1)[0])
        rh1 = ((r >> f) - rh0) & M64
        m0 = int(rng_u64(rng, 1)[0])
        m1 = (m - m0) & M64
        z0 = ol.trunc_postproc(0, 1, f, rh0, m0, xhat, b0, 1, 0, c0, 1, 0, -1, -1, n)
        z1 = ol.trunc_postproc(1, 1, f, rh1, m1, xhat, b1, 1, 0, c1, 1, 0, -1, -1, n)
        assert np.array_equal((z0 + z1).view(np.int64), v >> f), (f, r_msb)


def test_trunc_postproc_zero_base_is_shift():
    # test_cuda_trunc_postproc.cpp:48-82: party 0, carry/sign/wrap absent, base 0.
    rng = np.random.default_rng(4321)
    x = rng_u64(rng, 2048)
    out = ol.trunc_postproc(0, 0, 8, 0, 0, x, np.zeros(2048, np.uint64), 1, 0, None, 0, -1, -1,
                            -1, 2048)
    assert np.array_equal(out, x >> np.uint64(8))


def test_beaver_mul_reconstructs_product():
    rng = np.random.default_rng(1234)
    n = 5000
    x, y, a, b = (rng_u64(rng, n) for _ in range(4))
    c = a * b
    a0, a1 = split(rng, a)
    b0, b1 = split(rng, b)
    c0, c1 = split(rng, c)
    d = x - a
    e = y - b
    z = ol.beaver_mul(0, a0, b0, c0, d, e) + ol.beaver_mul(1, a1, b1, c1, d, e)
    assert np.array_equal(z, x * y)


def test_horner_closed_form():
    rng = np.random.default_rng(2024)
    n = 1000
    x, c0, c1, c2, c3 = (rng_u64(rng, n) for _ in range(5))
    got = ol.horner(x, c0, c1, c2, c3)
    for i in range(0, n, 37):
        X = int(x[i])
        exp = (int(c3[i]) * X ** 3 + int(c2[i]) * X ** 2 + int(c1[i]) * X + int(c0[i])) & M64
        assert int(got[i]) == exp


def test_row_broadcast_mul_reconstructs():
    rng = np.random.default_rng(9)
    rows, cols = 7, 33
    X = rng_u64(rng, rows * cols)
    v = rng_u64(rng, rows)
    A = rng_u64(rng, rows * cols)
    B = rng_u64(rng, rows)
    C = A * np.repeat(B, cols)
    A0, A1 = split(rng, A)
    B0, B1 = split(rng, B)
    C0, C1 = split(rng, C)
    d = X - A
    e = v - B
    lens = rng.integers(0, cols + 1, size=rows)
    z = (ol.row_broadcast_mul(0, A0, B0, C0, d, e, rows, cols, lens) +
         ol.row_broadcast_mul(1, A1, B1, C1, d, e, rows, cols, lens))
    exp = X * np.repeat(v, cols)
    mask = np.arange(cols)[None, :] < lens[:, None]
    assert np.array_equal(z.reshape(rows, cols)[mask], exp.reshape(rows, cols)[mask])
    assert not z.reshape(rows, cols)[~mask].any()


def test_row_reductions_closed_form():
    rng = np.random.default_rng(3)
    rows, cols = 9, 50
    mat = rng_u64(rng, rows * cols)
    lens = np.array([0, 1, 2, 4, 8, 16, 32, 37, 50])
    s = ol.row_sum(mat, rows, cols, lens)
    mu = ol.row_mean(mat, rows, cols, lens)
    var = ol.row_variance(mat, mu, rows, cols, lens)
    for r in range(rows):
        L = int(lens[r])
        vals = [int(v) for v in mat[r * cols:r * cols + L]]
        tot = sum(vals) & M64
        assert int(s[r]) == tot
        if L == 0:
            assert int(mu[r]) == 0 and int(var[r]) == 0
            continue
        exp_mu = tot >> (L.bit_length() - 1) if (L & (L - 1)) == 0 else tot // L
        assert int(mu[r]) == exp_mu
        assert int(var[r]) == sum(((v - exp_mu) & M64) ** 2 for v in vals) & M64
    offs = np.array([0, 0, 3, 10, 10, 40])
    vals = rng_u64(rng, 40)
    rs = ol.row_sum_ragged(vals, offs)
    for r in range(5):
        assert int(rs[r]) == sum(int(v) for v in vals[offs[r]:offs[r + 1]]) & M64


@pytest.mark.parametrize("eff_bits", [1, 3, 7, 12, 17, 31, 37, 50, 63, 64])
def test_pack_unpack_round_trip_and_layout(eff_bits):
    rng = np.random.default_rng(eff_bits)
    n = 301
    vals = rng_u64(rng, n)
    packed = ol.pack_eff_bits(vals, eff_bits)
    mask = (1 << eff_bits) - 1
    # Layout: element i occupies bits [i*eff, (i+1)*eff) of the little-endian stream.
    stream = 0
    for i, v in enumerate(vals):
        stream |= (int(v) & mask) << (i * eff_bits)
    words = [(stream >> (64 * w)) & M64 for w in range(len(packed))]
    assert [int(p) for p in packed] == words
    back = ol.unpack_eff_bits(packed, eff_bits, n)
    assert np.array_equal(back, vals & np.uint64(mask))


@pytest.mark.parametrize("ring_bits", [37, 50, 64])
@pytest.mark.parametrize("eff_bits", [37, 50, 64])
def test_open_add_closed_form(ring_bits, eff_bits):
    rng = np.random.default_rng(ring_bits * eff_bits)
    n = 200
    local = rng_u64(rng, n)
    remote = rng_u64(rng, n) & np.uint64((1 << eff_bits) - 1 if eff_bits < 64 else M64)
    packed = ol.pack_eff_bits(remote, eff_bits) if eff_bits < 64 else remote
    rmask = (1 << ring_bits) - 1 if ring_bits < 64 else M64
    for signed in (0, 1):
        got = ol.open_add(local, packed, eff_bits, n, ring_bits, rmask, signed)
        for i in range(n):
            v = (int(local[i]) + int(remote[i])) & rmask
            if signed and ring_bits < 64 and v >> (ring_bits - 1):
                v |= M64 ^ rmask
            assert int(got[i]) == v


def test_add_rout_aos():
    rng = np.random.default_rng(5)
    out = rng_u64(rng, 12 * 5)
    r = rng_u64(rng, 3)
    got = ol.add_rout_aos(out, 12, 5, r).reshape(12, 5)
    exp = out.reshape(12, 5).copy()
    exp[:, :3] += r
    assert np.array_equal(got, exp)


def test_beaver_matmul_reconstructs_product():
    rng = np.random.default_rng(10)
    M, K, N = 5, 11, 7
    X = rng_u64(rng, M * K).reshape(M, K)
    W = rng_u64(rng, K * N).reshape(K, N)
    A = rng_u64(rng, M * K).reshape(M, K)
    B = rng_u64(rng, K * N).reshape(K, N)

    def mm(P, Q):
        return np.array([[sum(int(P[i, k]) * int(Q[k, j]) for k in range(P.shape[1])) & M64
                          for j in range(Q.shape[1])] for i in range(P.shape[0])], dtype=np.uint64)

    C = mm(A, B)
    A0, A1 = split(rng, A.ravel())
    B0, B1 = split(rng, B.ravel())
    C0, C1 = split(rng, C.ravel())
    D = (X - A).ravel()
    E = (W - B).ravel()
    for wt in (0, 1):
        Ep = E.reshape(K, N).T.copy().ravel() if wt else E
        B0p = B0.reshape(K, N).T.copy().ravel() if wt else B0
        B1p = B1.reshape(K, N).T.copy().ravel() if wt else B1
        z = (ol.beaver_matmul(0, D, Ep, A0, B0p, C0, 1, M, K, N, wt) +
             ol.beaver_matmul(1, D, Ep, A1, B1p, C1, 1, M, K, N, wt))
        assert np.array_equal(z, mm(X, W).ravel()), wt


def test_beaver_scale_matches_int128():
    rng = np.random.default_rng(11)
    for _ in range(200):
        acc = int(rng_u64(rng, 1)[0])
        c = int(rng.integers(-2**40, 2**40))
        s = int(rng.integers(0, 80))
        sacc = acc - (1 << 64) if acc >> 63 else acc
        exp = ((sacc * c) >> s) & M64 if s > 0 else (sacc * c) & M64
        assert ol.LIB.orc_beaver_scale(acc, 1, c, s) == exp
        assert ol.LIB.orc_beaver_scale(acc, 0, c, s) == acc
