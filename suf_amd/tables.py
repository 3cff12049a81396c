"""Dealer-side piecewise tables of the softmax / LayerNorm gates, as SUF
builds them from doubles before keygen.

Each builder returns (alpha, coeffs): alpha is the ascending u64 piece
boundaries (alpha[0] = 0; the last piece runs to 2^64), coeffs the int64
x-form coefficient words of each piece (c0, c1, ...), in the layout the
interval LUT of the gate carries.

  nexp_table   make_nexp_piecewise_spec (include/gates/tables/
               nexp_piecewise_table.hpp:12-81) expanded to x-form cubics by
               build_silu_suf_from_piecewise / expand_to_x_coeffs
               (include/suf/suf_silu_builders.hpp:33-186): 4 words.
  recip_table  make_recip_affine_init_spec (include/gates/tables/
               recip_piecewise_affine_init.hpp:11-66) through the same
               expansion (RecipTask reads words 0 and 1,
               include/runtime/phase_tasks.hpp:3314-3326): 2 words.
  gelu_table   make_gelu_spline_spec (include/gates/tables/gelu_spline_table.hpp:
               57-92) through build_silu_suf_from_piecewise: 4 words.
  rsqrt_table  make_rsqrt_affine_init_spec (include/gates/tables/
               rsqrt_piecewise_affine_init.hpp:11-83) through
               build_rsqrt_affine_eval_suf (src/nn/transformer_layer.cpp:
               193-252): adj = a0 - (a1 * offset >> f), a1: 2 words.

Doubles are rounded with llround semantics (half away from zero); the last
piece's end (~0 in the reference's interval lists) is the 2^64 wrap.
"""
import math

import numpy as np

INT64_MAX = (1 << 63) - 1
INT64_MIN = -(1 << 63)
M64 = (1 << 64) - 1


def llround(v):
    """C llround: nearest integer, halves away from zero."""
    r = math.floor(abs(v) + 0.5)
    return int(r if v >= 0 else -r)


def _enc(v, frac_bits):
    return llround(v * math.ldexp(1.0, frac_bits))


def _pow(b, e):
    return math.pow(b, e)


def expand_to_x_coeffs(offset, coeffs, degree, frac_bits):
    """Polynomial in (x - x0) with Q(frac) coefficients -> Q(frac) coefficients
    of x^k (expand_to_x_coeffs, include/suf/suf_silu_builders.hpp:33-74)."""
    scale = math.ldexp(1.0, frac_bits)
    real = [(coeffs[i] / scale) if i < len(coeffs) else 0.0 for i in range(degree + 1)]
    x0 = offset / scale
    acc = [0.0] * (degree + 1)
    for k in range(degree + 1):
        ck = real[k]
        for i in range(k + 1):
            acc[i] += ck * float(math.comb(k, i)) * _pow(-x0, k - i)
    out = []
    for v in acc:
        v = v * scale
        v = min(max(v, float(INT64_MIN)), float(INT64_MAX))
        out.append(llround(v))
    return out


def _nexp_cubic(start, end, frac_bits):
    """make_nexp_cubic (nexp_piecewise_table.hpp:12-38): Hermite cubic of
    exp(-t) on [start, end], coefficients in (t - start)."""
    h = end - start
    y0, y1 = math.exp(-start), math.exp(-end)
    m0, m1 = -math.exp(-start), -math.exp(-end)
    c2 = (3.0 * (y1 - y0) - (2.0 * m0 + m1) * h) / (h * h)
    c3 = (2.0 * (y0 - y1) + (m0 + m1) * h) / (h * h * h)
    return [_enc(y0, frac_bits), _enc(m0, frac_bits), _enc(c2, frac_bits), _enc(c3, frac_bits)]


def _finish(pieces, words):
    """pieces: [(start_u64, offset, coeff list)] sorted by start, contiguous,
    starting at 0."""
    alpha = np.array([p[0] for p in pieces], dtype=np.uint64)
    if int(alpha[0]) != 0:
        raise ValueError("first piece must start at 0")
    c = np.zeros((len(pieces), words), dtype=np.int64)
    for i, (_, _, cs) in enumerate(pieces):
        c[i, :len(cs[:words])] = cs[:words]
    return alpha, c


def append_interval_signed(ivs, start_signed, end_signed, offset, coeffs):
    """append_interval_signed (include/gates/piecewise_poly.hpp:254-269): a
    signed [start, end) as u64 intervals, split at the wrap, the upper part
    ending at the ~0 surrogate of 2^64."""
    L, U = start_signed & M64, end_signed & M64

    def push(a, b):
        if a != b:
            ivs.append((a, b, offset, list(coeffs)))

    if L < U:
        push(L, U)
    else:
        push(0, U)
        push(L, M64)


def suf_from_piecewise(ivs, frac_bits, words=4):
    """build_silu_suf_from_piecewise (include/suf/suf_silu_builders.hpp:79-186):
    intervals sorted by start, a zero piece before the first when it starts
    above 0 and in every gap, overlaps trimmed, coefficients expanded to
    x-form cubics.  Returns (alpha, coeffs[words])."""
    pieces = []
    cur = 0
    seeded = False
    zero = [0] * words
    for start, end, off, cs in sorted(ivs, key=lambda t: t[0]):
        if end <= start:
            continue
        if not seeded:
            if start > 0:
                pieces.append((0, 0, zero))
            cur = start
            seeded = True
        if start < cur:
            start = cur
        if end <= start:
            continue
        if start > cur:
            pieces.append((cur, 0, zero))
            cur = start
        pieces.append((start, off, expand_to_x_coeffs(off, cs, 3, frac_bits)))
        cur = end
    if not pieces:
        pieces = [(0, 0, zero)]
    return _finish(pieces, words)


def _gelu(x):
    return 0.5 * x * (1.0 + math.erf(x * 0.70710678118654752440))


def _gelu_deriv(x):
    phi = 0.39894228040143267794 * math.exp(-0.5 * x * x)
    return 0.5 * (1.0 + math.erf(x * 0.70710678118654752440)) + x * phi


def gelu_table(frac_bits=12, segments=16):
    """make_gelu_spline_spec (include/gates/tables/gelu_spline_table.hpp:57-92):
    0 below -8, Hermite cubics of x Phi(x) on `segments` pieces of [-8, 8),
    y = x above 8; through build_silu_suf_from_piecewise: (alpha, coeffs[4])."""
    lo, hi = -8.0, 8.0
    step = (hi - lo) / segments
    ivs = []
    append_interval_signed(ivs, INT64_MIN, _enc(lo, frac_bits), 0, [0])
    for i in range(segments):
        start = lo + step * i
        end = hi if i == segments - 1 else start + step
        sf, ef = _enc(start, frac_bits), _enc(end, frac_bits)
        h = end - start
        y0, y1 = _gelu(start), _gelu(end)
        m0, m1 = _gelu_deriv(start), _gelu_deriv(end)
        c2 = (3.0 * (y1 - y0) - (2.0 * m0 + m1) * h) / (h * h)
        c3 = (2.0 * (y0 - y1) + (m0 + m1) * h) / (h * h * h)
        pack = [_enc(y0, frac_bits), _enc(m0, frac_bits), _enc(c2, frac_bits), _enc(c3, frac_bits)]
        append_interval_signed(ivs, sf, ef, sf, pack)
    append_interval_signed(ivs, _enc(hi, frac_bits), INT64_MAX, 0, [0, 1 << frac_bits])
    return suf_from_piecewise(ivs, frac_bits, 4)


def nexp_table(frac_bits=12, segments=16):
    """exp(-t) on [0, 16) in `segments` cubic pieces plus the constant tail
    [16, 2^64) = exp(-16): (alpha [segments + 1], coeffs [segments + 1][4])."""
    lo, hi = 0.0, 16.0
    step = (hi - lo) / segments
    pieces = []
    for i in range(segments):
        start = lo + step * i
        end = hi if i == segments - 1 else start + step
        start_fixed = _enc(start, frac_bits)
        pack = _nexp_cubic(start, end, frac_bits)
        pieces.append((start_fixed & M64, start_fixed,
                       expand_to_x_coeffs(start_fixed, pack, 3, frac_bits)))
    tail = [_enc(math.exp(-hi), frac_bits)]
    pieces.append((_enc(hi, frac_bits) & M64, 0, expand_to_x_coeffs(0, tail, 3, frac_bits)))
    return _finish(pieces, 4)


def recip_table(frac_bits=12, nmax=1024.0):
    """1/x affine init: constant 1 on [0, 1), chords of 1/x on [2^k, 2^(k+1))
    up to nmax, constant 1/nmax above: (alpha, coeffs [..][2] = c0, c1)."""
    pieces = [(0, 0, expand_to_x_coeffs(0, [_enc(1.0, frac_bits)], 3, frac_bits))]
    bounds = [1.0]
    cur = 1.0
    while cur < nmax:
        cur *= 2.0
        bounds.append(min(cur, nmax))
    for i in range(1, len(bounds)):
        L, U = bounds[i - 1], bounds[i]
        y0, y1 = 1.0 / L, 1.0 / U
        slope = (y1 - y0) / (U - L)
        off = _enc(L, frac_bits)
        pieces.append((off & M64, off,
                       expand_to_x_coeffs(off, [_enc(y0, frac_bits), _enc(slope, frac_bits)], 3,
                                          frac_bits)))
    pieces.append((_enc(nmax, frac_bits) & M64, 0,
                   expand_to_x_coeffs(0, [_enc(1.0 / nmax, frac_bits)], 3, frac_bits)))
    return _finish(pieces, 2)


def rsqrt_table(frac_bits=12, eps=1.0 / 1024.0, vmax=16.0):
    """1/sqrt(x) affine init: constant 1/sqrt(eps) below eps, chords on
    [eps 2^k, eps 2^(k+1)) up to vmax, constant 1/sqrt(vmax) above, as the
    x-form words (a0 - (a1 * offset >> f), a1)."""
    scale = math.ldexp(1.0, frac_bits)
    eps_q = _enc(eps, frac_bits)
    if eps_q == 0:
        eps_q = 1
    raw = [(0, eps_q, 0, [_enc(1.0 / math.sqrt(max(eps, 2.2250738585072014e-308)), frac_bits)])]
    bounds = [eps]
    cur = eps
    while cur < vmax:
        cur *= 2.0
        bounds.append(min(cur, vmax))
    bq = [eps_q]
    for b in bounds[1:]:
        q = _enc(b, frac_bits)
        if q <= bq[-1]:
            q = bq[-1] + 1
        bq.append(q)
    for i in range(1, len(bounds)):
        Lq, Uq = bq[i - 1], bq[i]
        if Uq <= Lq:
            continue
        L, U = Lq / scale, Uq / scale
        y0, y1 = 1.0 / math.sqrt(L), 1.0 / math.sqrt(U)
        slope = (y1 - y0) / (U - L)
        raw.append((Lq, Uq, Lq, [_enc(y0, frac_bits), _enc(slope, frac_bits)]))
    vq = bq[-1] if bq else _enc(vmax, frac_bits)
    raw.append((vq, M64, 0, [_enc(1.0 / math.sqrt(vmax), frac_bits)]))
    pieces = []
    for start, end, off, cs in raw:
        if start >= end:
            continue
        a0 = cs[0]
        a1 = cs[1] if len(cs) > 1 else 0
        adj = a0 - ((a1 * off) >> frac_bits)
        adj = min(max(adj, INT64_MIN), INT64_MAX)
        pieces.append((start, off, [adj, a1]))
    pieces.sort(key=lambda p: p[0])
    return _finish(pieces, 2)


def inv_len_qf(cols, frac_bits=12):
    """LayerNorm's public 1/L in Q(frac) (src/nn/transformer_layer.cpp:683-684)."""
    return llround((1.0 / cols) * math.ldexp(1.0, frac_bits))


def eps_qf(eps=1.0 / 1024.0, frac_bits=12):
    """LayerNorm's epsilon in Q(frac), added by party 0 (transformer_layer.cpp:685-686)."""
    return llround(eps * math.ldexp(1.0, frac_bits))
