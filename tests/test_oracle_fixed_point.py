"""Pins the closed forms of oracle/fixed_point.py (softmax / LayerNorm task
chains) and the dealer tables they evaluate, without any GPU:

  * against the real functions in float64 (exp(-t), 1/x, 1/sqrt(x), GeLU,
    softmax, layer norm, causal attention, a whole GPT-2 block) within the
    accuracy the 12-fraction-bit tables allow;
  * against brute force (row max, piece selection at every boundary);
  * against values computed by hand from the reference formulas.
A planted mistake (a dropped NR step, an off-by-one shift, a wrong piece)
fails at least one of these.
"""
import math
import os
import sys

import numpy as np
import pytest

from suf_amd import softmax, tables

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "oracle"))
import fixed_point as fp  # noqa: E402

F = 12
ONE = 1 << F


def test_llround_half_away_from_zero():
    assert [tables.llround(v) for v in (0.5, 1.5, -0.5, -1.5, 2.4999, -2.5)] == \
        [1, 2, -1, -2, 2, -3]


def test_nexp_table_tracks_exp():
    a, c = tables.nexp_table(F)
    assert len(a) == 17 and int(a[16]) == 16 * ONE and not c[16].any()
    t = np.arange(0, 20 * ONE, 3, dtype=np.int64)
    y = fp.cubic_task(a, c, t, F)
    assert np.abs(y / ONE - np.exp(-t / ONE)).max() < 2.5e-3
    # Segment 0 is exp's Hermite cubic on [0, 1): c = (1, -1, ...) in Q12.
    assert c[0, 0] == ONE and c[0, 1] == -ONE


def test_expand_to_x_coeffs_by_hand():
    # (x - 2)^2 / 2^12 in Q12 with offset 2.0: x^2 - 4x + 4.
    assert tables.expand_to_x_coeffs(2 * ONE, [0, 0, ONE, 0], 3, F) == [4 * ONE, -4 * ONE, ONE, 0]


def test_recip_table_and_task():
    a, c = tables.recip_table(F)
    assert list(a[:3]) == [0, ONE, 2 * ONE] and int(a[-1]) == 1024 * ONE
    # Piece [64, 128): chord slope -1/8192 rounds to -1/4096 in Q12 (llround(-0.5) = -1).
    k = int(np.searchsorted(a, 64 * ONE, side="right") - 1)
    assert list(c[k]) == [128, -1]
    # By hand at x = 127.0: y0 = 128 - 127 = 1; xy = 127; y = (1 * (8192 - 127)) >> 12 = 1.
    assert int(fp.recip_task(a, c, np.array([127 * ONE]), F)[0]) == 1
    # Well-conditioned range [1, 32): NR brings the chord init within 3% (Q12
    # quantisation of y ~ 1/32 alone is 0.8%).
    x = np.arange(ONE, 32 * ONE, 17, dtype=np.int64)
    y = fp.recip_task(a, c, x, F)
    assert np.max(np.abs(y / ONE - ONE / x) * (x / ONE)) < 0.03
    # Zero NR iterations is the init alone (a dropped iteration changes values).
    assert not np.array_equal(fp.recip_task(a, c, x, F, 0), y)
    assert np.array_equal(fp.recip_task(a, c, x, F, 0), fp.affine_init(a, c, x, F))


def test_rsqrt_table_and_task():
    a, c = tables.rsqrt_table(F)
    assert int(a[1]) == 4 and list(c[0]) == [32 * ONE, 0]  # 1/sqrt(eps) below eps
    x = np.arange(4, 16 * ONE, 7, dtype=np.int64)
    y = fp.rsqrt_task(a, c, x, F)
    assert np.max(np.abs(y / ONE - 1 / np.sqrt(x / ONE)) * np.sqrt(x / ONE)) < 6e-3
    # NR step by hand at x = 1.0 (piece [0.5, 1.0) ends there, so x = 1.0 is
    # in [1, 2)): init y0 = c0 + (c1 * 4096 >> 12).
    k = int(np.searchsorted(a, ONE, side="right") - 1)
    y0 = int(c[k, 0]) + ((int(c[k, 1]) * ONE) >> F)
    y2 = (y0 * y0) >> F
    h = (ONE * y2) >> (F + 1)
    want = (y0 * (3 * (ONE >> 1) - h)) >> F
    assert int(fp.rsqrt_task(a, c, np.array([ONE]), F)[0]) == want


def test_piece_index_at_boundaries():
    a, c = tables.nexp_table(F)
    b = a.astype(np.int64)
    xs = np.concatenate([b, b[1:] - 1])
    got = fp.piece_index(a, xs)
    want = [int(np.max(np.nonzero(a <= np.uint64(v))[0])) for v in xs]
    assert list(got) == want


def test_row_max_diff_brute_force():
    rng = np.random.default_rng(3)
    offs = np.array([0, 1, 2, 7, 70], dtype=np.int64)
    x = rng.integers(-(1 << 40), 1 << 40, size=70)
    d = fp.row_max_diff(x, offs)
    for r in range(4):
        seg = x[offs[r]:offs[r + 1]]
        assert np.array_equal(d[offs[r]:offs[r + 1]], seg.max() - seg)


def test_max_tree_plan_reaches_the_max():
    """Replaying the plan with exact max on each pair yields each row's max."""
    offs = softmax.causal_offsets(2, 9)
    rng = np.random.default_rng(4)
    x = rng.integers(-1000, 1000, size=int(offs[-1]))
    rounds, max_pos = softmax.max_tree_plan(offs)
    cur = x.copy()
    for src_a, src_b, n_in in rounds:
        assert n_in == cur.size
        nxt = np.where(src_b >= 0, np.maximum(cur[src_a], cur[np.maximum(src_b, 0)]), cur[src_a])
        cur = nxt
    for r in range(len(offs) - 1):
        assert cur[max_pos[r]] == x[offs[r]:offs[r + 1]].max()


def test_softmax_closed_form_tracks_float_softmax():
    offs = softmax.causal_offsets(2, 64)
    rng = np.random.default_rng(5)
    s = np.round(rng.normal(0, 2, size=int(offs[-1])) * ONE).astype(np.int64)
    prob, st = fp.softmax_block(s, offs, tables.nexp_table(F), tables.recip_table(F), F)
    for r in range(len(offs) - 1):
        seg = s[offs[r]:offs[r + 1]] / ONE
        p = np.exp(seg - seg.max())
        p /= p.sum()
        if st["sum"][r] < 32 * ONE:  # the reciprocal table is accurate there
            assert np.abs(prob[offs[r]:offs[r + 1]] / ONE - p).max() < 0.02
    assert np.all(st["delta"] >= 0)


def test_layernorm_closed_form_tracks_float():
    rows, cols = 8, 768
    rng = np.random.default_rng(6)
    x = np.round(rng.normal(0.3, 1.2, size=(rows, cols)) * ONE).astype(np.int64)
    y, st = fp.layernorm(x.reshape(-1), rows, cols, F, tables.inv_len_qf(cols),
                         tables.eps_qf(), tables.rsqrt_table(F))
    xf = x / ONE
    # The reference's mean uses invL = llround(2^12 / 768) = 5 (1/819.2, not 1/768).
    mu = np.floor(x.sum(axis=1) * 5 / ONE) / ONE
    assert np.array_equal(st["mu"], np.floor(x.sum(axis=1) * 5 / ONE).astype(np.int64))
    d = xf - mu[:, None]
    var = (d * d).sum(axis=1) * 5 / ONE
    ref = d / np.sqrt(var + 1 / 1024)[:, None]
    assert np.abs(y.reshape(rows, cols) / ONE - ref).max() < 0.05


def _erf_gelu(u):
    return 0.5 * u * (1.0 + np.vectorize(math.erf)(u / math.sqrt(2.0)))


def _float_ln(v):
    mu = v.mean(axis=1, keepdims=True)
    dd = v - mu
    return dd / np.sqrt((dd * dd).mean(axis=1, keepdims=True) + 1.0 / 1024)


def _float_attention(qkv, seq, d, heads):
    dh = d // heads
    out = np.zeros((seq, d))
    causal = np.tril(np.ones((seq, seq))) > 0
    for h in range(heads):
        Q = qkv[:, h * dh:(h + 1) * dh]
        K = qkv[:, d + h * dh:d + (h + 1) * dh]
        V = qkv[:, 2 * d + h * dh:2 * d + (h + 1) * dh]
        S = np.where(causal, Q @ K.T / math.sqrt(dh), -np.inf)
        P = np.exp(S - S.max(axis=1, keepdims=True))
        out[:, h * dh:(h + 1) * dh] = (P / P.sum(axis=1, keepdims=True)) @ V
    return out


def test_gelu_table_tracks_gelu():
    """x Phi(x) (erf form) on [-10, 10): within 0.005; 0 below -8, x above 8."""
    a, c = tables.gelu_table(F)
    x = np.arange(-10 * ONE, 10 * ONE, 7, dtype=np.int64)
    y = fp.cubic_task(a, c, x, F) / ONE
    assert np.abs(y - _erf_gelu(x / ONE)).max() < 0.005
    assert np.all(y[x < -8 * ONE] == 0)
    assert np.array_equal(fp.cubic_task(a, c, x[x >= 8 * ONE], F), x[x >= 8 * ONE])


def test_attention_closed_form_tracks_float():
    """Causal multi-head attention on Q12 QKV rows (4 heads of 16) against the
    float64 softmax(Q K^T / sqrt(dh)) V."""
    seq, d, heads = 16, 64, 4
    rng = np.random.default_rng(7)
    qkv = np.round(rng.normal(0, 1, size=(seq, 3 * d)) * ONE).astype(np.int64)
    ctx, st = fp.attention(qkv.reshape(-1), seq, d, heads, F, tables.nexp_table(F),
                           tables.recip_table(F))
    ref = _float_attention(qkv / ONE, seq, d, heads)
    assert np.abs(ctx.reshape(seq, d) / ONE - ref).max() < 0.05
    assert len(st["scores"]) == heads * seq * (seq + 1) // 2


def test_transformer_layer_closed_form_tracks_float():
    """The whole layer (weights N(0, 0.1), so that every branch moves the
    output by more than 1) against a float64 GPT-2 block without biases or
    gamma/beta; each stage also against float64 applied to the closed form's
    own input of that stage."""
    seq, d, heads, ffn = 16, 64, 4, 256
    rng = np.random.default_rng(8)
    W = {k: np.round(rng.normal(0, 0.1, size=sh) * ONE).astype(np.int64)
         for k, sh in [("Wqkv", (d, 3 * d)), ("Wout", (d, d)), ("W1", (d, ffn)),
                       ("W2", (ffn, d))]}
    x = np.round(rng.normal(0, 1, size=(seq, d)) * ONE).astype(np.int64)
    tabs = {"nexp": tables.nexp_table(F), "recip": tables.recip_table(F),
            "rsqrt": tables.rsqrt_table(F), "gelu": tables.gelu_table(F)}
    out, st = fp.transformer_layer(x.reshape(-1), W, seq, d, heads, ffn, F, tabs,
                                   tables.inv_len_qf(d), tables.eps_qf())
    Wf = {k: v / ONE for k, v in W.items()}
    xf = x / ONE
    r1 = _float_attention(_float_ln(xf) @ Wf["Wqkv"], seq, d, heads) @ Wf["Wout"] + xf
    ref = _erf_gelu(_float_ln(r1) @ Wf["W1"]) @ Wf["W2"] + r1
    assert np.abs(ref - xf).max() > 1.0
    assert np.abs(out.reshape(seq, d) / ONE - ref).max() < 0.06
    assert np.abs(st["h1"].reshape(seq, d) / ONE - _float_ln(xf)).max() < 0.02
    ctx_ref = _float_attention(st["qkv"].reshape(seq, 3 * d) / ONE, seq, d, heads)
    assert np.abs(st["ctx"].reshape(seq, d) / ONE - ctx_ref).max() < 0.05
    assert np.abs(st["g"] / ONE - _erf_gelu(st["u"] / ONE)).max() < 0.005


def test_mul_shift_refuses_out_of_range():
    with pytest.raises(ValueError):
        fp.mul_shift(np.array([1 << 40]), np.array([1 << 30]), F)
    assert int(fp.mul_shift(np.array([-3]), np.array([1]), 1)[0]) == -2  # floor, not toward 0
    assert math.floor(-1.5) == -2
