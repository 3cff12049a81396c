"""Closed forms of SUF's softmax and LayerNorm task chains over Z_2^64.

TEST INFRASTRUCTURE ONLY: the checker.  Only tests/, __graft_entry__.smoke()
and the cpu_baseline leg of bench.py import this module; the product never
does.

What a two-party run of each task chain must reconstruct to, as plain
fixed-point arithmetic on int64 numpy arrays.  Every truncation of the secure
chain is an exact arithmetic shift (floor division by 2^k; GapARS and
faithful ARS both reconstruct to it while |x| < 2^62), so the chains reduce
to these formulas.  Products are checked against 2^62 before they are
formed: an input outside that range raises instead of wrapping.

  spline_closed_form  the spline gate of CubicPolyTask's reference path
                  (include/runtime/phase_tasks.hpp:2933-2945) with exact shifts
  cubic_task      CubicPolyTask (include/runtime/phase_tasks.hpp:2933-3061)
  recip_task      RecipTask (phase_tasks.hpp:3190-3540; NR step of
                  ref_reciprocal_fixed, include/gates/reciprocal_gate.hpp:96-109)
  rsqrt_task      RsqrtTask (phase_tasks.hpp:1415-1640) with the init
                  c0 + (c1 x >> f) and the NR step of ref_rsqrt_fixed
                  (include/gates/rsqrt_gate.hpp:100-117)
  row_max_diff    RowMaxDiffTask (include/nn/row_maxdiff_task.hpp:49-165)
  softmax_block   SoftmaxBlockTask (include/nn/softmax_block_task.hpp:97-450)
  layernorm       LayerNormTask (phase_tasks.hpp:2232-2610) without gamma/beta,
                  as transformer_layer_forward runs it
                  (src/nn/transformer_layer.cpp:626-760)
  attention       attention_forward's causal prefill (src/nn/attention_block.cpp:
                  1500-1900): per-head Q K^T scaled by inv_sqrt and truncated by
                  2f, softmax over the causal rows, P V truncated by f
  transformer_layer  transformer_layer_forward (transformer_layer.cpp:435-830)
                  with mlp_forward (src/nn/mlp_block.cpp:378-767): LN, QKV,
                  attention, Wout, residual, LN, W1, GeLU cubic, W2, residual

Pinning (tests/test_oracle_fixed_point.py): each formula against the real
function it approximates (exp, 1/x, 1/sqrt, softmax, layer norm, a float64
GPT-2 layer with the same weights)
within the table's stated accuracy, against brute force (row max, piece
selection at every boundary), and against hand-computed values.
"""
import numpy as np

LIM = float(1 << 62)


def _i64(a):
    return np.asarray(a).astype(np.uint64).view(np.int64)


def _u64(a):
    return np.asarray(a, dtype=np.int64).view(np.uint64)


def _check(a, b, what):
    m = np.abs(a.astype(np.float64)) * np.abs(b.astype(np.float64))
    if m.size and float(m.max()) >= LIM * (1 - 1e-9):
        raise ValueError("%s: product outside the exact range (|a b| >= 2^62)" % what)


def mul_shift(a, b, s, what="mul_shift"):
    """floor(a * b / 2^s) for int64 arrays (the reconstruction of a Beaver
    product followed by an exact truncation by s)."""
    a = np.asarray(a, dtype=np.int64)
    b = np.asarray(b, dtype=np.int64)
    _check(a, b, what)
    return (a * b) >> s


def piece_index(alpha, x):
    """Piece of each u64 input: the last alpha_i <= x (alpha[0] = 0)."""
    return np.searchsorted(np.asarray(alpha, dtype=np.uint64), _u64(_i64(x)), side="right") - 1


def spline_closed_form(alpha, coeffs, x, frac_bits):
    """The spline gate at x (u64 ring values): piece i of the sorted piece
    starts alpha (x's last start <= x), then
    y = ((c3 x + c2 2^f) x >> f) + c1 2^f) x >> 2f) + c0 with arithmetic
    shifts (phase_tasks.hpp:2933-2945).  Raises if an intermediate could
    leave (-2^62, 2^62) for these inputs."""
    x = np.asarray(x, dtype=np.uint64)
    piece = np.searchsorted(alpha, x, side="right") - 1
    c = coeffs[piece]
    xs = x.view(np.int64)
    f = frac_bits
    cx = int(np.abs(coeffs).max())
    xm = int(np.abs(xs).max()) if xs.size else 0
    u_max = cx * xm + (cx << f)
    q_max = ((u_max * xm) >> f) + 1 + (cx << f)
    if max(u_max * xm, q_max * xm) >= 1 << 62:
        raise ValueError("spline_closed_form: inputs outside the exact int64 range")
    u = c[:, 3] * xs + (c[:, 2] << f)
    p2 = (u * xs) >> f
    q = p2 + (c[:, 1] << f)
    y = ((q * xs) >> (2 * f)) + c[:, 0]
    return y.view(np.uint64)


def cubic_task(alpha, coeffs, x, f):
    """y = trunc_2f((trunc_f((c3 x + c2 2^f) x) + c1 2^f) x) + c0."""
    x = _i64(x)
    c = np.asarray(coeffs, dtype=np.int64)[piece_index(alpha, x)]
    u = c[:, 3] * x + (c[:, 2] << f)
    _check(c[:, 3], x, "cubic c3 x")
    p2 = mul_shift(u, x, f, "cubic u x")
    q = p2 + (c[:, 1] << f)
    return mul_shift(q, x, 2 * f, "cubic q x") + c[:, 0]


def affine_init(alpha, coeffs, x, f):
    """c0 + trunc_f(c1 x) for the piece of x (the init of RecipTask / RsqrtTask)."""
    x = _i64(x)
    c = np.asarray(coeffs, dtype=np.int64)[piece_index(alpha, x)]
    return c[:, 0] + mul_shift(c[:, 1], x, f, "init c1 x")


def recip_task(alpha, coeffs, x, f, iters=1):
    """NR for 1/x: xy = trunc_f(y x); y = trunc_f(y (2^(f+1) - xy))."""
    x = _i64(x)
    y = affine_init(alpha, coeffs, x, f)
    two = np.int64(2 << f)
    for _ in range(iters):
        xy = mul_shift(y, x, f, "recip y x")
        y = mul_shift(y, two - xy, f, "recip y (2 - xy)")
    return y


def rsqrt_task(alpha, coeffs, x, f, iters=1):
    """NR for 1/sqrt(x): y2 = trunc_f(y y); h = trunc_f(x y2) >> 1
    (= trunc_(f+1)(x y2)); y = trunc_f(y (1.5 2^f - h))."""
    x = _i64(x)
    y = affine_init(alpha, coeffs, x, f)
    onept5 = np.int64(3 << (f - 1))
    for _ in range(iters):
        y2 = mul_shift(y, y, f, "rsqrt y y")
        h = mul_shift(x, y2, f + 1, "rsqrt x y2")
        y = mul_shift(y, onept5 - h, f, "rsqrt y inner")
    return y


def row_max_diff(x, offsets):
    """delta_i = max(row) - x_i over each row [offsets[r], offsets[r+1])."""
    x = _i64(x)
    out = np.zeros_like(x)
    for r in range(len(offsets) - 1):
        b, e = int(offsets[r]), int(offsets[r + 1])
        if e > b:
            out[b:e] = x[b:e].max() - x[b:e]
    return out


def row_sums(x, offsets):
    x = _i64(x)
    return np.array([int(x[int(offsets[r]):int(offsets[r + 1])].sum())
                     for r in range(len(offsets) - 1)], dtype=np.int64)


def row_of(offsets):
    offsets = np.asarray(offsets)
    return np.repeat(np.arange(len(offsets) - 1), np.diff(offsets))


def softmax_block(scores, offsets, nexp, recip, f, recip_iters=1):
    """Packed ragged rows of Q(f) scores -> Q(f) probabilities.
    nexp = (alpha, coeffs[4]); recip = (alpha, coeffs[2]).
    Returns (prob, dict of the intermediate stages)."""
    delta = row_max_diff(scores, offsets)
    e = cubic_task(nexp[0], nexp[1], delta, f)
    s = row_sums(e, offsets)
    inv = recip_task(recip[0], recip[1], s, f, recip_iters)
    prob = mul_shift(e, inv[row_of(offsets)], f, "softmax e inv")
    return prob, {"delta": delta, "exp": e, "sum": s, "inv": inv}


def layernorm(x, rows, cols, f, inv_len, eps_q, rsqrt, rsqrt_iters=1):
    """Row-major [rows x cols] Q(f) -> Q(f):
    mu = trunc_f(sum x * invL); d = x - mu; var = trunc_2f(sum d^2 * invL);
    r = rsqrt(var + eps); y = trunc_f(d r)."""
    x = _i64(x).reshape(rows, cols)
    s = x.sum(axis=1)
    mu = mul_shift(s, np.full(rows, inv_len, dtype=np.int64), f, "ln sum invL")
    d = x - mu[:, None]
    _check(d, d, "ln d d")
    sq = (d * d).sum(axis=1)
    var = mul_shift(sq, np.full(rows, inv_len, dtype=np.int64), 2 * f, "ln sq invL")
    v = var + np.int64(eps_q)
    r = rsqrt_task(rsqrt[0], rsqrt[1], v, f, rsqrt_iters)
    y = mul_shift(d, np.broadcast_to(r[:, None], d.shape), f, "ln d r")
    return y.reshape(-1), {"mu": mu, "var": var, "rsqrt": r}


def matmul_shift(X, W, s, what="matmul"):
    """floor(X W / 2^s) for int64 matrices, exact (checked against 2^62)."""
    X = np.asarray(X, dtype=np.int64)
    W = np.asarray(W, dtype=np.int64)
    k = X.shape[-1]
    bound = float(np.abs(X).max(initial=0)) * float(np.abs(W).max(initial=0)) * k
    if bound >= LIM * (1 - 1e-9):
        raise ValueError("%s: product outside the exact range" % what)
    return np.matmul(X, W) >> s


def causal_offsets(heads, seq):
    lens = np.tile(np.arange(1, seq + 1), heads)
    return np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)


def attention(qkv, seq, d, heads, f, nexp, recip):
    """Causal attention on Q(f) QKV rows [seq x 3d] -> context [seq x d]."""
    dh = d // heads
    qkv = _i64(qkv).reshape(seq, 3 * d)
    inv_sqrt = max(int(np.floor(abs((1.0 / np.sqrt(dh)) * (1 << f)) + 0.5)), 1)
    offs = causal_offsets(heads, seq)
    scores = []
    for h in range(heads):
        Q = qkv[:, h * dh:(h + 1) * dh]
        K = qkv[:, d + h * dh:d + (h + 1) * dh]
        S = matmul_shift(Q, K.T, 0, "attention Q K^T")
        S = mul_shift(S, np.full(S.shape, inv_sqrt, dtype=np.int64), 2 * f, "attention scale")
        for r in range(seq):
            scores.append(S[r, :r + 1])
    scores = np.concatenate(scores)
    prob, st = softmax_block(scores, offs, nexp, recip, f)
    ctx = np.zeros((seq, d), dtype=np.int64)
    for h in range(heads):
        P = np.zeros((seq, seq), dtype=np.int64)
        for r in range(seq):
            b = int(offs[h * seq + r])
            P[r, :r + 1] = prob[b:b + r + 1]
        V = qkv[:, 2 * d + h * dh:2 * d + (h + 1) * dh]
        ctx[:, h * dh:(h + 1) * dh] = matmul_shift(P, V, f, "attention P V")
    return ctx.reshape(-1), {"scores": scores, "prob": prob, **st}


def transformer_layer(x, W, seq, d, heads, ffn, f, tabs, inv_len, eps_q):
    """x [seq x d] Q(f) -> layer output; W: dict of int64 Wqkv [d x 3d],
    Wout [d x d], W1 [d x ffn], W2 [ffn x d]; tabs: dict of (alpha, coeffs)
    for "nexp", "recip", "rsqrt", "gelu"."""
    x = _i64(x).reshape(seq, d)
    h1, _ = layernorm(x, seq, d, f, inv_len, eps_q, tabs["rsqrt"])
    qkv = matmul_shift(h1.reshape(seq, d), W["Wqkv"], f, "qkv")
    ctx, st = attention(qkv, seq, d, heads, f, tabs["nexp"], tabs["recip"])
    r1 = matmul_shift(ctx.reshape(seq, d), W["Wout"], f, "out proj") + x
    h2, _ = layernorm(r1, seq, d, f, inv_len, eps_q, tabs["rsqrt"])
    u = matmul_shift(h2.reshape(seq, d), W["W1"], f, "w1")
    g = cubic_task(tabs["gelu"][0], tabs["gelu"][1], u.reshape(-1), f).reshape(seq, ffn)
    out = matmul_shift(g, W["W2"], f, "w2") + r1
    return out.reshape(-1), {"h1": h1, "qkv": qkv.reshape(-1), "ctx": ctx, "r1": r1.reshape(-1),
                             "h2": h2, "u": u.reshape(-1), "g": g.reshape(-1), **st}
