"""Two-party protocol steps composed from the CPU oracle (test infrastructure):
the share-level expectation for the GPU task chains, step by step, from the
same dealer material (keys and triples copied back from the device objects).

Each helper returns both parties' shares as host u64 arrays.
"""
import numpy as np

import oracle_lib as ol
from gpu_util import host

M64 = (1 << 64) - 1


def u(a):
    return np.asarray(a).astype(np.uint64) if np.asarray(a).dtype != np.uint64 else np.asarray(a)


def lut2(lut, xhat):
    """Both parties' coefficient rows [n][words] of a tasks.CoeffLut."""
    n = xhat.size
    return [ol.lut_eval(lut.blobs[p], lut.key_bytes, 1, u(xhat), lut.words).reshape(n, lut.words)
            for p in (0, 1)]


def beaver2(x, y, tri, row_of=None):
    """z_p of the Beaver product of shares x = (x0, x1), y = (y0, y1) with a
    tasks.Triples (row-broadcast when row_of is given: y and b per row)."""
    sh = [tri.shares(p) for p in (0, 1)]
    a = [sh[p][0] for p in (0, 1)]
    b = [sh[p][1] if row_of is None else sh[p][1][row_of] for p in (0, 1)]
    c = [sh[p][2] for p in (0, 1)]
    yy = [u(y[p]) if row_of is None else u(y[p])[row_of] for p in (0, 1)]
    d = ((u(x[0]) - a[0]) + (u(x[1]) - a[1])).astype(np.uint64)
    e = ((yy[0] - b[0]) + (yy[1] - b[1])).astype(np.uint64)
    return [ol.beaver_mul(p, a[p], b[p], c[p], d, e) for p in (0, 1)]


def open2(z, mask):
    return (u(z[0]) + u(z[1]) + np.uint64(mask & M64)).astype(np.uint64)


def trunc2(prg, tr, zhat):
    """Both parties' outputs of a tasks.Trunc at the masked open zhat."""
    return [ol.trunc_eval(prg, tr.kind, tr.f, host(tr.keys[p]), u(zhat)) for p in (0, 1)]


def beaver_trunc2(prg, x, y, tri, tr, row_of=None):
    z = beaver2(x, y, tri, row_of)
    return trunc2(prg, tr, open2(z, tr.mask))


def add2(x, y):
    return [(u(x[p]) + u(y[p])).astype(np.uint64) for p in (0, 1)]


def const2(x, c):
    """x + c with the public constant on party 0's share."""
    return [(u(x[0]) + np.uint64(c & M64)).astype(np.uint64), u(x[1])]


def neg2(x):
    return [(np.uint64(0) - u(x[p])).astype(np.uint64) for p in (0, 1)]


def recon(x):
    return (u(x[0]) + u(x[1])).astype(np.uint64)


def recip2(prg, rc, x, xhat):
    """softmax.Recip on shares x with masked open xhat."""
    f = rc.f
    coef = lut2(rc.lut, xhat)
    t = beaver_trunc2(prg, [coef[0][:, 1], coef[1][:, 1]], x, rc.tri[0], rc.tr[0])
    y = add2(t, [coef[0][:, 0], coef[1][:, 0]])
    for it in range(rc.iters):
        xy = beaver_trunc2(prg, y, x, rc.tri[1 + 2 * it], rc.tr[1 + 2 * it])
        y = beaver_trunc2(prg, y, const2(neg2(xy), 2 << f), rc.tri[2 + 2 * it],
                          rc.tr[2 + 2 * it])
    return y


def rsqrt2(prg, rs, v, vhat):
    """layernorm.Rsqrt on shares v with masked open vhat."""
    f = rs.f
    coef = lut2(rs.lut, vhat)
    t = beaver_trunc2(prg, [coef[0][:, 1], coef[1][:, 1]], v, rs.tri[0], rs.tr[0])
    y = add2(t, [coef[0][:, 0], coef[1][:, 0]])
    for it in range(rs.iters):
        ta, tb, tc = rs.tr[1 + 3 * it: 4 + 3 * it]
        ka, kb, kc = rs.tri[1 + 3 * it: 4 + 3 * it]
        y2 = beaver_trunc2(prg, y, y, ka, ta)
        h = beaver_trunc2(prg, v, y2, kb, tb)
        y = beaver_trunc2(prg, y, const2(neg2(h), 3 << (f - 1)), kc, tc)
    return y


def relu_rounds2(rm, x):
    """softmax.RowMaxDiff on shares x: delta shares."""
    cur = [u(x[0]), u(x[1])]
    for rd in rm.rounds:
        src_a, src_b = rd["src"]
        pair = src_b >= 0
        bb = np.where(pair, src_b, 0)
        xa = [cur[p][src_a] for p in (0, 1)]
        xb = [cur[p][bb] for p in (0, 1)]
        xhat = ((xa[0] - xb[0]) + (xa[1] - xb[1]) + np.uint64(rd["lut"].mask)).astype(np.uint64)
        q = lut2(rd["lut"], xhat)
        nxt = []
        for p in (0, 1):
            v = (xb[p] + q[p][:, 0] + q[p][:, 1] * xhat).astype(np.uint64)
            nxt.append(np.where(pair, v, xa[p]).astype(np.uint64))
        cur = nxt
    mi = host(rm.max_index).astype(np.int64)
    return [(cur[p][mi] - u(x[p])).astype(np.uint64) for p in (0, 1)]


def spline2(prg, gate, x, idx0=0, sl=None):
    """spline.SplineGate (CubicPolyTask) on shares x = (x0, x1): both
    parties' outputs.  sl: a slice of the gate's batch (x holds that slice;
    idx0 = its first element index, the LUT keystream counter uses it)."""
    x0, x1 = u(x[0]), u(x[1])
    n = x0.size
    sl = sl if sl is not None else slice(0, n)
    f = gate.f
    rin = sum(gate.rin) & M64
    xhat = (x0 + x1 + np.uint64(rin)).astype(np.uint64)
    lut = [host(gate.lut[p]) for p in (0, 1)]
    C = [ol.lut_eval(lut[p], gate.lut_key_bytes, 1, xhat, 4, idx0=idx0).reshape(n, 4)
         for p in (0, 1)]
    tri = [[host(t).view(np.uint64).reshape(-1, 3)[sl] for t in pr] for pr in gate.triples]

    def mul(a, b, t):
        d = (a[0] - t[0][:, 0]) + (a[1] - t[1][:, 0])
        e = (b[0] - t[0][:, 1]) + (b[1] - t[1][:, 1])
        return [ol.beaver_mul(p, t[p][:, 0], t[p][:, 1], t[p][:, 2], d, e) for p in (0, 1)]

    sh = np.uint64(f)
    m1 = mul([C[0][:, 3], C[1][:, 3]], [x0, x1], tri[0])
    m1 = [m1[p] + (C[p][:, 2] << sh) for p in (0, 1)]
    pz = mul(m1, [x0, x1], tri[1])
    t1, t2, t3 = gate.trunc
    y = trunc2(prg, t1, open2(pz, t1.mask))
    q = [y[p] + (C[p][:, 1] << sh) for p in (0, 1)]
    rz = mul(q, [x0, x1], tri[2])
    y2 = trunc2(prg, t2, open2(rz, t2.mask))
    z3 = [(y2[p] + (C[p][:, 0] << sh)).astype(np.uint64) for p in (0, 1)]
    return trunc2(prg, t3, open2(z3, t3.mask))


def softmax2(prg, sm, x):
    """softmax.SoftmaxBlock on shares x: (prob shares, stage shares)."""
    offs = sm.offsets
    row = np.repeat(np.arange(len(offs) - 1), np.diff(offs))
    delta = relu_rounds2(sm.rowmax, x)
    e = spline2(prg, sm.nexp, delta)
    s = [ol.row_sum_ragged(e[p], offs.astype(np.int32)) for p in (0, 1)]
    inv = recip2(prg, sm.recip, s, open2(s, sm.recip.lut.mask))
    prob = beaver_trunc2(prg, e, inv, sm.tri, sm.tr, row_of=row)
    return prob, {"delta": delta, "exp": e, "sum": s, "inv": inv}


def layernorm2(prg, ln, x):
    """layernorm.LayerNormBlock on shares x: output shares."""
    rows, cols = ln.rows, ln.cols
    row = np.repeat(np.arange(rows), cols)
    xs = [u(x[0]), u(x[1])]
    sums = [(ol.row_sum(xs[p], rows, cols) * np.uint64(ln.inv_len)).astype(np.uint64)
            for p in (0, 1)]
    mu = trunc2(prg, ln.tr_mean, open2(sums, ln.tr_mean.mask))
    diff = [(xs[p] - mu[p][row]).astype(np.uint64) for p in (0, 1)]
    sq = beaver2(diff, diff, ln.tri_sq)
    vs = [(ol.row_sum(sq[p], rows, cols) * np.uint64(ln.inv_len)).astype(np.uint64)
          for p in (0, 1)]
    va = trunc2(prg, ln.tr_var[0], open2(vs, ln.tr_var[0].mask))
    var = trunc2(prg, ln.tr_var[1], open2(va, ln.tr_var[1].mask))
    v = const2(var, ln.eps_q)
    rs = rsqrt2(prg, ln.rsqrt, v, open2(v, ln.rsqrt.lut.mask))
    return beaver_trunc2(prg, diff, rs, ln.tri_norm, ln.tr_norm, row_of=row)


def public_trunc2(prg, pm, x, add=None):
    """layer.PublicMatmulTrunc: trunc_f(X_p W) for both parties (the masked
    open Y_0 + Y_1 + r into the gate), plus the pair `add` (a residual)."""
    M, K, N = pm.M, pm.K, pm.N
    y = [ol.matmul_public(u(x[p]), pm.W, M, K, N) for p in (0, 1)]
    out = trunc2(prg, pm.tr, open2(y, pm.tr.mask))
    return out if add is None else add2(out, add)


def _batched_beaver2(tri, D, E):
    """Both parties' products C_p + D B_p + A_p E (+ D E, party 0) per batch
    of a layer.BatchedTriples, for the opens D [b][M x K], E [b][K x N]."""
    b, M, K, N = tri.shape
    A, B, C, A0, B0, C0 = tri.host
    sh = [(A0, B0, C0), ((A - A0).astype(np.uint64), (B - B0).astype(np.uint64),
                         (C - C0).astype(np.uint64))]
    D = u(D).reshape(b, M * K)
    E = u(E).reshape(b, K * N)
    out = []
    for p in (0, 1):
        a, bb, c = (np.ascontiguousarray(v, dtype=np.uint64).reshape(b, -1) for v in sh[p])
        z = np.empty((b, M * N), dtype=np.uint64)
        for h in range(b):
            z[h] = ol.beaver_matmul(p, D[h], E[h], a[h], bb[h], c[h], 1, M, K, N, threads=0)
        out.append(z.ravel())
    return out


def attention2(prg, at, qkv):
    """layer.AttentionCore on the QKV shares [seq x 3d]: the context shares
    [seq x d], and the stages."""
    mp = {k: host(v).astype(np.int64) for k, v in at.maps.items()}
    q = [u(qkv[p])[mp["gq"]] for p in (0, 1)]
    k = [u(qkv[p])[mp["gk"]] for p in (0, 1)]
    v = [u(qkv[p])[mp["gv"]] for p in (0, 1)]
    A_qk = at.tri_qk.host[3], (at.tri_qk.host[0] - at.tri_qk.host[3]).astype(np.uint64)
    B_qk = at.tri_qk.host[4], (at.tri_qk.host[1] - at.tri_qk.host[4]).astype(np.uint64)
    A_pv = at.tri_pv.host[3], (at.tri_pv.host[0] - at.tri_pv.host[3]).astype(np.uint64)
    B_pv = at.tri_pv.host[4], (at.tri_pv.host[1] - at.tri_pv.host[4]).astype(np.uint64)
    D = ((q[0] - A_qk[0].ravel()) + (q[1] - A_qk[1].ravel())).astype(np.uint64)
    E = ((k[0] - B_qk[0].ravel()) + (k[1] - B_qk[1].ravel())).astype(np.uint64)
    E2 = ((v[0] - B_pv[0].ravel()) + (v[1] - B_pv[1].ravel())).astype(np.uint64)
    S = _batched_beaver2(at.tri_qk, D, E)
    sc = [(S[p][mp["gs"]] * np.uint64(at.inv_sqrt)).astype(np.uint64) for p in (0, 1)]
    sa = trunc2(prg, at.tr_s[0], open2(sc, at.tr_s[0].mask))
    scores = trunc2(prg, at.tr_s[1], open2(sa, at.tr_s[1].mask))
    prob, _ = softmax2(prg, at.softmax, scores)
    pz = [np.concatenate([prob[p], np.zeros(1, np.uint64)]) for p in (0, 1)]
    pd = [pz[p][mp["gp"]] for p in (0, 1)]
    D2 = ((pd[0] - A_pv[0].ravel()) + (pd[1] - A_pv[1].ravel())).astype(np.uint64)
    Z = _batched_beaver2(at.tri_pv, D2, E2)
    zc = [Z[p][mp["gc"]] for p in (0, 1)]
    ctx = trunc2(prg, at.tr_c, open2(zc, at.tr_c.mask))
    return ctx, {"scores": scores, "prob": prob}


def layer2(prg, ly, x):
    """layer.TransformerLayer on the input shares x [seq x d]: the output
    shares and the stages, in the order the layer runs its protocol steps."""
    h1 = layernorm2(prg, ly.ln1, x)
    qkv = public_trunc2(prg, ly.qkv, h1)
    ctx, st = attention2(prg, ly.attn, qkv)
    r1 = public_trunc2(prg, ly.proj, ctx, add=x)
    h2 = layernorm2(prg, ly.ln2, r1)
    uu = public_trunc2(prg, ly.w1, h2)
    g = spline2(prg, ly.gelu, uu)
    out = public_trunc2(prg, ly.w2, g, add=r1)
    st.update({"h1": h1, "qkv": qkv, "ctx": ctx, "r1": r1, "h2": h2, "u": uu, "g": g})
    return out, st


def composite_bool2(g, pred, cut):
    """Both parties' [n][l] additive boolean outputs of a
    composite.CompositeGate from the XOR-shared bits pred[p] ([Q][n] uint8)
    and cut[p] ([C][n]): b2a of the cut bits and the one-hot selectors
    (selectors_from_cutbits_block, include/gates/composite_fss.hpp:893-974),
    each segment's boolean programs over XOR shares (eval_bool_xor_view,
    include/gates/bool_dag_xor.hpp:13-104, with a constant held by party 0),
    b2a of the output bits and the selector-weighted sum
    (composite_fss.hpp:2132-2200), every product on the gate's triple of its
    index."""
    n, C, ell = g.n, len(g.cuts), g.ell
    S = C + 1
    tri = [host(g.tri[p]).view(np.uint64).reshape(g.T, 3, n) for p in (0, 1)]
    bt = [host(g.bit_tri[p]).reshape(g.and_count, n) if g.and_count else None for p in (0, 1)]
    one, zero = np.ones(n, np.uint64), np.zeros(n, np.uint64)

    def mul(t, x, y):
        a = [tri[p][t, 0] for p in (0, 1)]
        b = [tri[p][t, 1] for p in (0, 1)]
        c = [tri[p][t, 2] for p in (0, 1)]
        d = ((u(x[0]) - a[0]) + (u(x[1]) - a[1])).astype(np.uint64)
        e = ((u(y[0]) - b[0]) + (u(y[1]) - b[1])).astype(np.uint64)
        return [(c[0] + d * b[0] + e * a[0] + d * e).astype(np.uint64),
                (c[1] + d * b[1] + e * a[1]).astype(np.uint64)]

    def b2a(t, b0, b1):
        b0, b1 = u(b0 & 1), u(b1 & 1)
        z = mul(t, [b0, zero], [zero, b1])
        return [(b0 - np.uint64(2) * z[0]).astype(np.uint64),
                (b1 - np.uint64(2) * z[1]).astype(np.uint64)]

    cut_add = [b2a(k, cut[0][k].astype(np.uint64), cut[1][k].astype(np.uint64))
               for k in range(C)]
    B = max(0, 2 * C - 1)
    and_idx = 0
    out = [np.zeros((n, ell), np.uint64), np.zeros((n, ell), np.uint64)]
    for s in range(S):
        if C == 0:
            sel = [one, zero]
        elif s == 0:
            sel = cut_add[0]
        elif s == C:
            sel = [(one - cut_add[C - 1][0]).astype(np.uint64),
                   (zero - cut_add[C - 1][1]).astype(np.uint64)]
        else:
            sel = mul(C + s - 1, [(one - cut_add[s - 1][0]).astype(np.uint64),
                                  (zero - cut_add[s - 1][1]).astype(np.uint64)], cut_add[s])
        for j in range(ell):
            k = s * ell + j
            stack = []
            for ins in g.prog[g.prog_off[k]:g.prog_off[k + 1]]:
                op, arg = ins & 0xF, ins >> 4
                if op == 0:  # query bit
                    stack.append([pred[0][arg] & 1, pred[1][arg] & 1])
                elif op == 1:  # wrap: low bit of the additive share
                    stack.append([np.full(n, int(g.wrap_share[p][arg]) & 1, np.uint8)
                                  for p in (0, 1)])
                elif op == 2:  # constant on party 0's share
                    stack.append([np.full(n, arg & 1, np.uint8), np.zeros(n, np.uint8)])
                elif op == 3:  # NOT
                    stack[-1] = [stack[-1][0] ^ 1, stack[-1][1]]
                else:
                    y = stack.pop()
                    x = stack.pop()
                    r = [x[0] ^ y[0], x[1] ^ y[1]]
                    if op in (5, 6):  # AND / OR: one bit triple
                        t = [bt[p][and_idx] for p in (0, 1)]
                        and_idx += 1
                        a = [t[p] & 1 for p in (0, 1)]
                        b = [(t[p] >> 1) & 1 for p in (0, 1)]
                        c = [(t[p] >> 2) & 1 for p in (0, 1)]
                        e = x[0] ^ x[1] ^ a[0] ^ a[1]
                        f = y[0] ^ y[1] ^ b[0] ^ b[1]
                        z = [c[0] ^ (e & b[0]) ^ (f & a[0]) ^ (e & f), c[1] ^ (e & b[1]) ^ (f & a[1])]
                        r = z if op == 5 else [r[0] ^ z[0], r[1] ^ z[1]]
                    stack.append(r)
            assert len(stack) == 1
            bx = stack[0]
            badd = b2a(B + k, bx[0].astype(np.uint64), bx[1].astype(np.uint64))
            z = mul(B + S * ell + k, sel, badd)
            out[0][:, j] += z[0]
            out[1][:, j] += z[1]
    return out
