"""Plaintext evaluation of a SUF (include/suf/ref_eval.hpp:11-78): what a
composite gate's two-party outputs must reconstruct to.

TEST INFRASTRUCTURE ONLY: the checker (tests/ and bench.py's CPU leg).

A spec is {"alpha": piece starts (alpha[0] = 0; the last piece runs to
2^64), "preds": primitive predicates, "pieces": [{"arith": [words],
"bools": [expressions]}]} with
  predicates  ("lt", beta) ("ltlow", f, gamma) ("msb",) ("msb_add", c)
              (eval_primitive, ref_eval.hpp:11-28)
  expressions ("const", b) ("var", i) ("not", e) ("xor", a, b) ("and", a, b)
              ("or", a, b) (eval_bool_expr, include/suf/bool_expr.hpp:62-92;
              a variable outside the predicate list is false)
and the piece of x is the i with alpha_i <= x < alpha_{i+1}, else the last
(select_interval, ref_eval.hpp:47-56).  The arithmetic outputs are the
pieces' degree-0 words.  Vectorised over a u64 numpy array x.

Pinned by tests/golden/suf_ref_eval.json, which the reference's own
eval_suf_ref writes for two gates (tests/golden/make_suf_ref.py).
"""
import numpy as np

M64 = (1 << 64) - 1


def eval_primitive(p, x):
    x = np.asarray(x, dtype=np.uint64)
    kind = p[0]
    if kind == "lt":
        return x < np.uint64(p[1])
    if kind == "ltlow":
        f = int(p[1])
        if f >= 64:
            return x < np.uint64(p[2])
        return (x & np.uint64((1 << f) - 1)) < np.uint64(p[2])
    if kind == "msb":
        return (x >> np.uint64(63)) != 0
    if kind == "msb_add":
        return ((x + np.uint64(p[1] & M64)) >> np.uint64(63)) != 0
    raise ValueError("unknown predicate %r" % (p,))


def eval_bool(e, prims, n):
    op = e[0]
    if op == "const":
        return np.full(n, bool(e[1]))
    if op == "var":
        i = int(e[1])
        return prims[i] if 0 <= i < len(prims) else np.zeros(n, dtype=bool)
    if op == "not":
        return ~eval_bool(e[1], prims, n)
    a, b = eval_bool(e[1], prims, n), eval_bool(e[2], prims, n)
    if op == "xor":
        return a ^ b
    if op == "and":
        return a & b
    if op == "or":
        return a | b
    raise ValueError("unknown expression %r" % (e,))


def piece_index(alpha, x):
    """select_interval over the boundaries alpha + [2^64 as the ~0 surrogate
    of the reference's lists]: x in [alpha_i, alpha_{i+1}) -> i; x = 2^64 - 1
    falls outside the last [alpha_{m-1}, ~0) and takes the last piece too."""
    a = np.asarray(alpha, dtype=np.uint64)
    return np.searchsorted(a, np.asarray(x, dtype=np.uint64), side="right") - 1


def eval_suf(spec, x):
    """(arith [n][r] u64, bools [n][l] bool, piece [n])."""
    x = np.asarray(x, dtype=np.uint64)
    n = x.size
    piece = piece_index(spec["alpha"], x)
    prims = [eval_primitive(p, x) for p in spec["preds"]]
    pieces = spec["pieces"]
    r, l = len(pieces[0]["arith"]), len(pieces[0]["bools"])
    arith = np.zeros((n, r), dtype=np.uint64)
    bools = np.zeros((n, l), dtype=bool)
    for k, pc in enumerate(pieces):
        sel = piece == k
        if not sel.any():
            continue
        for j in range(r):
            arith[sel, j] = np.uint64(int(pc["arith"][j]) & M64)
        for j in range(l):
            bools[sel, j] = eval_bool(pc["bools"][j], prims, n)[sel]
    return arith, bools, piece
