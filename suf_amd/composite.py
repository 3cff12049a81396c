"""Composite SUF gates with boolean outputs (l_out > 0) for two parties on one
GPU: dealer compilation, key material, and the online evaluation.

A gate is a SUF (include/suf/suf_ir.hpp): piece starts `alpha` over x
(alpha[0] = 0, the last piece runs to 2^64), per piece r constant
arithmetic words and l boolean expressions over primitive predicates
(include/suf/predicates.hpp, include/suf/bool_expr.hpp):

  predicates  ("lt", beta)         1[x < beta]
              ("ltlow", f, gamma)  1[x mod 2^f < gamma]
              ("msb",)             MSB(x)
              ("msb_add", c)       MSB(x + c)
  expressions ("const", b) ("var", i) ("not", e) ("xor", a, b)
              ("and", a, b) ("or", a, b)

Dealer (compile_suf_to_pfss_two_programs, src/compiler/suf_to_pfss.cpp:
300-554, with the mask rewrite of include/suf/mask_rewrite.hpp):
  * each predicate occurrence becomes a rotated-interval membership
    a XOR b XOR w over two comparison queries a = 1[x^ < theta0],
    b = 1[x^ < theta1] (queries shared between occurrences) and a fresh
    secret-shared wrap bit w = 1[theta1 < theta0] (suf_to_pfss.cpp:38-95);
  * the pieces rotated by r_in and split at the wrap, sorted, give the
    x^-domain segments; their starts after the first are the cut queries
    1[x^ < cut_k] of the selector network, and each segment evaluates the
    boolean outputs of the piece it comes from;
  * one broadcast myl7 DCF key pair (payload 1, XOR group) per query and per
    cut; bit triples for AND / OR; Beaver triples for the network.
Online: the DCF bits of every query and cut at the public x^ (one launch per
key and party), the whole selector / boolean network for both parties in one
launch (sufhip_composite_bool2), and the arithmetic words through the
interval LUT of the rotated pieces (sufhip_interval_lut_eval2).
"""
import numpy as np
import torch

from . import native, pfss
from .tasks import CoeffLut, Dealer, ptr, stream_ptr

M64 = (1 << 64) - 1
TOP = 1 << 63


def _rewrite_pred(p, r, queries, qmap, wraps):
    """(bits, theta0, theta1, wrap) of one predicate under the mask r_in
    (rewrite_lt_u64, rewrite_ltlow, rewrite_msb_add), as the membership
    expression over query and wrap indices."""
    kind = p[0]
    if kind == "lt":
        bits, t0 = 64, r
        t1 = (t0 + p[1]) & M64
    elif kind == "ltlow":
        f = int(p[1])
        m = M64 if f >= 64 else (1 << f) - 1
        bits, t0 = f, r & m
        t1 = (t0 + p[2]) & m
    elif kind in ("msb", "msb_add"):
        c = int(p[1]) if kind == "msb_add" else 0
        bits, t0 = 64, (r + TOP - c) & M64
        t1 = (t0 + TOP) & M64
    else:
        raise ValueError("unknown predicate %r" % (p,))

    def query(theta):
        key = (bits, theta)
        if key not in qmap:
            qmap[key] = len(queries)
            queries.append(key)
        return qmap[key]

    a, b = query(t0), query(t1)
    w = len(wraps)
    wraps.append(1 if t1 < t0 else 0)
    return ("xor", ("xor", ("q", a), ("q", b)), ("w", w))


def _rewrite(e, preds, r, queries, qmap, wraps):
    op = e[0]
    if op == "const":
        return e
    if op == "var":
        i = int(e[1])
        if i < 0 or i >= len(preds):
            return ("const", 0)
        return _rewrite_pred(preds[i], r, queries, qmap, wraps)
    if op == "not":
        return ("not", _rewrite(e[1], preds, r, queries, qmap, wraps))
    if op in ("xor", "and", "or"):
        return (op, _rewrite(e[1], preds, r, queries, qmap, wraps),
                _rewrite(e[2], preds, r, queries, qmap, wraps))
    raise ValueError("unknown expression %r" % (e,))


_OPS = {"q": native.BOOL_VAR, "w": native.BOOL_WRAP, "const": native.BOOL_CONST,
        "not": native.BOOL_NOT, "xor": native.BOOL_XOR, "and": native.BOOL_AND,
        "or": native.BOOL_OR}


def postfix(e, out):
    """Appends the instructions of a rewritten expression (left operand
    first: the order in which eval_bool_xor_view consumes bit triples)."""
    op = e[0]
    if op in ("q", "w", "const"):
        out.append(_OPS[op] | (int(e[1]) << 4))
    elif op == "not":
        postfix(e[1], out)
        out.append(_OPS[op])
    else:
        postfix(e[1], out)
        postfix(e[2], out)
        out.append(_OPS[op])
    return out


def segments(alpha, r):
    """The pieces [alpha_i, alpha_{i+1}) rotated by r, split at the wrap,
    sorted by start: [(start, piece)] with start[0] = 0."""
    bounds = [int(a) for a in alpha] + [1 << 64]
    segs = []
    for i in range(len(alpha)):
        if bounds[i + 1] <= bounds[i]:
            continue
        s = (bounds[i] + r) & M64
        e = (bounds[i + 1] + r) & M64
        if bounds[i + 1] - bounds[i] == 1 << 64:
            segs.append((0, i))
        elif s < e or e == 0:
            segs.append((s, i))
        else:
            segs.append((s, i))
            segs.append((0, i))
    segs.sort()
    return segs


def compile_bools(spec, r_in):
    """The boolean half of the dealer's compilation for mask r_in: the
    comparison queries [(bits, theta)], the wrap bits, the x^ segments
    [(start, piece)], the postfix programs (segment s, output j at
    prog[off[s l + j]:off[s l + j + 1]]) and their AND / OR count."""
    pieces = spec["pieces"]
    ell = len(pieces[0]["bools"])
    queries, qmap, wraps = [], {}, []
    rewritten = [[_rewrite(e, spec["preds"], r_in, queries, qmap, wraps) for e in p["bools"]]
                 for p in pieces]
    segs = segments(np.asarray(spec["alpha"], dtype=np.uint64), r_in)
    prog, offs = [], [0]
    for _, piece in segs:
        for j in range(ell):
            postfix(rewritten[piece][j], prog)
            offs.append(len(prog))
    ands = sum(1 for ins in prog if ins & 0xF in (native.BOOL_AND, native.BOOL_OR))
    return queries, wraps, segs, prog, offs, ands


class CompositeGate:
    """Dealer material of one composite gate over n elements, both parties,
    on the GPU.  spec: {"alpha": [...], "preds": [...], "pieces": [{"arith":
    [r words], "bools": [l expressions]}]}."""

    def __init__(self, spec, n, prg_state, seed=1, device="cuda"):
        self.n = n
        self.prg_state = bytes(prg_state)
        self.spec = spec
        alpha = np.asarray(spec["alpha"], dtype=np.uint64)
        pieces = spec["pieces"]
        self.r = len(pieces[0]["arith"])
        self.ell = len(pieces[0]["bools"])
        if not 1 <= self.ell <= native.COMPOSITE_MAX_ELL:
            raise ValueError("CompositeGate: 1 to %d boolean outputs" % native.COMPOSITE_MAX_ELL)
        dealer = Dealer(seed)
        # Arithmetic words: the interval LUT of the rotated pieces; its mask
        # is the gate's r_in.
        coeffs = np.array([[int(w) & M64 for w in p["arith"]] for p in pieces],
                          dtype=np.uint64).view(np.int64)
        self.lut = CoeffLut(dealer, alpha, coeffs, device) if self.r > 0 else None
        self.r_in = self.lut.mask if self.lut is not None else dealer.word()
        queries, wraps, segs, prog, offs, ands = compile_bools(spec, self.r_in)
        if len(segs) - 1 > native.COMPOSITE_MAX_CUTS:
            raise ValueError("CompositeGate: too many x^ segments")
        if len(wraps) > native.COMPOSITE_MAX_WRAP:
            raise ValueError("CompositeGate: too many wrap bits")
        if len(prog) > native.COMPOSITE_MAX_PROG:
            raise ValueError("CompositeGate: boolean programs too long")
        self.segs = segs
        self.cuts = [s for s, _ in segs[1:]]
        self.queries = queries
        self.wrap_bits = wraps
        self.prog, self.prog_off = prog, offs
        self.and_count = ands
        # Wrap bits, additively shared.
        w0 = dealer.words(max(1, len(wraps)))[:len(wraps)]
        self.wrap_share = [np.array(w0, dtype=np.uint64),
                           (np.array(wraps, dtype=np.uint64) - np.array(w0, dtype=np.uint64))
                           .astype(np.uint64)]
        # One broadcast DCF key pair per query and per cut.
        self.query_keys = [self._dcf_key(dealer, bits, theta, device) for bits, theta in queries]
        self.cut_keys = [self._dcf_key(dealer, 64, c, device) for c in self.cuts]
        # Bit triples: random XOR shares of a, b and of c = a AND b.
        if self.and_count:
            w = dealer.words(self.and_count * n * 3).reshape(3, self.and_count, n)
            a0, b0, c0 = (w[k] & np.uint64(1) for k in range(3))
            w2 = dealer.words(self.and_count * n * 2).reshape(2, self.and_count, n)
            a, b = w2[0] & np.uint64(1), w2[1] & np.uint64(1)
            c = a & b
            pack = lambda x, y, z: (x | (y << np.uint64(1)) | (z << np.uint64(2))).astype(np.uint8)
            self.bit_tri = [torch.from_numpy(pack(a0, b0, c0).ravel()).to(device),
                            torch.from_numpy(pack(a ^ a0, b ^ b0, c ^ c0).ravel()).to(device)]
        else:
            self.bit_tri = [None, None]
        # Beaver triples [T][3][n] per party.
        T = native.load().sufhip_composite_bool_triples(len(self.cuts), self.ell)
        self.T = T
        w = dealer.words(T * n * 5).reshape(5, T, n)
        a, b, a0, b0, c0 = w
        c = a * b
        t0 = np.stack([a0, b0, c0], axis=1)
        t1 = np.stack([a - a0, b - b0, c - c0], axis=1)
        self.tri = [torch.from_numpy(t.view(np.int64).ravel().copy()).to(device) for t in (t0, t1)]
        self.pred = [torch.empty(max(1, len(queries)) * n, dtype=torch.uint8, device=device)
                     for _ in range(2)]
        self.cutb = [torch.empty(max(1, len(self.cuts)) * n, dtype=torch.uint8, device=device)
                     for _ in range(2)]

    def _dcf_key(self, dealer, bits, theta, device):
        seeds = torch.from_numpy(dealer.words(4).view(np.uint8).copy()).to(device).reshape(1, 32)
        alpha = torch.tensor([int(theta) - (1 << 64) if int(theta) >> 63 else int(theta)],
                             dtype=torch.int64, device=device)
        one = torch.ones(1, dtype=torch.uint8, device=device)
        k0, k1 = pfss.dcf_gen(native.GROUP_XOR, bits, self.prg_state, alpha, one, seeds)
        return (bits, k0, k1)

    def pred_bits(self, xhat):
        """Both parties' XOR-shared bits of every query and cut at x^ (int64[n])."""
        n = self.n
        for q, (bits, k0, k1) in enumerate(self.query_keys):
            for p, k in ((0, k0), (1, k1)):
                pfss.dcf_eval(native.GROUP_XOR, bits, 1, self.prg_state, k, xhat, broadcast=True,
                              out=self.pred[p][q * n:(q + 1) * n])
        for c, (bits, k0, k1) in enumerate(self.cut_keys):
            for p, k in ((0, k0), (1, k1)):
                pfss.dcf_eval(native.GROUP_XOR, bits, 1, self.prg_state, k, xhat, broadcast=True,
                              out=self.cutb[p][c * n:(c + 1) * n])

    def args(self, out_bool):
        a = native.CompositeBoolArgs()
        a.n, a.queries, a.cuts, a.ell = self.n, len(self.queries), len(self.cuts), self.ell
        a.wraps, a.and_count, a.prog_len = len(self.wrap_bits), self.and_count, len(self.prog)
        for p in (0, 1):
            a.pred[p] = ptr(self.pred[p]) if self.queries else None
            a.cut[p] = ptr(self.cutb[p]) if self.cuts else None
            a.bit_tri[p] = ptr(self.bit_tri[p]) if self.and_count else None
            a.tri[p] = ptr(self.tri[p])
            a.out[p] = ptr(out_bool[p])
            for w, v in enumerate(self.wrap_share[p]):
                a.wrap[p][w] = int(v)
        for k, o in enumerate(self.prog_off):
            a.prog_off[k] = o
        for k, ins in enumerate(self.prog):
            a.prog[k] = ins
        return a

    def eval2(self, xhat, out_bool, out_arith=None):
        """xhat: the public masked inputs x + r_in (int64[n], device).
        out_bool: pair of int64 [n * l] (additive shares, [n][l]); out_arith:
        pair of int64 [n * r] (the pieces' words, additive shares)."""
        self.pred_bits(xhat)
        a = self.args(out_bool)
        native.call("sufhip_composite_bool2", native.ctypes.byref(a), stream_ptr())
        if out_arith is not None and self.lut is not None:
            self.lut.eval2(xhat, self.n, out_arith)
        return out_bool


def stage_bucket(jobs, bucket=None, device="cuda"):
    """Concatenates jobs' masked inputs into one device buffer in one launch
    (sufhip_stage_hatx): jobs of int64 device tensors, or (packed int64
    tensor, eff_bits, length) for eff_bits-packed uploads.  Returns the
    bucket and each job's (start, length)."""
    segs = (native.StageSeg * len(jobs))()
    slices, pos = [], 0
    for k, j in enumerate(jobs):
        if isinstance(j, tuple):
            t, eb, ln = j
        else:
            t, eb, ln = j, 64, j.numel()
        segs[k].src, segs[k].len, segs[k].dst, segs[k].eff_bits = ptr(t), ln, pos, eb
        slices.append((pos, ln))
        pos += ln
    if bucket is None:
        bucket = torch.empty(max(1, pos), dtype=torch.int64, device=device)
    native.call("sufhip_stage_hatx", segs, len(jobs), ptr(bucket), bucket.numel(), stream_ptr())
    return bucket, slices
