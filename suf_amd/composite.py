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

Offline key material travels as one composite tape per party
(gates::write_composite_tape, composite_fss.hpp:2458-2641; suf_amd/tape.py):
party_tape(p) writes it, and CompositeGate.from_tapes(compiled(), tapes)
rebuilds the gate's device key material from the two tapes and the dealer's
public compilation, as composite_eval_batch_from_tape pairs a tape with the
CompiledSUFGate (composite_fss.hpp:2622-2641).
"""
import numpy as np
import torch

from . import native, pfss
from . import tape as tapefmt
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
        # The mask's shares (the tapes' r_in_share), drawn last so that the
        # material above does not depend on them.
        s0 = dealer.word()
        self.r_in_share = [s0, (self.r_in - s0) & M64]
        self._buffers(device)

    def _buffers(self, device):
        n = self.n
        self.pred = [torch.empty(max(1, len(self.queries)) * n, dtype=torch.uint8, device=device)
                     for _ in range(2)]
        self.cutb = [torch.empty(max(1, len(self.cuts)) * n, dtype=torch.uint8, device=device)
                     for _ in range(2)]

    def compiled(self):
        """The dealer's public compilation (CompiledSUFGate's role): what the
        evaluation needs besides the parties' key material."""
        lut = None
        if self.lut is not None:
            lut = {"intervals": int(self.lut.intervals), "words": int(self.lut.words),
                   "key_bytes": int(self.lut.key_bytes), "mask": int(self.lut.mask)}
        return {"n": self.n, "r": self.r, "ell": self.ell, "r_in": int(self.r_in),
                "queries": [(int(b), int(t)) for b, t in self.queries],
                "cuts": [int(c) for c in self.cuts], "segs": list(self.segs),
                "wraps": len(self.wrap_bits), "prog": list(self.prog),
                "prog_off": list(self.prog_off), "and_count": self.and_count, "T": self.T,
                "lut": lut, "spec": self.spec}

    def party_key(self, p):
        """Party p's key material as a composite tape key (suf_amd/tape.py):
        the mask and wrap shares, one DCF key per query and per cut (XOR
        bytes, 1-byte payload, MSB-first), the interval-LUT blob of the
        arithmetic words (additive), T x n Beaver triples {a, b, c} (triple t
        of element i at t n + i) and and_count x n bit triples."""
        n = self.n
        k = tapefmt.empty_key()
        k["r_in_share"] = self.r_in_share[p]
        k["wrap_share"] = np.asarray(self.wrap_share[p], dtype=np.uint64)
        k["pred_keys"] = [bytes(kp[1 + p].cpu().numpy().tobytes()) for kp in self.query_keys]
        k["cut_pred_keys"] = [bytes(kp[1 + p].cpu().numpy().tobytes()) for kp in self.cut_keys]
        if self.lut is not None:
            k["coeff_keys"] = [bytes(self.lut.blobs[p].tobytes())]
        tri = self.tri[p].cpu().numpy().view(np.uint64).reshape(self.T, 3, n)
        k["triples"] = tri.transpose(0, 2, 1).reshape(self.T * n, 3)
        if self.and_count:
            bt = self.bit_tri[p].cpu().numpy()
            k["bit_triples"] = np.stack([bt & 1, (bt >> 1) & 1, (bt >> 2) & 1], axis=1)
        return k

    def party_tape(self, p):
        """Party p's composite tape (bytes)."""
        return tapefmt.write_composite_tape(self.party_key(p))

    @classmethod
    def from_tapes(cls, compiled, tapes, prg_state, device="cuda"):
        """A gate whose key material comes from the two parties' composite
        tapes (bytes), evaluated under the dealer's compilation `compiled`
        (CompositeGate.compiled()).  Raises ValueError if a tape does not fit
        the compilation."""
        c = compiled
        g = cls.__new__(cls)
        g.n, g.r, g.ell, g.r_in = c["n"], c["r"], c["ell"], c["r_in"]
        g.prg_state = bytes(prg_state)
        g.spec = c.get("spec")
        g.queries = [tuple(q) for q in c["queries"]]
        g.cuts, g.segs = list(c["cuts"]), list(c["segs"])
        g.prog, g.prog_off = list(c["prog"]), list(c["prog_off"])
        g.and_count, g.T = c["and_count"], c["T"]
        n = g.n
        keys = [tapefmt.read_composite_tape(t) for t in tapes]
        for p, k in enumerate(keys):
            def bad(what):
                return ValueError("CompositeGate.from_tapes: party %d tape: %s" % (p, what))
            if len(k["pred_keys"]) != len(g.queries) or len(k["cut_pred_keys"]) != len(g.cuts):
                raise bad("key counts differ from the compilation")
            if k["pred_meta"][1:] != (tapefmt.XOR_BYTES, 1) or \
                    k["cut_pred_meta"][1:] != (tapefmt.XOR_BYTES, 1):
                raise bad("predicate keys must be XOR bytes with a 1-byte output")
            if len(k["wrap_share"]) != c["wraps"]:
                raise bad("wrap share count")
            if k["triples"].shape[0] != g.T * n or k["bit_triples"].shape[0] != g.and_count * n:
                raise bad("triple counts")
            if len(k["coeff_keys"]) != (1 if c["lut"] else 0):
                raise bad("coefficient key count")
            for blob, (bits, _) in zip(k["pred_keys"], g.queries):
                if len(blob) != pfss.dcf_key_bytes(bits, 1) or blob[0] != bits:
                    raise bad("a predicate key has the wrong size or input width")
            for blob in k["cut_pred_keys"]:
                if len(blob) != pfss.dcf_key_bytes(64, 1) or blob[0] != 64:
                    raise bad("a cut key has the wrong size or input width")
        g.r_in_share = [k["r_in_share"] for k in keys]
        g.wrap_bits = [None] * c["wraps"]  # clear bits stay with the dealer
        g.wrap_share = [np.asarray(k["wrap_share"], dtype=np.uint64) for k in keys]

        def dev_bytes(blob):
            return torch.from_numpy(np.frombuffer(blob, dtype=np.uint8).copy()).to(device)

        g.query_keys = [(bits, dev_bytes(keys[0]["pred_keys"][q]), dev_bytes(keys[1]["pred_keys"][q]))
                        for q, (bits, _) in enumerate(g.queries)]
        g.cut_keys = [(64, dev_bytes(keys[0]["cut_pred_keys"][q]),
                       dev_bytes(keys[1]["cut_pred_keys"][q])) for q in range(len(g.cuts))]
        g.tri = []
        for k in keys:
            t = k["triples"].reshape(g.T, n, 3).transpose(0, 2, 1)
            g.tri.append(torch.from_numpy(np.ascontiguousarray(t).view(np.int64).ravel().copy())
                         .to(device))
        if g.and_count:
            g.bit_tri = []
            for k in keys:
                bt = k["bit_triples"].astype(np.uint8)
                packed = (bt[:, 0] & 1) | ((bt[:, 1] & 1) << 1) | ((bt[:, 2] & 1) << 2)
                g.bit_tri.append(torch.from_numpy(packed.astype(np.uint8)).to(device))
        else:
            g.bit_tri = [None, None]
        g.lut = None
        if c["lut"]:
            lut = CoeffLut.__new__(CoeffLut)
            lut.words, lut.intervals = c["lut"]["words"], c["lut"]["intervals"]
            lut.key_bytes, lut.mask = c["lut"]["key_bytes"], c["lut"]["mask"]
            lut.blobs = [np.frombuffer(k["coeff_keys"][0], dtype=np.uint8).copy() for k in keys]
            if any(b.size != lut.key_bytes for b in lut.blobs):
                raise ValueError("CompositeGate.from_tapes: coefficient key size")
            lut.keys = [torch.from_numpy(b.view(np.int64).copy()).to(device).view(torch.uint8)
                        for b in lut.blobs]
            g.lut = lut
        g._buffers(device)
        return g

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
