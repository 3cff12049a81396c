"""A GPT-2-shaped secure transformer layer for two parties on one GPU.

transformer_layer_forward (src/nn/transformer_layer.cpp:435-830) with
attention_forward (src/nn/attention_block.cpp:931-1900, causal prefill) and
mlp_forward (src/nn/mlp_block.cpp:378-767):

  h1  = LayerNorm(x)
  qkv = trunc_f(h1 Wqkv)                      public weights, MFMA digit GEMM
  s   = trunc_2f(inv_sqrt * Q_h K_h^T)        Beaver per head, causal rows packed
                                              (2f as two f-bit truncations)
  p   = Softmax(s)                            suf_amd.softmax.SoftmaxBlock
  c   = trunc_f(P_h V_h), heads merged        Beaver per head
  r1  = trunc_f(c Wout) + x
  h2  = LayerNorm(r1)
  u   = trunc_f(h2 W1); g = GeLU(u)           spline gate (CubicPolyTask)
  out = trunc_f(g W2) + r1

Every truncation is a GapARS gate with its own key; every Beaver product has
its own triple (one per head for the attention products; the reference
reuses one triple for all heads and one trunc key per task).  The score
scale inv_sqrt = llround(2^f / sqrt(d_head)) is a public factor folded into
the truncation's open (the reference applies (acc * inv_sqrt) >> f to each
share in the matmul epilogue, cuda_primitives.cu:391-417, which
reconstructs to the same value up to a carry of one unit before the
truncation).  No biases (the reference layer passes none).
"""
import math

import numpy as np
import torch

from . import native, spline, tables
from .layernorm import LayerNormBlock
from .softmax import SoftmaxBlock, causal_offsets
from .tasks import (Dealer, Prepared, Trunc, dev, dev_i32, lin2, lin2_batch, operand, pair, ptr,
                    stream_ptr, term, x_planes)

M64 = (1 << 64) - 1


class PublicMatmulTrunc:
    """Y = trunc_f(X W) for both parties; W public int64 [K x N] (host)."""

    def __init__(self, M, K, N, W, dealer, prg_state, frac_bits=12, device="cuda"):
        lib = native.load()
        self.M, self.K, self.N, self.f = M, K, N, frac_bits
        W = np.ascontiguousarray(W, dtype=np.int64).reshape(K, N)
        self.W = W
        self.digits = lib.sufhip_public_w_digits(W.ctypes.data, W.size)
        pb = lib.sufhip_public_w_planes_bytes(K, N, self.digits)
        if pb == 0:
            raise native.SufHipError("PublicMatmulTrunc: unsupported shape %r" % ((M, K, N),))
        self.planes = torch.empty((pb + 15) // 16 * 2, dtype=torch.int64, device=device)
        dW = dev(W, device)
        native.call("sufhip_public_w_prepare", ptr(dW), K, N, self.digits, ptr(self.planes),
                    stream_ptr())
        torch.cuda.current_stream().synchronize()
        wb = lib.sufhip_matmul_public2_work_bytes(M, K, N)
        self.work = torch.empty((wb + 15) // 16 * 2, dtype=torch.int64, device=device)
        self.work_bytes = self.work.numel() * 8
        self.tr = Trunc(dealer, frac_bits, M * N, prg_state, device=device)
        self.zhat = torch.empty(M * N, dtype=torch.int64, device=device)

    def truncs(self):
        return [self.tr]

    def product2(self, X, out=None, zhat=None, mask=0, trunc=None):
        tail = (ptr(self.planes), self.digits, ptr(out[0]) if out is not None else None,
                ptr(out[1]) if out is not None else None, ptr(zhat), mask & M64,
                native.ctypes.byref(trunc) if trunc is not None else None,
                ptr(self.work), self.work_bytes, stream_ptr())
        if X is None:
            native.call("sufhip_matmul_public2_planes", ptr(self.work), self.M, self.K, self.N,
                        *tail)
        else:
            native.call("sufhip_matmul_public2", ptr(X[0]), ptr(X[1]), self.M, self.K, self.N,
                        *tail)

    def x_planes(self):
        """(buffer, cols) into which a producer writes X's digit planes for
        eval2(None, ...): the first region of the workspace."""
        return (self.work, self.K)

    def eval2_qkv(self, opens):
        """The product of the producer-written X planes with its truncation,
        written as the attention's opens (AttentionCore.qkv_opens: the
        planes of Q_h - A, K_h^T - B and V_h - B2) instead of as Y
        (sufhip_matmul_public2_planes_qkv)."""
        epi = self.tr.epilogue((self.zhat, self.zhat))  # y is not written
        native.call("sufhip_matmul_public2_planes_qkv", ptr(self.work), self.M, self.K, self.N,
                    ptr(self.planes), self.digits, self.tr.mask & M64, native.ctypes.byref(epi),
                    native.ctypes.byref(opens), ptr(self.work), self.work_bytes, stream_ptr())

    def slices(self):
        """The product's k-slice count (above 1, eval2_slices can leave the
        reduction and the truncation to the consumer's launch)."""
        return native.load().sufhip_matmul_public2_slices(self.M, self.K, self.N)

    def eval2_slices(self, out, add=None):
        """The product of the producer-written X planes with its k-slices
        left unreduced (sufhip_matmul_public2_planes_partial): returns
        LayerNormBlock's `pre` for a block that reduces them, applies this
        product's truncation (prepared) and writes out = trunc_f(X W) (+ add)
        in its own launch."""
        sl = native.ctypes.c_void_p()
        native.call("sufhip_matmul_public2_planes_partial", ptr(self.work), self.M, self.K, self.N,
                    ptr(self.planes), self.digits, ptr(self.work), self.work_bytes,
                    native.ctypes.byref(sl), stream_ptr())
        return (sl.value, self.slices(), self.tr.epilogue(out, add), self.tr.mask)

    def eval2(self, X, out, add=None):
        """out = trunc_f(X W) (+ the pair `add`: a residual).  X = None: X's
        digit planes were written to x_planes() by its producer.  The
        truncation must have been prepared."""
        if self.tr.has_table():
            self.product2(X, mask=self.tr.mask, trunc=self.tr.epilogue(out, add))
        else:
            self.product2(X, zhat=self.zhat, mask=self.tr.mask)
            self.tr.finish(self.zhat, out)
            if add is not None:
                lin2(operand(term(out), term(add)), self.M * self.N, out=out)
        return out


def kb_planes(batches, rows, cols, device="cuda"):
    """A buffer for one operand's digit planes (sufhip_kb_split_batch)."""
    nb = native.load().sufhip_kb_planes_bytes(batches, rows, cols)
    return torch.empty(max(2, (nb + 15) // 8), dtype=torch.int64, device=device)


def kb_split(jobs):
    """Digit planes of up to 8 operands in one launch: jobs of (src, planes,
    batches, rows, cols, k_is_col[, planes_a0, a0]); with the last two also
    the planes of src + a0."""
    arr = (native.KbSplitJob * len(jobs))()
    for i, jb in enumerate(jobs):
        src, planes, b, r, c, kc = jb[:6]
        arr[i].src, arr[i].planes = ptr(src), ptr(planes)
        arr[i].batches, arr[i].rows, arr[i].cols, arr[i].k_is_col = b, r, c, int(kc)
        if len(jb) > 6:
            arr[i].planes_a0, arr[i].a0 = ptr(jb[6]), ptr(jb[7])
    native.call("sufhip_kb_split_batch", arr, len(jobs), stream_ptr())


def kb_open_split(jobs, prepare=None):
    """Masked opens written straight as digit planes, up to 8 in one launch:
    jobs of (a, b, planes, batches, rows, cols, k_is_col[, planes_a0, a0[,
    view]]) with a and b pairs of share arrays (b may be None); element i is
    a0 + a1 - b0 - b1, and with planes_a0 and a0 (either may be None) also
    its + a0[i] planes.  view = (offset, batch, row, col strides) in words:
    element (batch, row, col) of a[p] is a[p][offset + strides . index].
    prepare: optional truncation gates (tasks.Trunc, one PRG state) whose
    key-only halves run in the same launch when they fit beside the split
    (sufhip_kb_open_split_prepare), else in their own launches first."""
    arr = (native.KbOpenJob * len(jobs))()
    for i, jb in enumerate(jobs):
        a, b, planes, nb, r, c, kc = jb[:7]
        view = jb[9] if len(jb) > 9 else None
        off = 0
        if view is not None:
            off, sb, sr, sc = view
            last = off + (nb - 1) * sb + (r - 1) * sr + (c - 1) * sc  # the view's last element
            if min(sb, sr, sc, off) < 0 or min(a[0].numel(), a[1].numel()) <= last:
                raise ValueError("kb_open_split: the view runs outside a[p]")
        arr[i].a[0], arr[i].a[1] = ptr(a[0]) + 8 * off, ptr(a[1]) + 8 * off
        if b is not None:
            arr[i].b[0], arr[i].b[1] = ptr(b[0]), ptr(b[1])
        arr[i].planes = ptr(planes)
        arr[i].batches, arr[i].rows, arr[i].cols, arr[i].k_is_col = nb, r, c, int(kc)
        if len(jb) > 7 and jb[7] is not None:
            arr[i].planes_a0, arr[i].a0 = ptr(jb[7]), ptr(jb[8])
        if len(jb) > 9 and jb[9] is not None:
            arr[i].a_stride[0], arr[i].a_stride[1], arr[i].a_stride[2] = jb[9][1:4]
    if not prepare:
        native.call("sufhip_kb_open_split_batch", arr, len(jobs), stream_ptr())
        return
    state = prepare[0].prg_state
    if any(t.prg_state != state for t in prepare):
        raise ValueError("kb_open_split: gates with different PRG states")
    tj = [j for t in prepare for j in t.jobs()]
    tarr = (native.TruncJob * len(tj))(*tj)
    native.call("sufhip_kb_open_split_prepare", arr, len(jobs), prepare[0]._state, tarr, len(tj),
                stream_ptr())


class BatchedTriples:
    """Beaver matrix triples per batch: A [b][M x K], B [b][K x N] uniform,
    C = A B mod 2^64; party 0 holds the drawn shares.  When M, K, N are
    multiples of 32 the product runs on the matrix cores and the shares of A
    and B are also kept as digit planes (made here, with the triples);
    otherwise the VALU product's k-split workspace is kept."""

    def __init__(self, dealer, batches, M, K, N, device="cuda"):
        self.shape = (batches, M, K, N)
        self.mfma = M % 32 == 0 and K % 32 == 0 and N % 32 == 0 and K <= 4096
        wb = 0 if self.mfma else \
            native.load().sufhip_beaver_matmul2_batched_work_bytes(batches, M, K, N)
        self.work = torch.empty(max(2, (wb + 15) // 8), dtype=torch.int64, device=device)
        self.work_bytes = self.work.numel() * 8
        A = dealer.words(batches * M * K).reshape(batches, M, K)
        B = dealer.words(batches * K * N).reshape(batches, K, N)
        C = np.matmul(A, B)  # uint64: exact mod 2^64
        A0 = dealer.words(A.size).reshape(A.shape)
        B0 = dealer.words(B.size).reshape(B.shape)
        C0 = dealer.words(C.size).reshape(C.shape)
        self.A = (dev(A0, device), dev(A - A0, device))
        self.B = (dev(B0, device), dev(B - B0, device))
        self.C = (dev(C0, device), dev(C - C0, device))
        self.host = (A, B, C, A0, B0, C0)
        if self.mfma:
            self.Ap = tuple(kb_planes(batches, M, K, device) for _ in range(2))
            self.Bp = tuple(kb_planes(batches, K, N, device) for _ in range(2))
            self.Dp = kb_planes(batches, M, K, device)  # the opens' planes, per call
            self.Xp = kb_planes(batches, M, K, device)  # D + A_0: party 0's left operand with E
            self.Ep = kb_planes(batches, K, N, device)
            kb_split([(self.A[p], self.Ap[p], batches, M, K, 1) for p in (0, 1)] +
                     [(self.B[p], self.Bp[p], batches, K, N, 0) for p in (0, 1)])

    def split_jobs(self, D=None, E=None):
        """kb_split jobs of the opens D [b][M x K] (with the planes of
        D + A_0) and / or E [b][K x N]."""
        b, M, K, N = self.shape
        return ([(D, self.Dp, b, M, K, 1, self.Xp, self.A[0])] if D is not None else []) + \
            ([(E, self.Ep, b, K, N, 0)] if E is not None else [])

    def d_planes(self):
        """A producer's plane spec for the open D: its planes and those of D + A_0."""
        b, M, K, _ = self.shape
        return (self.Dp, b, M, K, 1, self.Xp, self.A[0])

    def mfma_args(self):
        """BeaverMfma2Args with this triple's planes and shape (balanced form)."""
        b, M, K, N = self.shape
        a = native.BeaverMfma2Args()
        a.Dp, a.Ep, a.Xp = ptr(self.Dp), ptr(self.Ep), ptr(self.Xp)
        for p in (0, 1):
            a.Ap[p], a.Bp[p], a.C[p] = ptr(self.Ap[p]), ptr(self.Bp[p]), ptr(self.C[p])
        a.batches, a.M, a.K, a.N = b, M, K, N
        return a


def _beaver_trunc_merged(tri, tr, out, planes=None):
    """out = tr(the product of tri's opens' planes), heads merged side by side
    ([m][b N + n]), in the product's launch; planes = (buffer, cols): also as
    a following public-weight product's digit planes."""
    a = tri.mfma_args()
    a.merge_heads = 1
    epi = tr.epilogue(out)
    a.trunc = native.ctypes.pointer(epi)
    a.mask = tr.mask & M64
    a.out_planes = x_planes(planes)
    native.call("sufhip_beaver_matmul2_mfma_ex", native.ctypes.byref(a), stream_ptr())


def _beaver_batched(D, E, tri, batches, M, K, N, out, split=True):
    """out = the two-party batched Beaver product of the opens D, E with the
    triples `tri`.  On the matrix cores the opens' planes are made here unless
    split is False (the caller made them, batched with other opens)."""
    if tri.mfma:
        if split:
            kb_split(tri.split_jobs(D, E))
        a = tri.mfma_args()
        a.out[0], a.out[1] = ptr(out[0]), ptr(out[1])
        native.call("sufhip_beaver_matmul2_mfma_ex", native.ctypes.byref(a), stream_ptr())
        return
    native.call("sufhip_beaver_matmul2_batched", ptr(D), ptr(E), ptr(tri.A[0]), ptr(tri.A[1]),
                ptr(tri.B[0]), ptr(tri.B[1]), ptr(tri.C[0]), ptr(tri.C[1]), batches, M, K, N,
                ptr(out[0]), ptr(out[1]), ptr(tri.work), tri.work_bytes, stream_ptr())


def attention_maps(seq, d, heads):
    """Index maps (int32) between the layouts of the attention core:
    gq/gk/gv gather Q_h [seq x dh], K_h^T [dh x seq], V_h [seq x dh] from the
    [seq x 3d] QKV rows; gs gathers the packed causal scores from the dense
    [heads][seq][seq] products; gp gathers dense P_h from the packed
    probabilities (masked entries read the zero slot n_packed); gc merges the
    heads' [heads][seq][dh] context into [seq x d]."""
    dh = d // heads
    h = np.arange(heads)[:, None, None]
    m = np.arange(seq)[None, :, None]
    k = np.arange(dh)[None, None, :]
    gq = m * 3 * d + h * dh + k                                   # [h][m][k]
    kk = np.arange(dh)[None, :, None]
    nn_ = np.arange(seq)[None, None, :]
    gk = nn_ * 3 * d + d + h * dh + kk                            # [h][k][n]
    ks = np.arange(seq)[None, :, None]
    nd = np.arange(dh)[None, None, :]
    gv = ks * 3 * d + 2 * d + h * dh + nd                         # [h][k][n]
    offs = causal_offsets(heads, seq)
    n_packed = int(offs[-1])
    rows = np.repeat(np.arange(heads * seq), np.tile(np.arange(1, seq + 1), heads))
    col = np.arange(n_packed) - offs[:-1][rows]
    gs = (rows // seq) * seq * seq + (rows % seq) * seq + col      # packed -> dense index
    r = np.arange(seq)[None, :, None]
    c = np.arange(seq)[None, None, :]
    row_id = h * seq + r
    gp = np.where(c <= r, offs[:-1][row_id] + c, n_packed)       # [h][m][k]
    t = np.arange(seq)[:, None]
    j = np.arange(d)[None, :]
    gc = (j // dh) * seq * dh + t * dh + (j % dh)                 # [t][j]
    return {"gq": gq.ravel(), "gk": gk.ravel(), "gv": gv.ravel(), "gs": gs.ravel(),
            "gp": gp.ravel(), "gc": gc.ravel(), "offsets": offs, "n_packed": n_packed}


class AttentionCore:
    """Causal multi-head attention on opened-nothing QKV shares [seq x 3d]:
    per-head Beaver QK^T, scaled truncation into packed causal rows, the
    softmax block, per-head Beaver PV, truncation into [seq x d]."""

    def __init__(self, seq, d, heads, dealer, prg_state, frac_bits=12, device="cuda"):
        self.seq, self.d, self.heads, self.f = seq, d, heads, frac_bits
        self.dh = dh = d // heads
        inv_sqrt = tables.llround((1.0 / math.sqrt(dh)) * math.ldexp(1.0, frac_bits))
        self.inv_sqrt = max(inv_sqrt, 1)
        mp = attention_maps(seq, d, heads)
        self.offsets, self.n = mp["offsets"], mp["n_packed"]
        self.maps = {k: dev_i32(mp[k], device) for k in ("gq", "gk", "gv", "gs", "gp", "gc")}
        self.tri_qk = BatchedTriples(dealer, heads, seq, dh, seq, device)
        self.tri_pv = BatchedTriples(dealer, heads, seq, seq, dh, device)
        # QK^T's B shares also as [heads][seq][dh] (B transposed per head), for
        # a QKV product that subtracts them in its epilogue (qkv_opens).
        self.qk_bt = tuple(b.reshape(heads, dh, seq).transpose(1, 2).contiguous().reshape(-1)
                           for b in self.tri_qk.B)
        # The scores' truncation by 2f as two f-bit table gates (same floor).
        self.tr_s = [Trunc(dealer, frac_bits, self.n, prg_state, device=device)
                     for _ in range(2)]
        self.tr_c = Trunc(dealer, frac_bits, seq * d, prg_state, device=device)
        self.softmax = SoftmaxBlock(self.offsets, prg_state, frac_bits, seed=dealer.word() >> 1,
                                    device=device)
        hsd = heads * seq * dh
        self.D = torch.empty(hsd, dtype=torch.int64, device=device)
        self.E = torch.empty(hsd, dtype=torch.int64, device=device)
        self.E2 = torch.empty(hsd, dtype=torch.int64, device=device)
        self.D2 = torch.empty(heads * seq * seq, dtype=torch.int64, device=device)
        self.S = pair(heads * seq * seq, device)
        self.Z = pair(hsd, device)
        self.sa = pair(self.n, device)
        self.scores = pair(self.n, device)
        self.prob = pair(self.n + 1, device)  # slot n stays 0: the masked entries of P
        for t in self.prob:
            t[self.n:].zero_()
        self.side = torch.cuda.Stream(device=device)

    def truncs(self):
        return self.tr_s + [self.tr_c] + self.softmax.truncs()

    def qkv_opens(self):
        """sufhip_qkv_opens for a QKV product that writes this core's three
        opens itself (PublicMatmulTrunc.eval2_qkv; matrix-core products):
        the planes of Q_h - A (with + A_0), K_h^T - B and V_h - B2."""
        from .tasks import kb_planes_out
        tq, tp = self.tri_qk, self.tri_pv
        h, seq, dh = self.heads, self.seq, self.dh
        o = native.QkvOpens()
        o.heads, o.seq, o.dh = h, seq, dh
        for j, sub in enumerate((tq.A, self.qk_bt, tp.B)):
            o.sub[j][0], o.sub[j][1] = ptr(sub[0]), ptr(sub[1])
        o.out[0] = kb_planes_out((tq.Dp, h, seq, dh, 1, tq.Xp, tq.A[0]))
        o.out[1] = kb_planes_out((tq.Ep, h, dh, seq, 0))
        o.out[2] = kb_planes_out((tp.Ep, h, seq, dh, 0))
        return o

    def eval2(self, qkv, out, prep=None, fused=True, planes=None, sm_marks=None,
              sm_spin=None):
        """prep: (tasks.Prepared, batch) holding the key-only halves of
        truncs(), or None to issue them here.  fused: scores, softmax and the
        next open in one launch (sufhip_softmax2); else launch by launch.
        planes = (buffer, cols): the context also as the output projection's
        digit planes (matrix-core products only).  sm_marks: optional list
        that receives two timing events around the one-launch softmax block
        (eager profiling); sm_spin: optional callable that queues device work
        before the first of them (a spin that hides the host's staging of the
        launch, so the events bracket the kernel).  qkv = None (matrix-core
        products): the QKV product already wrote the three opens
        (qkv_opens)."""
        seq, d, h, dh, mp = self.seq, self.d, self.heads, self.dh, self.maps
        if prep is None:
            prep = (Prepared(self.side, [self.truncs()]), 0)
        # D = open(Q_h - A), E = open(K_h^T - B), and already the second
        # product's E2 = open(V_h - B2), in one launch; then the per-head products.
        hsd = h * seq * dh
        if qkv is None and not self.mfma():
            raise ValueError("AttentionCore.eval2: qkv = None needs the matrix-core products")
        if self.mfma():
            # The three opens go straight to the products' digit planes, each
            # head's Q, K^T and V read through a strided view of the QKV rows
            # (the index maps gq, gk, gv as strides), whole plane segments
            # per lane.
            tq, tp = self.tri_qk, self.tri_pv
            if qkv is not None:
                kb_open_split([(qkv, tq.A, tq.Dp, h, seq, dh, 1, tq.Xp, tq.A[0],
                                (0, dh, 3 * d, 1)),
                               (qkv, tq.B, tq.Ep, h, dh, seq, 0, None, None, (d, dh, 1, 3 * d)),
                               (qkv, tp.B, tp.Ep, h, seq, dh, 0, None, None,
                                (2 * d, dh, 3 * d, 1))])
            _beaver_batched(self.D, self.E, self.tri_qk, h, seq, dh, seq, self.S, split=False)
        else:
            gq = operand(term(qkv, index=mp["gq"]), term(self.tri_qk.A, neg=True))
            gk = operand(term(qkv, index=mp["gk"]), term(self.tri_qk.B, neg=True))
            gv = operand(term(qkv, index=mp["gv"]), term(self.tri_pv.B, neg=True))
            lin2_batch([(gq, hsd, self.D, 0), (gk, hsd, self.E, 0), (gv, hsd, self.E2, 0)])
            _beaver_batched(self.D, self.E, self.tri_qk, h, seq, dh, seq, self.S)
        prep[0].wait(prep[1])
        scaled = operand(term(self.S, index=mp["gs"], mul=self.inv_sqrt))
        if fused and self.softmax.fusable():
            # One launch: the masked open of inv_sqrt * S at the packed causal
            # positions truncated by 2f, the softmax block, and the open of
            # P - A over the dense [heads][seq][seq] layout (also as PV's
            # digit planes on the matrix cores).
            dp = self.tri_pv.d_planes() if self.mfma() else None
            if sm_marks is not None:
                if sm_spin is not None:
                    sm_spin()
                sm_marks.append(torch.cuda.Event(enable_timing=True))
                sm_marks[-1].record()
            self.softmax.eval_block(scaled, pre=self.tr_s,
                                    dense=(self.D2, self.tri_pv.A, seq, dp))
            if sm_marks is not None:
                sm_marks.append(torch.cuda.Event(enable_timing=True))
                sm_marks[-1].record()
        else:
            lin2(scaled, self.n, into=(self.tr_s[0], self.sa))
            lin2(operand(term(self.sa)), self.n, into=(self.tr_s[1], self.scores))
            self.softmax.eval2(self.scores, self.prob, prep=prep, fused=False)
            lin2(operand(term(self.prob, index=mp["gp"]), term(self.tri_pv.A, neg=True)),
                 h * seq * seq, xhat=self.D2)
        if self.mfma():
            # PV, the context's truncation and the head merge in one launch.
            if not (fused and self.softmax.fusable()):
                kb_split(self.tri_pv.split_jobs(D=self.D2))
            _beaver_trunc_merged(self.tri_pv, self.tr_c, out, planes)
            return out
        if planes is not None:
            raise ValueError("AttentionCore.eval2: planes need the matrix-core products")
        _beaver_batched(self.D2, self.E2, self.tri_pv, h, seq, seq, dh, self.Z)
        lin2(operand(term(self.Z, index=mp["gc"])), seq * d, into=(self.tr_c, out))
        return out

    def mfma(self):
        """The per-head products run on the matrix cores, and the context's
        truncation is a table gate folded into the PV launch."""
        return self.tri_qk.mfma and self.tri_pv.mfma and self.tr_c.has_table()


def synthetic_weights(d=768, ffn=3072, frac_bits=12, seed=13):
    """round(N(0, 0.02) 2^f) weights (Box-Muller on std::mt19937_64): Wqkv
    from mt(seed), Wout mt(100 seed + 1), W1 mt(100 seed + 2), W2 mt(100 seed + 3)."""
    from . import pfss

    def w(s, k, n):
        return pfss.host_normal_fixed(s, 0.02, 0.0, frac_bits, k * n).view(np.int64).reshape(k, n)

    return {"Wqkv": w(seed, d, 3 * d), "Wout": w(100 * seed + 1, d, d),
            "W1": w(100 * seed + 2, d, ffn), "W2": w(100 * seed + 3, ffn, d)}


class TransformerLayer:
    """One GPT-2-shaped layer over x [seq x d] Q(f) shares, both parties."""

    def __init__(self, prg_state, weights, seq=128, d=768, heads=12, ffn=3072, frac_bits=12,
                 seed=13, device="cuda", keep_intermediates=False):
        """keep_intermediates: also write h1, Q K V, h2 and g as int64 shares
        (they otherwise go only to the next product's digit planes, Q K V to
        the attention's opens)."""
        self.seq, self.d, self.heads, self.ffn, self.f = seq, d, heads, ffn, frac_bits
        self.keep = keep_intermediates
        self.prg_state = bytes(prg_state)
        dealer = Dealer(seed)
        sub = lambda: dealer.word() >> 1  # noqa: E731
        self.ln1 = LayerNormBlock(seq, d, self.prg_state, frac_bits, seed=sub(), device=device)
        self.qkv = PublicMatmulTrunc(seq, d, 3 * d, weights["Wqkv"], dealer, self.prg_state,
                                     frac_bits, device)
        self.attn = AttentionCore(seq, d, heads, dealer, self.prg_state, frac_bits, device)
        self.proj = PublicMatmulTrunc(seq, d, d, weights["Wout"], dealer, self.prg_state,
                                      frac_bits, device)
        self.ln2 = LayerNormBlock(seq, d, self.prg_state, frac_bits, seed=sub(), device=device)
        self.w1 = PublicMatmulTrunc(seq, d, ffn, weights["W1"], dealer, self.prg_state,
                                    frac_bits, device)
        self.gelu_table = tables.gelu_table(frac_bits)
        self.gelu = spline.SplineGate(seq * ffn, self.gelu_table[0], self.gelu_table[1],
                                      self.prg_state, frac_bits, seed=sub(), nonce=dealer.word())
        self.w2 = PublicMatmulTrunc(seq, ffn, d, weights["W2"], dealer, self.prg_state,
                                    frac_bits, device)
        self.side = torch.cuda.Stream(device=device)
        self.host_walks = True
        n = seq * d
        self.h1, self.qkvs, self.ctx = pair(n), pair(3 * n), pair(n)
        self.r1, self.h2, self.u, self.g = pair(n), pair(n), pair(seq * ffn), pair(seq * ffn)

    def stage_truncs(self):
        """The layer's truncation gates in three batches, in order of need:
        LN1 and the QKV product; the attention core; the whole second half
        (issued once the QKV product is queued, see eval2)."""
        return [self.ln1.truncs() + self.qkv.truncs(),
                self.attn.truncs(),
                self.proj.truncs() + self.ln2.truncs() + self.w1.truncs() + self.gelu.truncs() +
                self.w2.truncs()]

    def hosted_walks(self):
        """The gates whose key-only halves the two LayerNorm launches prepare
        on the CUs their rows leave free: (in the first, in the second).  A
        LayerNorm holds one 512-lane workgroup per CU, and its walks take
        three local levels (4096 lanes per table, two tables per gate) in one
        pass of seven eighths of the free CUs: at 128 rows on 256 CUs, seven
        gates, about as long as the rows take (measured, one LayerNorm of
        128 x 768 rows, L2-warm: 16.4 us alone, 17.0 / 20.7 / 21.6 / 21.8 /
        31.0 us walking 4 / 5 / 6 / 7 / 8 gates).  The first takes the second
        LayerNorm's gates, the second the MLP's."""
        cus = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
        k = max(cus - self.seq, 0) * 7 * 512 // (8 * 2 * 4096)
        mlp = self.w1.truncs() + self.gelu.truncs() + self.w2.truncs()
        first = (self.ln2.truncs() + mlp)[:k]
        return first, [t for t in mlp if all(t is not u for u in first)][:k]

    def eval2(self, x, out, marks=None, overlap_prepare=False, sm_marks=None, sm_spin=None):
        """x, out: pairs of int64 [seq * d] device tensors.  marks: optional
        list of torch events recorded after each stage (profiling).  The
        key-only halves of the truncation gates run first, in one batched
        walk on the current stream, except those of hosted_walks(), which the
        fused LayerNorm launches walk on their spare CUs (host_walks; always
        before the gates' first use).  With overlap_prepare they all run on a
        side stream instead, in three batches, each ahead of the stage that
        needs it (a fork or join between streams costs about as much as it
        hides).  sm_marks, sm_spin: see AttentionCore.eval2."""
        # LayerNorm and GeLU outputs feed only the next public-weight product:
        # they are written as its digit planes when the block runs fused.
        fused_ln = self.ln1.fusable() and self.ln2.fusable()
        hosted = ([], [])
        if overlap_prepare:
            prep = Prepared(self.side, self.stage_truncs(), upfront=2)
            b = lambda k: k  # noqa: E731
        else:
            if self.host_walks and fused_ln:
                hosted = self.hosted_walks()
            skip = {id(t) for t in hosted[0] + hosted[1]}
            prep = Prepared(None, [[t for t in sum(self.stage_truncs(), []) if id(t) not in skip]])
            b = lambda k: 0  # noqa: E731

        def mark():
            if marks is not None:
                ev = torch.cuda.Event(enable_timing=True)
                ev.record()
                marks.append(ev)

        mark()
        # With the matrix-core attention the QKV product writes the attention's
        # three opens as digit planes instead of Q, K and V (unsliced product,
        # Q, K and V not kept).
        qkv_opens = fused_ln and self.attn.mfma() and not self.keep and \
            self.qkv.slices() == 1 and self.qkv.tr.has_table() and self.attn.dh % 32 == 0 and \
            self.d % 64 == 0
        if fused_ln:
            self.ln1.eval2(x, self.h1, prep=(prep, b(0)), planes=self.qkv.x_planes(),
                           write_out=self.keep, walk=hosted[0])
            mark()
            if qkv_opens:
                self.qkv.eval2_qkv(self.attn.qkv_opens())
            else:
                self.qkv.eval2(None, self.qkvs)
        else:
            self.ln1.eval2(x, self.h1, prep=(prep, b(0)))
            mark()
            self.qkv.eval2(self.h1, self.qkvs)
        prep.release()  # the second half's gates, after the QKV product
        mark()
        pre = None
        if self.attn.mfma():
            self.attn.eval2(None if qkv_opens else self.qkvs, self.ctx, prep=(prep, b(1)),
                            planes=self.proj.x_planes(), sm_marks=sm_marks, sm_spin=sm_spin)
            mark()
            prep.wait(b(2))
            if fused_ln and self.proj.slices() > 1 and self.proj.tr.has_table():
                # r1 = trunc(ctx Wout) + x: the k-slices' reduction and the
                # truncation run in the second LayerNorm's launch.
                pre = self.proj.eval2_slices(self.r1, add=x)
            else:
                self.proj.eval2(None, self.r1, add=x)  # r1 = trunc(ctx Wout) + x
        else:
            self.attn.eval2(self.qkvs, self.ctx, prep=(prep, b(1)), sm_marks=sm_marks,
                            sm_spin=sm_spin)
            mark()
            prep.wait(b(2))
            self.proj.eval2(self.ctx, self.r1, add=x)
        mark()
        if fused_ln:
            self.ln2.eval2(self.r1, self.h2, prep=(prep, b(2)), planes=self.w1.x_planes(),
                           write_out=self.keep, pre=pre, walk=hosted[1])
            mark()
            self.w1.eval2(None, self.u)
        else:
            self.ln2.eval2(self.r1, self.h2, prep=(prep, b(2)))
            mark()
            self.w1.eval2(self.h2, self.u)
        mark()
        self.gelu.eval2(self.u, self.g, prep=(prep, b(2)), planes=self.w2.x_planes(),
                        write_out=self.keep)
        mark()
        self.w2.eval2(None, out, add=self.r1)  # out = trunc(g W2) + r1
        mark()
        return out
