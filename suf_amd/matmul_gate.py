"""Beaver matmul over Z_2^64 followed by a GapARS truncation, for two parties
on one GPU: Y = trunc_f(X * W) with X [M x K] and W [K x N] both additively
shared.

Protocol (the matmul tasks of src/nn/attention_block.cpp:452-900 and the CPU
form src/nn/matmul_beaver.cpp:139-161, then SUF's AutoTrunc lowered to
GapARS):
  D = open(X - A), E = open(W - B)
  Z_p = C_p + D*B_p + A_p*E (+ D*E for party 0)      (launch_beaver_matmul2d;
                                                     int8-limb MFMA form when the
                                                     shape allows)
  Y_p = trunc_f(open(Z + r))                         (truncation gate)
Every step runs in libsuf_hip.so; the dealer's triple product C = A*B is
computed by the same matmul kernel (party 0 form with C = 0, D = A, E = B).
"""
import numpy as np
import torch

from . import native, pfss

M64 = (1 << 64) - 1


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _p(t):
    return t.data_ptr() if t is not None else None


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int64).copy()).cuda()


def _matmul(party, D, E, A, B, C, M, K, N, out, work=None):
    """The int8-limb matrix-core product when the shape allows it and a
    workspace is given, else the VALU kernel (same result bits)."""
    if work is not None:
        native.call("sufhip_beaver_matmul2d_mfma", party, _p(D), _p(E), _p(A), _p(B), _p(C), M, K,
                    N, _p(out), _p(work), work.numel() * 8, _stream())
    else:
        native.call("sufhip_beaver_matmul2d", party, _p(D), _p(E), _p(A), _p(B), _p(C), M, K, N, 0,
                    0, 0, 0, _p(out), _stream())


def mfma_ok(M, K, N):
    return M % 32 == 0 and N % 64 == 0 and K % 32 == 0 and K <= 8191


class BeaverMatmulTrunc:
    """Dealer material (triples, truncation keys) for Y = trunc_f(X W), both
    parties.  Randomness: std::mt19937_64(seed) streams."""

    def __init__(self, M, K, N, prg_state, frac_bits=12, seed=10, use_mfma=True):
        self.M, self.K, self.N, self.f = M, K, N, frac_bits
        self.prg_state = bytes(prg_state)
        lib = native.load()
        w = pfss.host_mt19937_64(seed, 2 * M * K + 2 * K * N + M * N)
        o = 0
        A = w[o:o + M * K]; o += M * K
        A0 = w[o:o + M * K]; o += M * K
        B = w[o:o + K * N]; o += K * N
        B0 = w[o:o + K * N]; o += K * N
        C0 = w[o:o + M * N]
        dA, dB = _dev(A), _dev(B)
        zero_mk = torch.zeros(M * K, dtype=torch.int64, device="cuda")
        zero_kn = torch.zeros(K * N, dtype=torch.int64, device="cuda")
        zero_mn = torch.zeros(M * N, dtype=torch.int64, device="cuda")
        Cfull = torch.empty(M * N, dtype=torch.int64, device="cuda")
        _matmul(0, dA, dB, zero_mk, zero_kn, zero_mn, M, K, N, Cfull)  # C = A * B
        self.A = (_dev(A0), dA - _dev(A0))
        self.B = (_dev(B0), dB - _dev(B0))
        dC0 = _dev(C0)
        self.C = (dC0, Cfull - dC0)
        rnd = pfss.host_mt19937_64(seed + 1, native.TRUNC_RAND_WORDS)
        r = int(rnd[0])
        self.rin = (int(rnd[1]), (r - int(rnd[1])) & M64)
        self.keys = pfss.trunc_gen(native.TRUNC_GAPARS, frac_bits, self.prg_state, rnd)
        # Two-party matrix-core form: both parties' products in one launch with
        # the truncation folded in, the triple shares' digit planes made here.
        # The launch-per-step form's buffers (u64 opens, products, masked open,
        # truncation workspaces) exist only when it is the form in use.
        self.fused = (use_mfma and M % 32 == 0 and K % 32 == 0 and N % 32 == 0 and K <= 4096 and
                      frac_bits <= 13)
        self.mm_work = None
        if not self.fused:
            self.work_bytes = lib.sufhip_trunc_work_bytes(frac_bits, M * N)
            self.work = [torch.empty(max(2, (self.work_bytes + 15) // 8), dtype=torch.int64,
                                     device="cuda") for _ in range(2)]
            self.side = torch.cuda.Stream()
            self.D = torch.empty(M * K, dtype=torch.int64, device="cuda")
            self.E = torch.empty(K * N, dtype=torch.int64, device="cuda")
            self.Z = [torch.empty(M * N, dtype=torch.int64, device="cuda") for _ in range(2)]
            self.zhat = torch.empty(M * N, dtype=torch.int64, device="cuda")
            if use_mfma and mfma_ok(M, K, N):
                wb = lib.sufhip_beaver_matmul2d_mfma_work_bytes(M, K, N)
                self.mm_work = torch.empty((wb + 7) // 8, dtype=torch.int64, device="cuda")
        else:
            from . import layer, tasks
            self.tr = tasks.Trunc(None, frac_bits, M * N, self.prg_state, rnd=rnd)
            self.Ap = tuple(layer.kb_planes(1, M, K) for _ in range(2))
            self.Bp = tuple(layer.kb_planes(1, K, N) for _ in range(2))
            self.Dp, self.Ep = layer.kb_planes(1, M, K), layer.kb_planes(1, K, N)
            self.Xp = layer.kb_planes(1, M, K)  # D + A_0, party 0's left operand with E
            layer.kb_split([(self.A[p], self.Ap[p], 1, M, K, 1) for p in (0, 1)] +
                           [(self.B[p], self.Bp[p], 1, K, N, 0) for p in (0, 1)])

    def eval2(self, X, W, out, events=None):
        """X, W, out: pairs of device int64 tensors (party shares).  events:
        optional list of 2 torch events recorded around the matmul, or of 3
        in the fused form: before the opens, between the opens and the
        product, after the product."""
        M, K, N, s = self.M, self.K, self.N, _stream()
        if self.fused:
            return self._eval2_fused(X, W, out, events)
        # Key-only half of the truncation (both parties) on a side stream,
        # overlapped with the opens and the matmuls.
        start = torch.cuda.Event()
        start.record()
        self.side.wait_event(start)
        for p in (0, 1):
            native.call("sufhip_trunc_prepare", native.TRUNC_GAPARS, self.f,
                        pfss._state_buf(self.prg_state), _p(self.keys[p]), self.keys[p].numel(),
                        M * N, _p(self.work[p]), self.work_bytes, self.side.cuda_stream)
        prepared = torch.cuda.Event()
        prepared.record(self.side)
        native.call("sufhip_open2_diff", _p(X[0]), _p(X[1]), _p(self.A[0]), _p(self.A[1]), M * K,
                    _p(self.D), s)
        native.call("sufhip_open2_diff", _p(W[0]), _p(W[1]), _p(self.B[0]), _p(self.B[1]), K * N,
                    _p(self.E), s)
        if events:
            events[0].record()
        for p in (0, 1):
            _matmul(p, self.D, self.E, self.A[p], self.B[p], self.C[p], M, K, N, self.Z[p],
                    self.mm_work)
        if events:
            events[1].record()
        native.call("sufhip_open2_masked", _p(self.Z[0]), _p(self.Z[1]), self.rin[0], self.rin[1],
                    M * N, _p(self.zhat), s)
        torch.cuda.current_stream().wait_event(prepared)
        for p in (0, 1):
            native.call("sufhip_trunc_finish", native.TRUNC_GAPARS, self.f,
                        pfss._state_buf(self.prg_state), _p(self.keys[p]), self.keys[p].numel(),
                        _p(self.zhat), M * N, _p(out[p]), _p(self.work[p]), self.work_bytes, s)
        return out

    def _eval2_fused(self, X, W, out, events=None):
        """The truncation's key-only half with the opens D = X - A and E = W - B
        written straight as their digit planes (one launch), then both
        parties' products with the truncation of their masked open in one
        launch; all on the current stream."""
        from . import layer
        M, K, N = self.M, self.K, self.N
        # The product's arguments are staged first, so that its launch
        # follows the opens' with no host work in between.
        a = native.BeaverMfma2Args()
        a.Dp, a.Ep, a.Xp = _p(self.Dp), _p(self.Ep), _p(self.Xp)
        for p in (0, 1):
            a.Ap[p], a.Bp[p], a.C[p] = _p(self.Ap[p]), _p(self.Bp[p]), _p(self.C[p])
        a.batches, a.M, a.K, a.N = 1, M, K, N
        epi = self.tr.epilogue(out)
        a.trunc = native.ctypes.pointer(epi)
        a.mask = self.tr.mask & M64
        if events:
            events[0].record()
        # The truncation's key-only walks run in the opens' launch.
        layer.kb_open_split([(X, self.A, self.Dp, 1, M, K, 1, self.Xp, self.A[0]),
                             (W, self.B, self.Ep, 1, K, N, 0)], prepare=[self.tr])
        if events and len(events) > 2:
            events[1].record()
        native.call("sufhip_beaver_matmul2_mfma_ex", native.ctypes.byref(a), _stream())
        if events:
            events[-1].record()
        return out
