"""Piecewise-cubic spline gate (SiLU / GeLU shape) for two parties on one GPU.

Protocol, as SUF runs it for SiLU/GeLU-style gates:
  * coefficients: an interval LUT over the public x^ = x + r_in returns
    additive shares of the piece's (c0, c1, c2, c3)
    (composite_eval_batch_backend fast path, include/gates/composite_fss.hpp:
    1248-1330; intervals rotated by r_in and split at the wrap,
    src/compiler/suf_to_pfss.cpp:506-523);
  * Horner with two truncations (CubicPolyTask, include/runtime/
    phase_tasks.hpp:2962-3061):
        m1 = c3 * x; u = m1 + c2 << f; p = u * x; p2 = trunc_f(p);
        q = p2 + c1 << f; r = q * x; y = trunc_2f(r) + c0
    with three Beaver products and GapARS truncation gates.  trunc_2f(r) + c0
    is evaluated as trunc_f(trunc_f(r) + c0 << f): floor(floor(r / 2^f) /
    2^f) = floor(r / 2^2f) and adding a multiple of 2^f commutes with the
    shift, so the reconstruction is the same while every gate is an f-bit
    table gate (one round more, no 2f-bit DCF walk per element).
The output mask r_out of spline gates is 0 (include/gates/silu_composite.hpp:
92), so the LUT's coefficient shares are used directly.

Every step runs in libsuf_hip.so: by default the whole chain in one launch
(sufhip_gate_chain2: LUT, products and table truncations per element, both
parties); round by round, interval_lut_eval2 (the open of x in the same
launch), mul2x and lin2, each truncation folded into the launch producing its
masked open.  The truncations' key-only precomputation runs on a side
stream, overlapped with the first rounds.  The
dealer builds keys with the library's key builders and host std::mt19937_64
streams.
"""
import numpy as np
import torch

from . import native, pfss
from .tasks import (AosTriples, Prepared, Trunc, chain2, lin2, mul2x, operand, rotated_lut,
                    term)

M64 = (1 << 64) - 1
LUT_TWEAK = 7  # seed_from_id tweak of interval LUT keys (cuda/pfss_backend_gpu.cu:508-515)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _p(t):
    return t.data_ptr() if t is not None else None


def spline_spec(frac_bits=12, seed=6, coeff_bits=15):
    """18 pieces over the ring in unsigned order: [k, k+1) for k = 0..7, the
    positive tail [8, 2^63), the negative tail [-2^63, -8), and [-k, -k+1) for
    k = 8..1 (units of 2^frac_bits).  Coefficients c0..c3 are signed Q(frac)
    words drawn from std::mt19937_64(seed): (w mod 2^coeff_bits) - 2^(coeff_bits-1).
    Returns (alpha [18] u64 ascending, coeffs int64 [18, 4])."""
    one = 1 << frac_bits
    alpha = [k * one for k in range(9)] + [1 << 63] + [(1 << 64) - k * one for k in range(8, 0, -1)]
    w = pfss.host_mt19937_64(seed, 4 * len(alpha))
    half = 1 << (coeff_bits - 1)
    c = (w % np.uint64(1 << coeff_bits)).astype(np.int64) - half
    return np.array(alpha, dtype=np.uint64), c.reshape(len(alpha), 4)


def _split(v, s):
    return s & M64, (v - s) & M64


class SplineGate:
    """Dealer material for one spline gate instance over n elements, both
    parties, resident on the GPU.  Randomness: std::mt19937_64(seed) words
    for r_in, the Beaver triples and the truncation keys."""

    def __init__(self, n, alpha, coeffs, prg_state, frac_bits=12, seed=7, nonce=1,
                 device="cuda"):
        self.n = n
        self.f = frac_bits
        self.prg_state = bytes(prg_state)
        lib = native.load()
        head = pfss.host_mt19937_64(seed, 2 + 2 * native.TRUNC_RAND_WORDS)
        r_in = int(head[0])
        self.rin = _split(r_in, int(head[1]))
        cuts, payload, k = rotated_lut(alpha, coeffs, r_in)
        self.intervals = k
        kb = lib.sufhip_interval_lut_key_bytes(k, 4)
        seed16 = native.ctypes.create_string_buffer(16)
        lib.sufhip_seed_from_id(nonce, LUT_TWEAK, seed16)
        self.lut_key_bytes = kb
        self.lut = []
        for party in (0, 1):
            blob = np.zeros(kb, dtype=np.uint8)
            native.call("sufhip_interval_lut_build_key", party, nonce, 64, 4, cuts.ctypes.data, k,
                        payload.ctypes.data, seed16, blob.ctypes.data)
            self.lut.append(torch.from_numpy(blob.view(np.int64).copy()).to(device).view(torch.uint8))
        # Beaver triples: a, b uniform, c = a*b; party 0 holds the drawn share.
        w = pfss.host_mt19937_64(seed + 1000, 3 * 5 * n).reshape(3, 5, n)
        self.triples = []
        for j in range(3):
            a, b, a0, b0, c0 = w[j]
            c = a * b
            t0 = np.stack([a0, b0, c0], axis=1)
            t1 = np.stack([a - a0, b - b0, c - c0], axis=1)
            self.triples.append(tuple(torch.from_numpy(t.view(np.int64).copy()).to(device)
                                      for t in (t0, t1)))
        # Truncation gates, all GapARS by f: after the 2nd product, and twice
        # after the 3rd (the 2f truncation as two f truncations).
        self.trunc = []
        w3 = pfss.host_mt19937_64(seed + 2000, native.TRUNC_RAND_WORDS)
        for j in range(3):
            rnd = head[2 + j * native.TRUNC_RAND_WORDS: 2 + (j + 1) * native.TRUNC_RAND_WORDS] \
                if j < 2 else w3
            self.trunc.append(Trunc(None, frac_bits, n, self.prg_state, rnd=rnd, device=device))
        self.side = torch.cuda.Stream(device=device)
        # Scratch for the online phase.
        self.xhat = torch.empty(n, dtype=torch.int64, device=device)
        self.coef = [torch.empty((n, 4), dtype=torch.int64, device=device) for _ in range(2)]
        self.u = [torch.empty(n, dtype=torch.int64, device=device) for _ in range(2)]
        self.y = [torch.empty(n, dtype=torch.int64, device=device) for _ in range(2)]
        self.y2 = [torch.empty(n, dtype=torch.int64, device=device) for _ in range(2)]
        self.tri = [AosTriples(t) for t in self.triples]

    def truncs(self):
        return list(self.trunc)

    def eval2(self, x, out, prep=None, fused=True, planes=None, write_out=True):
        """x, out: pairs of int64[n] device tensors (party 0, party 1 shares).
        prep: (tasks.Prepared, batch) holding this gate's key-only halves, or
        None to issue them here on the gate's side stream.  fused: the whole
        chain in one launch (sufhip_gate_chain2); else round by round.
        planes = (buffer, cols), fused only: the output also as a public-weight
        product's digit planes (write_out False: only those)."""
        n, f, s = self.n, self.f, torch.cuda.current_stream().cuda_stream
        if prep is None:
            prep = (Prepared(self.side, [self.truncs()]), 0)
        if fused:
            prep[0].wait(prep[1])
            chain2(native.CHAIN_CUBIC, f, operand(term(x)), n, self.lut, self.lut_key_bytes,
                   self.intervals, self.rin[0] + self.rin[1], self.tri, self.trunc, out,
                   planes=planes, write_out=write_out)
            return out
        if planes is not None:
            raise ValueError("SplineGate.eval2: planes need the fused chain")
        xs = operand(term(x))
        # Both parties' coefficient rows at x^ = x + r_in, opened in the launch.
        native.call("sufhip_interval_lut_eval2", _p(self.lut[0]), _p(self.lut[1]),
                    self.lut_key_bytes, self.intervals, 4, native.ctypes.byref(xs), None,
                    (self.rin[0] + self.rin[1]) & M64, n, _p(self.coef[0]), _p(self.coef[1]), s)
        # u = c3 * x + c2 << f
        mul2x(operand(term(self.coef, stride=4, off=3)), xs, self.tri[0], n, z=self.u,
              z_add=operand(term(self.coef, stride=4, off=2, shift=f)))
        prep[0].wait(prep[1])
        t1, t2, t3 = self.trunc
        # y = trunc_f(u * x)
        mul2x(operand(term(self.u)), xs, self.tri[1], n, into=(t1, self.y))
        # y2 = trunc_f((y + c1 << f) * x); out = trunc_f(y2 + c0 << f)
        mul2x(operand(term(self.y), term(self.coef, stride=4, off=1, shift=f)), xs, self.tri[2],
              n, into=(t2, self.y2))
        lin2(operand(term(self.y2), term(self.coef, stride=4, off=0, shift=f)), n,
             into=(t3, out))
        return out
