"""SUF's softmax block for two parties on one GPU.

Task chain (SoftmaxBlockTask, include/nn/softmax_block_task.hpp:97-450, fed
by RowMaxDiffTask, include/nn/row_maxdiff_task.hpp:49-165, as
attention_forward runs them, src/nn/attention_block.cpp:1240-1760), over
packed ragged rows (row r holds elements [offsets[r], offsets[r+1])):

  RowMaxDiff   pairwise max tree, max(a, b) = b + ReLU(a - b), one ReLU
               gate per round (interval LUT of ReLU's public-x^
               coefficients), then delta = max(row) - x
  nExp         CubicPolyTask on delta with the exp(-t) spline table
               (suf_amd/spline.SplineGate)
  row sum      s = sum of exp over the row (local), opened with the
               reciprocal's mask
  Recip        RecipTask: affine-init LUT (c0, c1), y = c0 + trunc_f(c1 s),
               NR y <- trunc_f(y (2 - trunc_f(y s)))
  normalise    MulRowBroadcastTask e * inv(row), then trunc_f

Every truncation is a GapARS gate with its own key (the reference shares one
trunc key among a task's truncations; reconstruction is the same exact
shift); those by f are folded into the launch of the product they truncate
(a table read, the key-only half prepared on a side stream beforehand).
Randomness: suf_amd.tasks.Dealer(seed).
"""
import numpy as np
import torch

from . import native, spline, tables
from .tasks import (M64, RELU_ALPHA, chain2, chain2_args, CoeffLut, Dealer, dev_i32, kb_planes_out,
                    lin2, mul2x, operand, pair, Prepared, relu_coeffs_for, row_sum2, stream_ptr,
                    term, triple2, Triples, Trunc)


def causal_offsets(heads, seq):
    """Row offsets of `heads` causal [seq x seq] score blocks, packed: row r
    of each head keeps its first r + 1 columns."""
    lens = np.tile(np.arange(1, seq + 1), heads)
    return np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)


def max_tree_plan(offsets):
    """Rounds of the pairwise max over packed rows (RowMaxDiffTask's
    RoundPrep, row_maxdiff_task.hpp:60-125): per round the source indices of
    each next-level slot (src_b = -1 for a carried odd element), and the
    final position of each row's max."""
    offsets = np.asarray(offsets, dtype=np.int64)
    lens = np.diff(offsets)
    cur_off = offsets.copy()
    cur_len = lens.copy()
    rounds = []
    round_off = []
    while np.any(cur_len > 1):
        nxt_len = (cur_len + 1) // 2
        nxt_off = np.concatenate([[0], np.cumsum(nxt_len)])
        src_a = np.empty(int(nxt_off[-1]), dtype=np.int32)
        src_b = np.empty(int(nxt_off[-1]), dtype=np.int32)
        for r in range(len(cur_len)):
            L, b, o = int(cur_len[r]), int(cur_off[r]), int(nxt_off[r])
            pairs = L // 2
            src_a[o:o + pairs] = b + 2 * np.arange(pairs)
            src_b[o:o + pairs] = b + 2 * np.arange(pairs) + 1
            if L & 1:
                src_a[o + pairs] = b + L - 1
                src_b[o + pairs] = -1
        rounds.append((src_a, src_b, int(cur_off[-1])))
        round_off.append(nxt_off[:-1].copy())
        cur_off, cur_len = nxt_off, nxt_len
    # Row r's max sits at cur_off[r] of the last level (rows are non-empty).
    max_tree_plan.round_offsets = round_off
    return rounds, cur_off[:-1].astype(np.int64)


def max_tree_round_offsets(offsets):
    """[rounds][rows] int32: each row's first output slot in each round."""
    max_tree_plan(offsets)
    ro = max_tree_plan.round_offsets
    rows = len(offsets) - 1
    return np.array(ro, dtype=np.int32).reshape(len(ro), rows) if ro else \
        np.zeros((0, rows), dtype=np.int32)


class RowMaxDiff:
    """delta = max(row) - x for packed ragged rows, both parties."""

    def __init__(self, offsets, dealer, device="cuda"):
        self.offsets = np.asarray(offsets, dtype=np.int64)
        if np.any(np.diff(self.offsets) < 1):
            raise ValueError("RowMaxDiff: every row needs at least one element")
        self.n = int(self.offsets[-1])
        self.rows = len(self.offsets) - 1
        rounds, max_pos = max_tree_plan(self.offsets)
        self.rounds = []
        for src_a, src_b, n_in in rounds:
            lut = CoeffLut(dealer, RELU_ALPHA, [[0, 0], [0, 0]], device,
                           coeffs_for_rin=relu_coeffs_for)
            self.rounds.append({"a": dev_i32(src_a, device), "b": dev_i32(src_b, device),
                                "n_in": n_in, "n_out": len(src_a), "lut": lut,
                                "out": pair(len(src_a), device),
                                "src": (src_a, src_b)})
        row = np.repeat(np.arange(self.rows), np.diff(self.offsets))
        self.max_index = dev_i32(max_pos[row], device)
        self.max_len = self.rows
        self.max_row = int(np.diff(self.offsets).max())
        self.offs_dev = dev_i32(self.offsets, device)
        ro = max_tree_round_offsets(self.offsets)
        self.round_off = dev_i32(ro.ravel() if ro.size else np.zeros(1), device)
        self.tree_ok = self.max_row <= 512 and len(self.rounds) <= 16
        self.round_keys = (native.ReluRoundKey * max(1, len(self.rounds)))()
        for k, rd in enumerate(self.rounds):
            lut = rd["lut"]
            rk = self.round_keys[k]
            rk.key[0], rk.key[1] = lut.keys[0].data_ptr(), lut.keys[1].data_ptr()
            rk.key_bytes, rk.intervals, rk.mask = lut.key_bytes, lut.intervals, lut.mask

    def eval2(self, x, delta, fused=True):
        """x, delta: pairs of int64 [n] device tensors.  fused: the whole tree
        in one launch (rows up to 512 elements); else one launch per round."""
        if fused and self.tree_ok:
            native.call("sufhip_relu_max_tree2", x[0].data_ptr(), x[1].data_ptr(), self.rows,
                        self.offs_dev.data_ptr(), self.max_row, len(self.rounds),
                        self.round_off.data_ptr(), self.round_keys, delta[0].data_ptr(),
                        delta[1].data_ptr(), stream_ptr())
            return delta
        cur = x
        for rd in self.rounds:
            lut = rd["lut"]
            native.call("sufhip_relu_max_round2", cur[0].data_ptr(), cur[1].data_ptr(),
                        rd["n_in"], rd["a"].data_ptr(), rd["b"].data_ptr(), rd["n_out"],
                        lut.keys[0].data_ptr(), lut.keys[1].data_ptr(), lut.key_bytes,
                        lut.intervals, lut.mask, rd["out"][0].data_ptr(),
                        rd["out"][1].data_ptr(), stream_ptr())
            cur = rd["out"]
        lin2(operand(term(cur, index=self.max_index, length=cur[0].numel()),
                     term(x, neg=True)), self.n, out=delta)
        return delta


class Recip:
    """RecipTask over n values whose shares x and masked open
    xhat = x + lut.mask the caller provides."""

    def __init__(self, n, dealer, prg_state, frac_bits=12, table=None, iters=1, device="cuda"):
        self.n, self.f, self.iters = n, frac_bits, iters
        alpha, coeffs = table if table is not None else tables.recip_table(frac_bits)
        self.table = (alpha, coeffs)
        self.lut = CoeffLut(dealer, alpha, coeffs, device)
        self.tri = [Triples(dealer, n, device=device) for _ in range(1 + 2 * iters)]
        self.tr = [Trunc(dealer, frac_bits, n, prg_state, device=device)
                   for _ in range(1 + 2 * iters)]
        self.coef = pair(n, device, 2)
        self.zhat = torch.empty(n, dtype=torch.int64, device=device)
        self.t = pair(n, device)
        self.xy = pair(n, device)
        self.y = pair(n, device)

    def truncs(self):
        return self.tr

    def eval2(self, x, xhat=None, out=None, fused=True):
        """x: shares of the values; xhat: their masked open with lut.mask, or
        None to open them inside the LUT launch.  The gate's truncations must
        have been prepared.  fused (one NR step, no xhat): the whole chain in
        one launch."""
        n, f = self.n, self.f
        out = self.y if out is None else out
        xs = operand(term(x))
        if fused and self.iters == 1 and xhat is None:
            chain2(native.CHAIN_RECIP, f, xs, n, self.lut.keys, self.lut.key_bytes,
                   self.lut.intervals, self.lut.mask, self.tri, self.tr, out)
            return out
        self.lut.eval2(xhat, n, self.coef, x=xs if xhat is None else None)
        mul2x(operand(term(self.coef, stride=2, off=1)), xs, self.tri[0], n,
              into=(self.tr[0], self.t))
        y = operand(term(self.t), term(self.coef, stride=2, off=0))
        for it in range(self.iters):
            t1, t2 = self.tr[1 + 2 * it], self.tr[2 + 2 * it]
            mul2x(y, xs, self.tri[1 + 2 * it], n, into=(t1, self.xy))
            two_minus = operand(term(self.xy, neg=True), const=2 << f)
            mul2x(y, two_minus, self.tri[2 + 2 * it], n, into=(t2, out))
            y = operand(term(out))
        if self.iters == 0:
            lin2(y, n, out=out)
        return out


class SoftmaxBlock:
    """Probabilities of packed ragged Q(f) score rows, both parties."""

    def __init__(self, offsets, prg_state, frac_bits=12, seed=11, recip_iters=1, nexp=None,
                 recip=None, device="cuda"):
        self.offsets = np.asarray(offsets, dtype=np.int64)
        self.n = int(self.offsets[-1])
        self.rows = len(self.offsets) - 1
        self.f = frac_bits
        self.prg_state = bytes(prg_state)
        dealer = Dealer(seed)
        self.rowmax = RowMaxDiff(self.offsets, dealer, device)
        self.nexp_table = nexp if nexp is not None else tables.nexp_table(frac_bits)
        self.nexp = spline.SplineGate(self.n, self.nexp_table[0], self.nexp_table[1],
                                      self.prg_state, frac_bits, seed=dealer.word() >> 1,
                                      nonce=dealer.word())
        self.recip = Recip(self.rows, dealer, self.prg_state, frac_bits, recip, recip_iters,
                           device)
        row = np.repeat(np.arange(self.rows), np.diff(self.offsets))
        self.row_index = dev_i32(row, device)
        self.tri = Triples(dealer, self.n, row_of=row, device=device)
        self.tr = Trunc(dealer, frac_bits, self.n, self.prg_state, device=device)
        self.offs_dev = dev_i32(self.offsets, device)
        self.side = torch.cuda.Stream(device=device)
        self.delta = pair(self.n, device)
        self.e = pair(self.n, device)
        self.s = pair(self.rows, device)
        self.shat = torch.empty(self.rows, dtype=torch.int64, device=device)

    def truncs(self):
        return self.nexp.truncs() + self.recip.truncs() + [self.tr]

    def fusable(self):
        rm = self.rowmax
        return (rm.max_row <= 512 and len(rm.rounds) <= 10 and self.recip.iters == 1 and
                all(t.has_table() for t in self.truncs()))

    def block_args(self, x, out=None, pre=(), dense=None):
        """sufhip_softmax2_args of the one-launch block: x an operand over the
        packed scores, pre up to two Trunc gates applied to its open first,
        out a pair for the probabilities and/or dense = (d_open, (a0, a1),
        cols) for the open P - A of the next Beaver product."""
        a = native.Softmax2Args()
        a.x = x
        a.pre_truncs = len(pre)
        for q, t in enumerate(pre):
            a.pre[q] = t.epilogue(self.delta)
            a.pre_mask[q] = t.mask & M64
        rm = self.rowmax
        a.rows, a.d_row_offsets, a.max_row = self.rows, rm.offs_dev.data_ptr(), rm.max_row
        a.rounds, a.d_round_offsets = len(rm.rounds), rm.round_off.data_ptr()
        for k in range(len(rm.rounds)):
            a.keys[k] = rm.round_keys[k]
        g = self.nexp
        a.nexp = chain2_args(native.CHAIN_CUBIC, self.f, None, self.n, g.lut, g.lut_key_bytes,
                             g.intervals, g.rin[0] + g.rin[1], g.tri, g.trunc, self.e)
        rc = self.recip
        a.recip = chain2_args(native.CHAIN_RECIP, self.f, None, self.rows, rc.lut.keys,
                              rc.lut.key_bytes, rc.lut.intervals, rc.lut.mask, rc.tri, rc.tr,
                              rc.y)
        a.norm = triple2(self.tri)
        a.tr_norm = self.tr.epilogue(self.e)
        a.norm_mask = self.tr.mask & M64
        if out is not None:
            a.out[0], a.out[1] = out[0].data_ptr(), out[1].data_ptr()
        if dense is not None:
            a.d_dense = dense[0].data_ptr()
            a.dense_a[0], a.dense_a[1] = dense[1][0].data_ptr(), dense[1][1].data_ptr()
            a.dense_cols = dense[2]
            if len(dense) > 3 and dense[3] is not None:
                a.dense_planes = kb_planes_out(dense[3])
        return a

    def eval_block(self, x, out=None, pre=(), dense=None):
        """The whole block in one launch (sufhip_softmax2); see block_args.
        The gates' key-only halves must have been prepared."""
        a = self.block_args(x, out, pre, dense)
        native.call("sufhip_softmax2", native.ctypes.byref(a), stream_ptr())

    def eval2(self, x, out, prep=None, fused=True):
        """x, out: pairs of int64 [n] device tensors (packed rows).  prep:
        (tasks.Prepared, batch) holding this block's key-only halves, or None
        to issue them here on the block's side stream.  fused: the whole
        block in one launch (sufhip_softmax2); else launch by launch."""
        if prep is None:
            prep = (Prepared(self.side, [self.truncs()]), 0)
        if fused and self.fusable():
            prep[0].wait(prep[1])
            self.eval_block(operand(term(x)), out)
            return out
        self.rowmax.eval2(x, self.delta)
        self.nexp.eval2(self.delta, self.e, prep=prep)
        row_sum2(operand(term(self.e)), self.rows, offsets=self.offs_dev, sums=self.s)
        inv = self.recip.eval2(self.s)
        mul2x(operand(term(self.e)), operand(term(inv, index=self.row_index)), self.tri, self.n,
              into=(self.tr, out))
        return out
