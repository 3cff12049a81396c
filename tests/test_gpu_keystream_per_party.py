"""The per-party keystream policy (sufhip_set_keystream_per_party): every
two-party LUT launch computes each party's keystream and interval search
from its own blob, as two parties in separate processes do.  The shares must
be those of the oracle's per-party evaluation (and so those of the shared
policy) for the gate chain, the max tree, the softmax and LayerNorm blocks
and the whole layer, eager and as a HIP graph captured under the policy and
replayed after it is switched back."""
import numpy as np
import pytest
import torch

import fixed_point as fp
import oracle_lib as ol
import twoparty_oracle as tp
from gpu_util import dev, say, u64
from suf_amd import layer, layernorm, native, pfss, softmax, spline, tables, tasks

pytestmark = pytest.mark.gpu

STATE = ol.mt64_bytes(3, ol.PRG_STATE_BYTES).tobytes()
F = 12


@pytest.fixture(scope="module", autouse=True)
def _init():
    native.call("sufhip_init", 0)
    assert native.load().sufhip_keystream_per_party() == 0


def _share(x, seed):
    x = np.asarray(x).astype(np.uint64)
    x0 = pfss.host_mt19937_64(seed, x.size)
    return x0, (x - x0).astype(np.uint64)


def _pair(n):
    return tuple(torch.empty(n, dtype=torch.int64, device="cuda") for _ in range(2))


def _h(t):
    return [u64(t[0]), u64(t[1])]


def _same(a, b):
    return np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_policy_switch_round_trips():
    with pfss.keystream_per_party():
        assert native.load().sufhip_keystream_per_party() == 1
        with pfss.keystream_per_party(False):
            assert native.load().sufhip_keystream_per_party() == 0
        assert native.load().sufhip_keystream_per_party() == 1
    assert native.load().sufhip_keystream_per_party() == 0


@pytest.mark.parametrize("fused", [True, False])
def test_spline_gate_per_party(fused):
    n = 3000
    alpha, coeffs = spline.spline_spec(F, seed=6)
    x = pfss.host_normal_fixed(15, 3.0, 8.0, F, n)
    x0, x1 = _share(x, 48)
    say("spline gate per-party keystreams n=%d fused=%s" % (n, fused))
    gate = spline.SplineGate(n, alpha, coeffs, STATE, F, seed=8)
    xd = [dev(x0), dev(x1)]
    out = _pair(n)
    with pfss.keystream_per_party():
        gate.eval2(xd, out, fused=fused)
    got = _h(out)
    gate.eval2(xd, out, fused=fused)
    assert _same(got, _h(out))
    assert _same(got, tp.spline2(ol.Prg(STATE), gate, [x0, x1]))
    assert np.array_equal((got[0] + got[1]).astype(np.uint64),
                          fp.spline_closed_form(alpha, coeffs, x, F))


@pytest.mark.parametrize("fused", [True, False])
def test_row_max_diff_per_party(fused):
    offsets = np.cumsum([0, 1, 2, 3, 300, 5, 64, 7, 128, 17]).astype(np.int64)
    x = pfss.host_normal_fixed(25, 2.0, 0.0, F, int(offsets[-1]))
    x0, x1 = _share(x, 26)
    say("row max diff per-party keystreams n=%d fused=%s" % (offsets[-1], fused))
    rm = softmax.RowMaxDiff(offsets, softmax.Dealer(7))
    delta = _pair(int(offsets[-1]))
    with pfss.keystream_per_party():
        rm.eval2((dev(x0), dev(x1)), delta, fused=fused)
    got = _h(delta)
    assert _same(got, tp.relu_rounds2(rm, [x0, x1]))
    assert np.array_equal((got[0] + got[1]).astype(np.uint64),
                          fp.row_max_diff(x, offsets).view(np.uint64))


@pytest.mark.parametrize("heads,seq", [(1, 8), (2, 33), (12, 128)])
def test_softmax_block_per_party(heads, seq):
    offs = softmax.causal_offsets(heads, seq)
    n = int(offs[-1])
    x = pfss.host_normal_fixed(80 + seq, 2.0, 0.0, F, n)
    x0, x1 = _share(x, 81)
    say("softmax block per-party keystreams heads=%d seq=%d" % (heads, seq))
    sm = softmax.SoftmaxBlock(offs, STATE, F, seed=19)
    xin = (dev(x0), dev(x1))
    out = _pair(n)
    with pfss.keystream_per_party():
        sm.eval2(xin, out)
    got = _h(out)
    sm.eval2(xin, out)
    assert _same(got, _h(out))
    prob, _ = fp.softmax_block(x, offs, sm.nexp_table, sm.recip.table, F)
    assert np.array_equal((got[0] + got[1]).astype(np.uint64), prob.view(np.uint64))
    if n <= 4096:
        o, _ = tp.softmax2(ol.Prg(STATE), sm, [x0, x1])
        assert _same(got, o)


@pytest.mark.parametrize("rows,cols", [(3, 1100), (128, 768)])
def test_layernorm_block_per_party(rows, cols):
    x = pfss.host_normal_fixed(62, 1.0, 0.0, F, rows * cols)
    x0, x1 = _share(x, 63)
    say("layernorm per-party keystreams %dx%d" % (rows, cols))
    ln = layernorm.LayerNormBlock(rows, cols, STATE, F, seed=15)
    xin = (dev(x0), dev(x1))
    out = _pair(rows * cols)
    with pfss.keystream_per_party():
        ln.eval2(xin, out)
    got = _h(out)
    ln.eval2(xin, out)
    assert _same(got, _h(out))
    y, _ = fp.layernorm(x, rows, cols, F, ln.inv_len, ln.eps_q, ln.rsqrt.table)
    assert np.array_equal((got[0] + got[1]).astype(np.uint64), y.view(np.uint64))
    if rows * cols <= 4096:
        assert _same(got, tp.layernorm2(ol.Prg(STATE), ln, [x0, x1]))


def test_layer_per_party_eager_and_graph():
    """The small layer captured as a HIP graph under the per-party policy:
    its replays after the policy is switched back give the oracle's shares,
    as do eager runs under either policy between the replays."""
    seq, d, heads, ffn = 32, 64, 2, 128
    W = layer.synthetic_weights(d, ffn, F, 41)
    x = pfss.host_normal_fixed(42, 1.0, 0.0, F, seq * d)
    x0, x1 = _share(x, 43)
    say("transformer layer per-party keystreams, eager and graph seq=%d d=%d" % (seq, d))
    ly = layer.TransformerLayer(STATE, W, seq, d, heads, ffn, F, seed=44)
    xin = (dev(x0), dev(x1))
    out = _pair(seq * d)
    want, _ = tp.layer2(ol.Prg(STATE), ly, (x0, x1))
    with pfss.keystream_per_party():
        ly.eval2(xin, out)
        torch.cuda.synchronize()
        assert _same(_h(out), want)
        g = tasks.capture(lambda: ly.eval2(xin, out))
    torch.cuda.synchronize()
    for rep in range(3):
        out[0].fill_(0)
        out[1].fill_(0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert _same(_h(out), want), "replay %d" % rep
        ly.eval2(xin, out)  # eager, shared policy, between the replays
        torch.cuda.synchronize()
        assert _same(_h(out), want)
    fwant, _ = fp.transformer_layer(x, W, seq, d, heads, ffn, F,
                                    {"nexp": tables.nexp_table(F), "recip": tables.recip_table(F),
                                     "rsqrt": tables.rsqrt_table(F),
                                     "gelu": tables.gelu_table(F)},
                                    tables.inv_len_qf(d), tables.eps_qf())
    assert np.array_equal((want[0] + want[1]).astype(np.uint64), fwant.view(np.uint64))
