"""Spline gate (interval LUT + Beaver Horner + two GapARS truncations) for two
parties on one GPU: both parties' output shares equal the oracle composition
of the same protocol steps (orc_lut_eval, orc_beaver_mul, orc_trunc_eval), and
the reconstruction equals the closed form of CubicPolyTask's reference path
(include/runtime/phase_tasks.hpp:2933-2945)."""
import numpy as np
import pytest
import torch

import oracle_lib as ol
from gpu_util import dev, host, say, u64
from suf_amd import native, pfss, spline

pytestmark = pytest.mark.gpu

STATE = ol.mt64_bytes(3, ol.PRG_STATE_BYTES).tobytes()
F = 12


@pytest.fixture(scope="module", autouse=True)
def _init():
    native.call("sufhip_init", 0)


def _shares(x, seed):
    x0 = pfss.host_mt19937_64(seed, x.size)
    return x0, (x - x0).astype(np.uint64)


def _oracle_pipeline(gate, x0, x1):
    """Both parties' outputs, step by step on the CPU oracle."""
    prg = ol.Prg(STATE)
    n = x0.size
    rin = sum(gate.rin) & spline.M64
    xhat = (x0 + x1 + np.uint64(rin)).astype(np.uint64)
    C = [ol.lut_eval(host(gate.lut[p]), gate.lut_key_bytes, 1, xhat, 4).reshape(n, 4)
         for p in (0, 1)]
    tri = [[u64(t).reshape(n, 3) for t in pair] for pair in gate.triples]

    def mul(u, v, t):
        d = (u[0] - t[0][:, 0]) + (u[1] - t[1][:, 0])
        e = (v[0] - t[0][:, 1]) + (v[1] - t[1][:, 1])
        return [ol.beaver_mul(p, t[p][:, 0], t[p][:, 1], t[p][:, 2], d, e) for p in (0, 1)]

    sh = np.uint64(F)
    u = mul([C[0][:, 3], C[1][:, 3]], [x0, x1], tri[0])
    u = [u[p] + (C[p][:, 2] << sh) for p in (0, 1)]
    pz = mul(u, [x0, x1], tri[1])
    t1, t2 = gate.trunc
    phat = (pz[0] + pz[1] + np.uint64(sum(t1["rin"]) & spline.M64)).astype(np.uint64)
    y = [ol.trunc_eval(prg, ol.TRUNC_GAPARS, t1["f"], host(t1["keys"][p]), phat) for p in (0, 1)]
    q = [y[p] + (C[p][:, 1] << sh) for p in (0, 1)]
    rz = mul(q, [x0, x1], tri[2])
    rhat = (rz[0] + rz[1] + np.uint64(sum(t2["rin"]) & spline.M64)).astype(np.uint64)
    y2 = [ol.trunc_eval(prg, ol.TRUNC_GAPARS, t2["f"], host(t2["keys"][p]), rhat) for p in (0, 1)]
    return [(y2[p] + C[p][:, 0]).astype(np.uint64) for p in (0, 1)]


@pytest.mark.parametrize("n,seed", [(3000, 7), (777, 8)])
def test_shares_match_oracle_pipeline(n, seed):
    alpha, coeffs = spline.spline_spec(F, seed=6)
    x = pfss.host_normal_fixed(5 + seed, 3.0, 8.0, F, n)
    x[:6] = np.array([0, 8 << F, (-8 << F) & spline.M64, 1, spline.M64, (3 << F) - 1],
                     dtype=np.uint64)
    x0, x1 = _shares(x, 40 + seed)
    say("spline gate n=%d seed=%d" % (n, seed))
    gate = spline.SplineGate(n, alpha, coeffs, STATE, F, seed=seed)
    out = [torch.empty(n, dtype=torch.int64, device="cuda") for _ in range(2)]
    gate.eval2([dev(x0), dev(x1)], out)
    g = [u64(o) for o in out]
    o = _oracle_pipeline(gate, x0, x1)
    assert np.array_equal(g[0], o[0]) and np.array_equal(g[1], o[1])
    rec = (g[0] + g[1]).astype(np.uint64)
    assert np.array_equal(rec, spline.spline_eval_ref(alpha, coeffs, x, F))


def test_full_size_reconstructs_twice():
    n = 1 << 20
    alpha, coeffs = spline.spline_spec(F, seed=6)
    x = pfss.host_normal_fixed(5, 3.0, 8.0, F, n)
    x0, x1 = _shares(x, 41)
    say("spline gate full size n=%d" % n)
    gate = spline.SplineGate(n, alpha, coeffs, STATE, F, seed=7)
    xd = [dev(x0), dev(x1)]
    out = [torch.empty(n, dtype=torch.int64, device="cuda") for _ in range(2)]
    want = spline.spline_eval_ref(alpha, coeffs, x, F)
    for _ in range(2):  # the gate's scratch is reused across calls
        gate.eval2(xd, out)
        rec = (u64(out[0]) + u64(out[1])).astype(np.uint64)
        assert np.array_equal(rec, want)
