"""Spline gate (interval LUT + Beaver Horner + two GapARS truncations) for two
parties on one GPU: both parties' output shares equal the oracle composition
of the same protocol steps (orc_lut_eval, orc_beaver_mul, orc_trunc_eval), and
the reconstruction equals the closed form of CubicPolyTask's reference path
(include/runtime/phase_tasks.hpp:2933-2945)."""
import numpy as np
import pytest
import torch

import fixed_point as fp
import oracle_lib as ol
import twoparty_oracle as tp
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
    return tp.spline2(ol.Prg(STATE), gate, [x0, x1])


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("n,seed", [(3000, 7), (777, 8),
                                    # two full passes and a partial third of the chain
                                    # kernel's wide form
                                    (2 * 256 * 1024 + 777, 9)])
def test_shares_match_oracle_pipeline(n, seed, fused):
    alpha, coeffs = spline.spline_spec(F, seed=6)
    x = pfss.host_normal_fixed(5 + seed, 3.0, 8.0, F, n)
    x[:6] = np.array([0, 8 << F, (-8 << F) & spline.M64, 1, spline.M64, (3 << F) - 1],
                     dtype=np.uint64)
    x0, x1 = _shares(x, 40 + seed)
    say("spline gate n=%d seed=%d" % (n, seed))
    gate = spline.SplineGate(n, alpha, coeffs, STATE, F, seed=seed)
    out = [torch.empty(n, dtype=torch.int64, device="cuda") for _ in range(2)]
    gate.eval2([dev(x0), dev(x1)], out, fused=fused)
    g = [u64(o) for o in out]
    o = _oracle_pipeline(gate, x0, x1)
    assert np.array_equal(g[0], o[0]) and np.array_equal(g[1], o[1])
    rec = (g[0] + g[1]).astype(np.uint64)
    assert np.array_equal(rec, fp.spline_closed_form(alpha, coeffs, x, F))


def test_full_size_reconstructs_twice():
    n = 1 << 20
    alpha, coeffs = spline.spline_spec(F, seed=6)
    x = pfss.host_normal_fixed(5, 3.0, 8.0, F, n)
    x0, x1 = _shares(x, 41)
    say("spline gate full size n=%d" % n)
    gate = spline.SplineGate(n, alpha, coeffs, STATE, F, seed=7)
    xd = [dev(x0), dev(x1)]
    out = [torch.empty(n, dtype=torch.int64, device="cuda") for _ in range(2)]
    want = fp.spline_closed_form(alpha, coeffs, x, F)
    for _ in range(2):  # the gate's scratch is reused across calls
        gate.eval2(xd, out)
        rec = (u64(out[0]) + u64(out[1])).astype(np.uint64)
        assert np.array_equal(rec, want)
