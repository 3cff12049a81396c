"""Beaver matmul + GapARS truncation for two parties on one GPU: shares equal
the oracle composition (orc_beaver_matmul per party, then orc_trunc_eval),
and the reconstruction at the 128 x 768 x 3072 shape equals (X W) >> 12."""
import numpy as np
import pytest
import torch

import oracle_lib as ol
from gpu_util import dev, host, say, u64
from suf_amd import matmul_gate, native, pfss

pytestmark = pytest.mark.gpu

STATE = ol.mt64_bytes(3, ol.PRG_STATE_BYTES).tobytes()
F = 12


@pytest.fixture(scope="module", autouse=True)
def _init():
    native.call("sufhip_init", 0)


def _operands(M, K, N, seed):
    X = pfss.host_normal_fixed(seed, 1.0, 0.0, F, M * K)
    W = pfss.host_normal_fixed(seed + 1, 0.02, 0.0, F, K * N)
    X0 = pfss.host_mt19937_64(seed + 100, M * K)
    W0 = pfss.host_mt19937_64(seed + 101, K * N)
    return X, W, (X0, (X - X0).astype(np.uint64)), (W0, (W - W0).astype(np.uint64))


def _expected(X, W, M, K, N):
    prod = X.view(np.int64).reshape(M, K) @ W.view(np.int64).reshape(K, N)
    return (prod >> F).view(np.uint64).reshape(-1)


@pytest.mark.parametrize("M,K,N", [(16, 40, 24), (5, 7, 70), (128, 64, 96)])
def test_shares_match_oracle(M, K, N):
    X, W, Xs, Ws = _operands(M, K, N, 8 + M)
    say("beaver matmul+trunc %dx%dx%d" % (M, K, N))
    g = matmul_gate.BeaverMatmulTrunc(M, K, N, STATE, F, seed=10 + N)
    out = [torch.empty(M * N, dtype=torch.int64, device="cuda") for _ in range(2)]
    g.eval2([dev(Xs[0]), dev(Xs[1])], [dev(Ws[0]), dev(Ws[1])], out)
    got = [u64(o) for o in out]
    A = [u64(a) for a in g.A]
    B = [u64(b) for b in g.B]
    C = [u64(c) for c in g.C]
    # The dealer's triple is a real product.
    assert np.array_equal((C[0] + C[1]).astype(np.uint64),
                          ol.beaver_matmul(0, A[0] + A[1], B[0] + B[1], np.zeros(M * K),
                                           np.zeros(K * N), np.zeros(M * N), 1, M, K, N))
    D = (Xs[0] - A[0]) + (Xs[1] - A[1])
    E = (Ws[0] - B[0]) + (Ws[1] - B[1])
    Z = [ol.beaver_matmul(p, D, E, A[p], B[p], C[p], 1, M, K, N) for p in (0, 1)]
    zhat = (Z[0] + Z[1] + np.uint64(sum(g.rin) & matmul_gate.M64)).astype(np.uint64)
    prg = ol.Prg(STATE)
    for p in (0, 1):
        want = ol.trunc_eval(prg, ol.TRUNC_GAPARS, F, host(g.keys[p]), zhat)
        assert np.array_equal(got[p], want), p
    assert np.array_equal((got[0] + got[1]).astype(np.uint64), _expected(X, W, M, K, N))


def test_config_shape_reconstructs():
    M, K, N = 128, 768, 3072
    X, W, Xs, Ws = _operands(M, K, N, 8)
    say("beaver matmul+trunc config shape")
    g = matmul_gate.BeaverMatmulTrunc(M, K, N, STATE, F, seed=10)
    out = [torch.empty(M * N, dtype=torch.int64, device="cuda") for _ in range(2)]
    g.eval2([dev(Xs[0]), dev(Xs[1])], [dev(Ws[0]), dev(Ws[1])], out)
    rec = (u64(out[0]) + u64(out[1])).astype(np.uint64)
    assert np.array_equal(rec, _expected(X, W, M, K, N))
