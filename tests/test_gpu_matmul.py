"""GPU Beaver matrix product (libsuf_hip.so through the C ABI) against the
oracle, and the config-3 shape (X[128x768] * W[768x3072]) by reconstruction:
z0 + z1 == X * W mod 2^64."""
import numpy as np
import pytest
import torch

import oracle_lib as ol
from gpu_util import Pins, say, u64
from suf_amd import native

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _init():
    native.call("sufhip_init", 0)


def rng_u64(rng, n):
    return rng.integers(0, 2**63, size=n, dtype=np.uint64) * np.uint64(2) + \
        rng.integers(0, 2, size=n, dtype=np.uint64)


@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (5, 11, 7), (32, 16, 64), (33, 17, 65), (70, 40, 130)])
@pytest.mark.parametrize("wt", [0, 1])
@pytest.mark.parametrize("batches", [1, 3])
@pytest.mark.parametrize("scale", [(0, 0, 0), (1, 3, 12), (1, -7, 70), (1, 5, 0)])
def test_matmul_matches_oracle(M, K, N, wt, batches, scale):
    say("matmul %dx%dx%d wt=%d b=%d scale=%s" % (M, K, N, wt, batches, scale))
    P = Pins()
    rng = np.random.default_rng(M * 1000 + K * 10 + N + wt)
    D = rng_u64(rng, batches * M * K)
    E = rng_u64(rng, batches * K * N)
    A = rng_u64(rng, M * K)
    B = rng_u64(rng, K * N)
    C = rng_u64(rng, M * N)
    hs, mc, ms = scale
    for party in (0, 1):
        out = torch.empty(batches * M * N, dtype=torch.int64, device="cuda")
        if batches == 1:
            native.call("sufhip_beaver_matmul2d", party, P(D), P(E), P(A), P(B), P(C), M, K, N, wt,
                        hs, mc, ms, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
        else:
            native.call("sufhip_beaver_matmul2d_batched", party, P(D), P(E), P(A), P(B), P(C),
                        batches, M, K, N, wt, hs, mc, ms, out.data_ptr(),
                        torch.cuda.current_stream().cuda_stream)
        exp = ol.beaver_matmul(party, D, E, A, B, C, batches, M, K, N, wt, hs, mc, ms)
        assert np.array_equal(u64(out), exp), party


def test_config3_shape_reconstructs_xw():
    """X[128x768] (Q12) times W[768x3072] (Q12), secret-shared via seeded triples."""
    say("matmul config-3 shape")
    P = Pins()
    M, K, N = 128, 768, 3072
    rng = np.random.default_rng(8)
    X = (np.round(rng.normal(0, 1, M * K) * 4096)).astype(np.int64).view(np.uint64)
    W = (np.round(rng.normal(0, 0.02, K * N) * 4096)).astype(np.int64).view(np.uint64)
    A, B = rng_u64(rng, M * K), rng_u64(rng, K * N)
    # C = A * B mod 2^64 via the oracle's product with zero openings
    zeros_d = np.zeros(M * K, np.uint64)
    zeros_e = np.zeros(K * N, np.uint64)
    C = ol.beaver_matmul(1, zeros_d, B, A, zeros_e, np.zeros(M * N, np.uint64), 1, M, K, N)
    A0 = rng_u64(rng, M * K)
    B0 = rng_u64(rng, K * N)
    C0 = rng_u64(rng, M * N)
    shares = ((A0, B0, C0), (A - A0, B - B0, C - C0))
    D, E = X - A, W - B
    outs = []
    for party, (a, b, c) in enumerate(shares):
        out = torch.empty(M * N, dtype=torch.int64, device="cuda")
        native.call("sufhip_beaver_matmul2d", party, P(D), P(E), P(a), P(b), P(c), M, K, N, 0, 0,
                    0, 0, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
        outs.append(u64(out))
    z = outs[0] + outs[1]
    xw = ol.beaver_matmul(1, zeros_d, W, X, zeros_e, np.zeros(M * N, np.uint64), 1, M, K, N)
    assert np.array_equal(z, xw)


@pytest.mark.parametrize("M,K,N", [(32, 32, 64), (64, 96, 128), (128, 768, 3072), (96, 3072, 64)])
def test_mfma_limb_matmul_matches_valu_and_oracle(M, K, N):
    say("mfma limb matmul %dx%dx%d" % (M, K, N))
    P = Pins()
    rng = np.random.default_rng(M + 7 * K + 13 * N)
    D = rng_u64(rng, M * K)
    E = rng_u64(rng, K * N)
    A = rng_u64(rng, M * K)
    B = rng_u64(rng, K * N)
    C = rng_u64(rng, M * N)
    # Digit edge cases: all-ones (every digit -1 with borrows), 2^63, 0x80 bytes.
    D[:8] = [2**64 - 1, 2**63, 0x8080808080808080, 0x7F7F7F7F7F7F7F7F, 1, 0, 0xFF, 2**63 - 1]
    E[:8] = [2**64 - 1, 0x8080808080808080, 2**63, 3, 0, 2**64 - 1, 0x80, 0xFFFFFFFF00000000]
    lib = native.load()
    wb = lib.sufhip_beaver_matmul2d_mfma_work_bytes(M, K, N)
    work = torch.empty((wb + 7) // 8, dtype=torch.int64, device="cuda")
    for party in (0, 1):
        out = torch.empty(M * N, dtype=torch.int64, device="cuda")
        ref = torch.empty(M * N, dtype=torch.int64, device="cuda")
        native.call("sufhip_beaver_matmul2d_mfma", party, P(D), P(E), P(A), P(B), P(C), M, K, N,
                    out.data_ptr(), work.data_ptr(), wb, None)
        native.call("sufhip_beaver_matmul2d", party, P(D), P(E), P(A), P(B), P(C), M, K, N, 0, 0,
                    0, 0, ref.data_ptr(), None)
        torch.cuda.synchronize()
        got = u64(out)
        assert np.array_equal(got, u64(ref)), party
        if M * N * K <= 64 * 96 * 128:
            assert np.array_equal(got, ol.beaver_matmul(party, D, E, A, B, C, 1, M, K, N))


def test_mfma_limb_matmul_rejects_bad_shapes():
    lib = native.load()
    for M, K, N in [(33, 32, 64), (32, 31, 64), (32, 32, 96), (32, 8192, 64)]:
        rc = lib.sufhip_beaver_matmul2d_mfma(0, 1, 1, 1, 1, 1, M, K, N, 1, 16, 1 << 30, None)
        assert rc == -1  # SUFHIP_ERR_INVALID, before any device work
