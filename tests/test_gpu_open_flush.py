"""One flush of a two-party open collector (sufhip_open_flush2, through the C
ABI) against the oracle's pack_eff_bits and open_add
(src/runtime/open_collector.cpp:357-791, cuda/cuda_primitives.cu:26-112):
ragged requests, eff_bits below, at and above the ring width, plain and
sign-extended opens, and the secret recovered where the packing is exact."""
import numpy as np
import pytest
import torch

import oracle_lib as ol
from gpu_util import dev, say, u64
from suf_amd import native

pytestmark = pytest.mark.gpu

M64 = (1 << 64) - 1


@pytest.fixture(scope="module", autouse=True)
def _init():
    native.call("sufhip_init", 0)


def S():
    return torch.cuda.current_stream().cuda_stream


def rng_u64(rng, n):
    return rng.integers(0, 2**63, size=n, dtype=np.uint64) * np.uint64(2) + \
        rng.integers(0, 2, size=n, dtype=np.uint64)


def flush(shares0, shares1, eff_bits, ring_bits, sign_extend):
    held = [dev(s) if len(s) else None for s in shares0 + shares1]
    k = len(shares0)
    reqs = (native.OpenReq * max(k, 1))()
    for i in range(k):
        n = len(shares0[i])
        reqs[i].share[0] = held[i].data_ptr() if n else None
        reqs[i].share[1] = held[k + i].data_ptr() if n else None
        reqs[i].len = n
    total = sum(len(s) for s in shares0)
    wb = native.load().sufhip_open_flush2_work_bytes(total, eff_bits)
    work = torch.empty(max(wb, 8), dtype=torch.uint8, device="cuda")
    out = torch.empty(max(total, 1), dtype=torch.int64, device="cuda")
    rmask = (1 << ring_bits) - 1 if ring_bits < 64 else M64
    native.call("sufhip_open_flush2", reqs, k, eff_bits, ring_bits, sign_extend, out.data_ptr(),
                work.data_ptr(), wb, S())
    return u64(out)[:total], rmask


def expected(shares0, shares1, eff_bits, ring_bits, rmask, sign_extend):
    s0 = np.concatenate(shares0) if shares0 else np.zeros(0, np.uint64)
    s1 = np.concatenate(shares1) if shares1 else np.zeros(0, np.uint64)
    n = len(s0)
    msg1 = ol.pack_eff_bits(s1, eff_bits) if eff_bits < 64 else s1
    return ol.open_add(s0, msg1, eff_bits, n, ring_bits, rmask, sign_extend)


LENS = [[1], [5, 0, 1000, 3], [65537, 17], [7] * 70 + [300]]


@pytest.mark.parametrize("lens", LENS, ids=["one", "ragged", "large", "many"])
@pytest.mark.parametrize("ring_bits,eff_bits", [(64, 64), (50, 50), (64, 50), (50, 64),
                                                (37, 13), (13, 13)])
@pytest.mark.parametrize("sign_extend", [0, 1])
def test_flush_matches_oracle(lens, ring_bits, eff_bits, sign_extend):
    say("open_flush2 lens=%s ring=%d eff=%d sx=%d" % (lens[:4], ring_bits, eff_bits, sign_extend))
    rng = np.random.default_rng(sum(lens) + 7 * ring_bits + eff_bits + 1000 * sign_extend)
    s0 = [rng_u64(rng, n) for n in lens]
    s1 = [rng_u64(rng, n) for n in lens]
    got, rmask = flush(s0, s1, eff_bits, ring_bits, sign_extend)
    assert np.array_equal(got, expected(s0, s1, eff_bits, ring_bits, rmask, sign_extend))


@pytest.mark.parametrize("ring_bits,eff_bits", [(64, 64), (50, 50), (37, 37), (64, 40)])
def test_flush_recovers_the_secret(ring_bits, eff_bits):
    """x = s0 + s1 over Z_2^ring: with eff_bits >= ring_bits every split opens
    to x; with eff_bits < ring_bits, splits whose party-1 share fits eff_bits
    (the reference's dynamic packing) do."""
    say("open_flush2 secret ring=%d eff=%d" % (ring_bits, eff_bits))
    rng = np.random.default_rng(ring_bits * 64 + eff_bits)
    rmask = np.uint64((1 << ring_bits) - 1 if ring_bits < 64 else M64)
    lens = [3000, 1, 257]
    xs = [rng_u64(rng, n) & rmask for n in lens]
    fit = np.uint64((1 << eff_bits) - 1 if eff_bits < 64 else M64)
    s1 = [rng_u64(rng, n) & fit & rmask for n in lens]
    s0 = [(x - b) & rmask for x, b in zip(xs, s1)]
    got, _ = flush(s0, s1, eff_bits, ring_bits, 0)
    assert np.array_equal(got, np.concatenate(xs))


def test_flush_rejects_bad_arguments():
    reqs = (native.OpenReq * 1)()
    reqs[0].len = 4
    with pytest.raises(native.SufHipError):
        native.call("sufhip_open_flush2", reqs, 1, 64, 64, 0, None, None, 0, None)
    rng = np.random.default_rng(3)
    a, b = dev(rng_u64(rng, 4)), dev(rng_u64(rng, 4))
    reqs[0].share[0], reqs[0].share[1] = a.data_ptr(), b.data_ptr()
    out = torch.empty(4, dtype=torch.int64, device="cuda")
    small = torch.empty(8, dtype=torch.uint8, device="cuda")
    with pytest.raises(native.SufHipError):
        native.call("sufhip_open_flush2", reqs, 1, 64, 64, 0, out.data_ptr(), small.data_ptr(), 8,
                    None)
    with pytest.raises(native.SufHipError):
        native.call("sufhip_open_flush2", reqs, 1, 0, 64, 0, out.data_ptr(), small.data_ptr(), 8,
                    None)
