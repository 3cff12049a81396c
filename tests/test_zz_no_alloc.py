"""sufhip_trunc_eval_noalloc (static per-GPU workspace, no allocation)
against sufhip_trunc_eval with a caller workspace: byte-equal shares on two
calls in a row, the second with a smaller batch (and a different gate), plus
a reconstruction check and the size limit's error; a warm call leaves the
device's free memory unchanged, and the call recorded in a HIP graph gives
the eager shares on every replay with a refilled input."""
import numpy as np
import pytest
import torch

import oracle_lib as ol
from gpu_util import dev, say, u64
from suf_amd import native, pfss, tasks

pytestmark = pytest.mark.gpu

M64 = (1 << 64) - 1
STATE = ol.mt64_bytes(3, ol.PRG_STATE_BYTES).tobytes()


@pytest.fixture(scope="module", autouse=True)
def _init():
    native.call("sufhip_init", 0)


def _noalloc(kind, f, key, xd):
    n = xd.numel()
    y = torch.empty(n, dtype=torch.int64, device="cuda")
    native.call("sufhip_trunc_eval_noalloc", kind, f, pfss._state_buf(STATE), key.data_ptr(),
                key.numel(), xd.data_ptr(), n, y.data_ptr(), pfss._stream())
    return y


def _case(kind, f, n, seed):
    rng = np.random.default_rng(seed)
    rnd = rng.integers(0, 1 << 64, ol.TRUNC_RAND_WORDS, dtype=np.uint64)
    say("no-alloc trunc kind=%d f=%d n=%d work=%d" %
        (kind, f, n, native.load().sufhip_trunc_work_bytes(f, n)))
    k0, k1 = pfss.trunc_gen(kind, f, STATE, rnd)
    lim = 1 << 40
    xs = rng.integers(-lim, lim, n, dtype=np.int64).view(np.uint64)
    xhat = (xs + rnd[0]).astype(np.uint64)
    xd = dev(xhat)
    got, want = [], []
    for k in (k0, k1):
        got.append(u64(_noalloc(kind, f, k, xd)))
        want.append(u64(pfss.trunc_eval(kind, f, STATE, k, xd)))
    torch.cuda.synchronize()
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
    rec = (got[0] + got[1]).astype(np.uint64)
    if kind == ol.TRUNC_TR:
        want_rec = xs >> np.uint64(f)
    else:
        want_rec = (xs.view(np.int64) >> f).view(np.uint64)
    assert np.array_equal(rec, want_rec)


def test_noalloc_two_calls_second_smaller():
    # Full-domain table at f = 14 (the largest table), then a smaller batch
    # with a different gate and width: the second call must not see the
    # first one's table.
    _case(ol.TRUNC_GAPARS, 14, 1 << 18, 1)
    _case(ol.TRUNC_GAPARS, 12, 3000, 2)
    # A prefix frontier (f = 24, n < 2^16) and the 64-bit wrap key path.
    _case(ol.TRUNC_ARS, 24, 20000, 3)
    _case(ol.TRUNC_TR, 12, 777, 4)


def test_noalloc_rejects_oversize():
    f, n = 30, 1 << 20
    assert native.load().sufhip_trunc_work_bytes(f, n) > \
        native.load().sufhip_trunc_noalloc_max_work_bytes()
    rng = np.random.default_rng(5)
    rnd = rng.integers(0, 1 << 64, ol.TRUNC_RAND_WORDS, dtype=np.uint64)
    k0, _ = pfss.trunc_gen(ol.TRUNC_GAPARS, f, STATE, rnd)
    xd = torch.zeros(n, dtype=torch.int64, device="cuda")
    with pytest.raises(native.SufHipError, match="static workspace"):
        _noalloc(ol.TRUNC_GAPARS, f, k0, xd)


def test_noalloc_allocates_nothing_and_replays_in_a_graph():
    kind, f, n = ol.TRUNC_GAPARS, 12, 1 << 16
    rng = np.random.default_rng(6)
    rnd = rng.integers(0, 1 << 64, ol.TRUNC_RAND_WORDS, dtype=np.uint64)
    k0, _ = pfss.trunc_gen(kind, f, STATE, rnd)
    lim = 1 << 40
    xd = dev((rng.integers(-lim, lim, n, dtype=np.int64).view(np.uint64) + rnd[0])
             .astype(np.uint64))
    y = torch.empty(n, dtype=torch.int64, device="cuda")
    state = pfss._state_buf(STATE)

    def run():
        native.call("sufhip_trunc_eval_noalloc", kind, f, state, k0.data_ptr(), k0.numel(),
                    xd.data_ptr(), n, y.data_ptr(), pfss._stream())

    say("no-alloc trunc: warm call, then free memory around a second call")
    run()
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    run()
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free0 == free1, "free device memory changed: %d -> %d" % (free0, free1)
    say("no-alloc trunc: captured in a HIP graph, three replays with refilled inputs")
    g = tasks.capture(run)
    for rep in range(3):
        xs = rng.integers(-lim, lim, n, dtype=np.int64).view(np.uint64)
        xd.copy_(dev((xs + rnd[0]).astype(np.uint64)))
        y.fill_(0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = u64(pfss.trunc_eval(kind, f, STATE, k0, xd))
        torch.cuda.synchronize()
        assert np.array_equal(u64(y), want), "replay %d differs from the eager call" % rep
