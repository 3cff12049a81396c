"""Composite gates with boolean outputs (sufhip_composite_bool2) and the
bucket staging of x^ (sufhip_stage_hatx) on the GPU.

  * staging: the bucket equals the concatenation of the jobs' inputs, plain
    u64 and eff_bits-packed (the oracle's pack_eff_bits layout);
  * composite gate: both parties' boolean shares equal the oracle's two-party
    restatement of the selector / boolean network (tests/twoparty_oracle.py)
    on the same dealer material and DCF bits; the DCF bits equal the oracle's
    myl7 evaluation; the reconstruction of the boolean and arithmetic
    outputs equals the reference's SUF evaluation (oracle/suf_ref.py, pinned
    to the reference's eval_suf_ref) -- at N = 2^16 and N = 2^20;
  * malformed programs and segments are refused on the host."""
import numpy as np
import pytest
import torch

import composite_specs as cs
import oracle_lib as ol
import suf_ref
import twoparty_oracle as tp
from gpu_util import dev, host, say, u64
from suf_amd import composite, native

pytestmark = pytest.mark.gpu

STATE = ol.mt64_bytes(3, ol.PRG_STATE_BYTES).tobytes()
M64 = (1 << 64) - 1


@pytest.fixture(scope="module", autouse=True)
def _init():
    native.call("sufhip_init", 0)


def test_stage_bucket_concatenates_plain_and_packed():
    say("stage_hatx plain + packed segments")
    g = np.random.default_rng(3)
    vals, jobs = [], []
    for ln, eb in ((1000, 64), (777, 13), (4096, 40), (1, 1), (3000, 64), (513, 63)):
        m = M64 if eb == 64 else (1 << eb) - 1
        v = (g.integers(0, 2**64, ln, dtype=np.uint64) & np.uint64(m)).astype(np.uint64)
        vals.append(v)
        if eb == 64:
            jobs.append(dev(v))
        else:
            jobs.append((dev(ol.pack_eff_bits(v, eb)), eb, ln))
    bucket, slices = composite.stage_bucket(jobs)
    torch.cuda.synchronize()
    assert np.array_equal(u64(bucket)[:sum(v.size for v in vals)], np.concatenate(vals))
    assert slices[1] == (1000, 777)


def test_stage_bucket_refuses_bad_segments():
    b = torch.zeros(100, dtype=torch.int64, device="cuda")
    src = torch.zeros(100, dtype=torch.int64, device="cuda")
    segs = (native.StageSeg * 2)()
    segs[0].src, segs[0].len, segs[0].dst, segs[0].eff_bits = src.data_ptr(), 60, 0, 64
    segs[1].src, segs[1].len, segs[1].dst, segs[1].eff_bits = src.data_ptr(), 40, 50, 64
    with pytest.raises(native.SufHipError, match="overlap"):
        native.call("sufhip_stage_hatx", segs, 2, b.data_ptr(), 100, 0)
    segs[1].dst, segs[1].len = 60, 60
    with pytest.raises(native.SufHipError, match="past the bucket"):
        native.call("sufhip_stage_hatx", segs, 2, b.data_ptr(), 100, 0)
    segs[1].dst, segs[1].len, segs[1].eff_bits = 60, 10, 0
    with pytest.raises(native.SufHipError, match="eff_bits"):
        native.call("sufhip_stage_hatx", segs, 2, b.data_ptr(), 100, 0)


def _inputs(n, seed):
    g = np.random.default_rng(seed)
    x = g.integers(0, 2**64, n, dtype=np.uint64)
    near = [0, 999, 1000, 1001, 2047, 2048, 4095, 4096, (1 << 62) - 1, 1 << 62, (1 << 63) - 5001,
            (1 << 63) - 5000, (1 << 63) - 1, 1 << 63, (1 << 63) + (1 << 62), M64]
    x[:len(near)] = near
    k = n // 4
    x[len(near):len(near) + k] = (g.integers(-8192, 8192, k).astype(np.int64)).view(np.uint64)
    return x


def _run(spec, n, seed, share_check=True, oracle_bits=0):
    say("composite gate n=%d seed=%d pieces=%d" % (n, seed, len(spec["pieces"])))
    gate = composite.CompositeGate(spec, n, STATE, seed=seed)
    x = _inputs(n, seed)
    xhat = (x + np.uint64(gate.r_in)).astype(np.uint64)
    xd = dev(xhat)
    ob = tuple(torch.empty(n * gate.ell, dtype=torch.int64, device="cuda") for _ in range(2))
    oa = tuple(torch.empty(n * gate.r, dtype=torch.int64, device="cuda") for _ in range(2))
    gate.eval2(xd, ob, oa)
    torch.cuda.synchronize()
    arith, bools, _ = suf_ref.eval_suf(spec, x)
    rec_b = (u64(ob[0]) + u64(ob[1])).astype(np.uint64).reshape(n, gate.ell)
    assert np.array_equal(rec_b, bools.astype(np.uint64))
    rec_a = (u64(oa[0]) + u64(oa[1])).astype(np.uint64).reshape(n, gate.r)
    assert np.array_equal(rec_a, arith)
    pred = [host(gate.pred[p]).reshape(-1, n) for p in (0, 1)]
    cut = [host(gate.cutb[p]).reshape(-1, n) for p in (0, 1)]
    if share_check:
        want = tp.composite_bool2(gate, pred, cut)
        for p in (0, 1):
            assert np.array_equal(u64(ob[p]).reshape(n, gate.ell), want[p]), p
    if oracle_bits:
        # The DCF bits of the first queries and cuts against the oracle's myl7
        # evaluation at a sample of points.
        prg = ol.Prg(STATE)
        idx = np.arange(min(n, oracle_bits))
        for (bits, k0, k1), got in list(zip(gate.query_keys, zip(*pred)))[:3] + \
                list(zip(gate.cut_keys, zip(*cut)))[:2]:
            for p, k in ((0, k0), (1, k1)):
                kk = np.repeat(host(k).reshape(1, -1), idx.size, axis=0)
                o = ol.myl7_eval_many_bit(prg, ol.GROUP_XOR, bits, kk, xhat[idx], threads=0)
                assert np.array_equal(o, got[p][idx] & 1)
    return gate


@pytest.mark.parametrize("spec", [cs.MIXED, cs.DRELU], ids=["mixed", "drelu"])
def test_composite_gate_shares_and_reconstruction(spec):
    g = _run(spec, 1 << 16, 5, share_check=True, oracle_bits=512)
    if spec is cs.MIXED:
        assert g.and_count > 0 and len(g.wrap_bits) > 0 and len(g.cuts) >= 3


@pytest.mark.parametrize("spec", [cs.MIXED, cs.DRELU], ids=["mixed", "drelu"])
def test_composite_gate_full_size(spec):
    _run(spec, 1 << 20, 9, share_check=True)


def test_composite_refuses_malformed_programs():
    gate = composite.CompositeGate(cs.MIXED, 256, STATE, seed=2)
    ob = tuple(torch.empty(256 * gate.ell, dtype=torch.int64, device="cuda") for _ in range(2))
    gate.pred_bits(dev(np.zeros(256, np.uint64)))
    a = gate.args(ob)
    a.prog[0] = 9  # unknown opcode
    with pytest.raises(native.SufHipError, match="malformed"):
        native.call("sufhip_composite_bool2", native.ctypes.byref(a), 0)
    a = gate.args(ob)
    a.and_count += 1
    with pytest.raises(native.SufHipError, match="and_count"):
        native.call("sufhip_composite_bool2", native.ctypes.byref(a), 0)
    a = gate.args(ob)
    a.prog[0] = native.BOOL_VAR | (a.queries << 4)  # query index out of range
    with pytest.raises(native.SufHipError, match="malformed"):
        native.call("sufhip_composite_bool2", native.ctypes.byref(a), 0)


@pytest.mark.parametrize("spec", [cs.MIXED, cs.DRELU], ids=["mixed", "drelu"])
def test_composite_gate_from_tapes_gives_the_dealt_shares(spec, tmp_path):
    """Each party's key material written to a composite tape file
    (write_composite_tape's format), read back, and loaded into a gate built
    from the tapes and the dealer's compilation alone: the boolean and
    arithmetic shares equal those of the dealt gate, byte for byte."""
    n = 1 << 14
    gate = _run(spec, n, 11, share_check=False)
    x = _inputs(n, 11)
    xd = dev((x + np.uint64(gate.r_in)).astype(np.uint64))
    paths = []
    for p in (0, 1):
        path = tmp_path / ("party%d.tape" % p)
        path.write_bytes(gate.party_tape(p))
        paths.append(path)
    tapes = [pth.read_bytes() for pth in paths]
    say("composite gate from tapes n=%d (%d + %d tape bytes)" % (n, len(tapes[0]), len(tapes[1])))
    g2 = composite.CompositeGate.from_tapes(gate.compiled(), tapes, STATE)
    assert (g2.r_in_share[0] + g2.r_in_share[1]) & M64 == gate.r_in
    outs = []
    for g in (gate, g2):
        ob = tuple(torch.empty(n * g.ell, dtype=torch.int64, device="cuda") for _ in range(2))
        oa = tuple(torch.empty(n * g.r, dtype=torch.int64, device="cuda") for _ in range(2))
        g.eval2(xd, ob, oa)
        torch.cuda.synchronize()
        outs.append([u64(t) for t in ob + oa])
    for a, b in zip(*outs):
        assert np.array_equal(a, b)
    # A tape whose key counts do not fit the compilation is refused.
    other = composite.CompositeGate(cs.DRELU if spec is cs.MIXED else cs.MIXED, n, STATE, seed=12)
    with pytest.raises(ValueError, match="from_tapes"):
        composite.CompositeGate.from_tapes(gate.compiled(), [other.party_tape(0),
                                                             other.party_tape(1)], STATE)
