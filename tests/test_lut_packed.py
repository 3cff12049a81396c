"""Interval LUT and packed compare (reference GPU blob formats).

CPU: the oracle reconstructs to the closed forms (payload row of the
interval containing x; bitmask 1[x < thr_j]) on the reference's own test
vectors (src/demo/test_cuda_packed_pfss.cpp:31-136) and on random tables;
the product's host blob builders are byte-identical to the oracle's.
GPU: kernel shares equal the oracle's shares, keyed and broadcast.
"""
import numpy as np
import pytest
import torch

import oracle_lib as ol
from gpu_util import Pins, say, u64
from suf_amd import native

M64 = (1 << 64) - 1


def lib():
    return native.load()


def product_lut_key(party, nonce, in_bits, out_words, cuts, payload, seed):
    cuts = np.ascontiguousarray(cuts, dtype=np.uint64)
    payload = np.ascontiguousarray(payload, dtype=np.uint64).ravel()
    intervals = len(cuts) - 1
    blob = np.zeros(lib().sufhip_interval_lut_key_bytes(intervals, out_words), dtype=np.uint8)
    native.call("sufhip_interval_lut_build_key", party, nonce, in_bits, out_words, cuts.ctypes.data,
                intervals, payload.ctypes.data, np.ascontiguousarray(seed).ctypes.data,
                blob.ctypes.data)
    return blob


def product_packed_key(party, nonce, in_bits, thr, seed):
    thr = np.ascontiguousarray(thr, dtype=np.uint64)
    blob = np.zeros(lib().sufhip_packed_lt_key_bytes(len(thr)), dtype=np.uint8)
    native.call("sufhip_packed_lt_build_key", party, nonce, in_bits, thr.ctypes.data, len(thr),
                np.ascontiguousarray(seed).ctypes.data, blob.ctypes.data)
    return blob


def lut_expect(x, cuts, payload, out_words, in_bits):
    m = (1 << in_bits) - 1 if in_bits < 64 else M64
    x &= m
    cs = [int(c) & m for c in cuts[:-1]]
    iv = 0
    for i, c in enumerate(cs):
        if c <= x:
            iv = i
    return [int(v) for v in payload[iv * out_words:(iv + 1) * out_words]]


# ------------------------------------------------------------------ CPU --
def test_seed_from_id_matches_oracle():
    for i, tw in ((1, 0), (2, 7), (12345, 7), (2**63 + 5, 3)):
        s = np.zeros(16, dtype=np.uint8)
        lib().sufhip_seed_from_id(i, tw, s.ctypes.data)
        assert s.tobytes() == ol.seed_from_id(i, tw).tobytes()


def test_blob_builders_match_oracle():
    seed = ol.seed_from_id(3, 7)
    cuts = [0, 20, 40, 64]
    pay = [100, 200, 300, 400, 500, 600]
    for p in (0, 1):
        assert product_lut_key(p, 3, 6, 2, cuts, pay, seed).tobytes() == \
            ol.lut_key(p, 3, 6, 2, cuts, pay, seed).tobytes()
        for thr in ([5, 12, 33, 48, 60], [60, 5, 33], list(range(1, 130))):
            assert product_packed_key(p, 9, 6, thr, seed).tobytes() == \
                ol.packed_key(p, 9, 6, thr, seed).tobytes()


def test_oracle_reference_vectors_reconstruct():
    # test_cuda_packed_pfss.cpp:31-61 and :101-136
    seed = ol.seed_from_id(1, 0)
    thr = [5, 12, 33, 48, 60]
    k0, k1 = ol.packed_key(0, 1, 6, thr, seed), ol.packed_key(1, 1, 6, thr, seed)
    xs = np.array([0, 15, 63], dtype=np.uint64)
    for bc in (0, 1):
        keys0 = k0 if bc else np.tile(k0, (3, 1))
        keys1 = k1 if bc else np.tile(k1, (3, 1))
        r = ol.packed_eval(keys0, len(k0), bc, xs, 1) ^ ol.packed_eval(keys1, len(k1), bc, xs, 1)
        for i, x in enumerate(xs):
            assert int(r[i, 0]) == sum(1 << j for j, t in enumerate(thr) if int(x) < t)
    seed = ol.seed_from_id(2, 7)
    cuts, pay = [0, 20, 40, 64], [100, 200, 300, 400, 500, 600]
    l0, l1 = ol.lut_key(0, 2, 6, 2, cuts, pay, seed), ol.lut_key(1, 2, 6, 2, cuts, pay, seed)
    xs = np.array([0, 25, 50], dtype=np.uint64)
    r = ol.lut_eval(np.tile(l0, (3, 1)), len(l0), 0, xs, 2) + \
        ol.lut_eval(np.tile(l1, (3, 1)), len(l1), 0, xs, 2)
    assert r.tolist() == [[100, 200], [300, 400], [500, 600]]


@pytest.mark.parametrize("in_bits,intervals,ow", [(64, 17, 4), (12, 5, 3), (6, 1, 1), (40, 64, 2)])
def test_oracle_lut_closed_form_random(in_bits, intervals, ow):
    rng = np.random.default_rng(intervals * ow)
    m = (1 << in_bits) - 1 if in_bits < 64 else M64
    cuts = np.sort(rng.integers(0, 2**63, size=intervals + 1).astype(np.uint64) & np.uint64(m))
    pay = rng.integers(0, 2**63, size=intervals * ow).astype(np.uint64)
    seed = ol.seed_from_id(intervals, 7)
    k0, k1 = ol.lut_key(0, 5, in_bits, ow, cuts, pay, seed), ol.lut_key(1, 5, in_bits, ow, cuts, pay, seed)
    xs = rng.integers(0, 2**63, size=300).astype(np.uint64)
    xs[:intervals] = cuts[:intervals]
    xs[-1] = 0
    r = ol.lut_eval(k0, len(k0), 1, xs, ow) + ol.lut_eval(k1, len(k1), 1, xs, ow)
    for i, x in enumerate(xs):
        assert r[i].tolist() == lut_expect(int(x), cuts, pay, ow, in_bits)


@pytest.mark.parametrize("num_thr", [1, 5, 64, 65, 130])
@pytest.mark.parametrize("sorted_thr", [True, False])
def test_oracle_packed_closed_form_random(num_thr, sorted_thr):
    rng = np.random.default_rng(num_thr)
    in_bits = 20
    thr = rng.integers(0, 1 << in_bits, size=num_thr).astype(np.uint64)
    if sorted_thr:
        thr = np.sort(thr)
    seed = ol.seed_from_id(num_thr, 0)
    k0, k1 = ol.packed_key(0, 3, in_bits, thr, seed), ol.packed_key(1, 3, in_bits, thr, seed)
    ow = (num_thr + 63) // 64
    xs = rng.integers(0, 1 << in_bits, size=200).astype(np.uint64)
    r = ol.packed_eval(k0, len(k0), 1, xs, ow) ^ ol.packed_eval(k1, len(k1), 1, xs, ow)
    for i, x in enumerate(xs):
        v = sum(1 << j for j, t in enumerate(thr) if int(x) < int(t))
        assert [int(w) for w in r[i]] == [(v >> (64 * w)) & M64 for w in range(ow)]


def test_eval_rejects_bad_geometry():
    rc = lib().sufhip_interval_lut_eval(1, 216, 1, 3, 2, 1, 4, 1, None)
    assert rc == -1 and b"key_bytes" in lib().sufhip_last_error()
    rc = lib().sufhip_packed_lt_eval(1, 248, 1, 5, 2, 1, 4, 1, None)
    assert rc == -1 and b"out_words" in lib().sufhip_last_error()


# ------------------------------------------------------------------ GPU --
@pytest.mark.gpu
@pytest.mark.parametrize("in_bits,intervals,ow", [(64, 18, 4), (12, 5, 3), (6, 3, 2), (64, 1, 1),
                                                  (64, 2000, 5)])
@pytest.mark.parametrize("broadcast", [True, False])
def test_gpu_lut_matches_oracle(in_bits, intervals, ow, broadcast):
    native.call("sufhip_init", 0)
    say("lut in_bits=%d intervals=%d ow=%d bcast=%s" % (in_bits, intervals, ow, broadcast))
    P = Pins()
    rng = np.random.default_rng(in_bits + intervals + ow)
    m = (1 << in_bits) - 1 if in_bits < 64 else M64
    n = 5000 if broadcast else 700
    cuts = np.sort(rng.integers(0, 2**63, size=intervals + 1).astype(np.uint64) & np.uint64(m))
    pay = rng.integers(0, 2**63, size=intervals * ow).astype(np.uint64)
    xs = rng.integers(0, 2**63, size=n).astype(np.uint64) * np.uint64(2)
    xs[: min(n, intervals)] = cuts[: min(n, intervals)]
    for party in (0, 1):
        seed = ol.seed_from_id(7, 7)
        if broadcast:
            key = ol.lut_key(party, 7, in_bits, ow, cuts, pay, seed)
            keys = key
        else:
            # distinct keys per element (nonce varies)
            keys = np.stack([ol.lut_key(party, 100 + i, in_bits, ow, cuts, pay, seed)
                             for i in range(n)])
        kb = keys.shape[-1]
        out = torch.empty(n * ow, dtype=torch.int64, device="cuda")
        native.call("sufhip_interval_lut_eval", P(keys), kb, int(broadcast), intervals, ow, P(xs),
                    n, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
        exp = ol.lut_eval(keys, kb, int(broadcast), xs, ow)
        assert np.array_equal(u64(out).reshape(n, ow), exp), party


@pytest.mark.gpu
@pytest.mark.parametrize("num_thr", [5, 64, 65, 200, 1500])
@pytest.mark.parametrize("sorted_thr", [True, False])
@pytest.mark.parametrize("broadcast", [True, False])
def test_gpu_packed_matches_oracle(num_thr, sorted_thr, broadcast):
    native.call("sufhip_init", 0)
    say("packed thr=%d sorted=%s bcast=%s" % (num_thr, sorted_thr, broadcast))
    P = Pins()
    rng = np.random.default_rng(num_thr + 2 * sorted_thr)
    in_bits = 37
    thr = rng.integers(0, 1 << in_bits, size=num_thr).astype(np.uint64)
    if sorted_thr:
        thr = np.sort(thr)
    ow = (num_thr + 63) // 64
    n = 3000 if broadcast else 300
    xs = rng.integers(0, 1 << in_bits, size=n).astype(np.uint64)
    seed = ol.seed_from_id(num_thr, 0)
    for party in (0, 1):
        if broadcast:
            keys = ol.packed_key(party, 11, in_bits, thr, seed)
        else:
            keys = np.stack([ol.packed_key(party, 50 + i, in_bits, thr, seed) for i in range(n)])
        kb = keys.shape[-1]
        out = torch.empty(n * ow, dtype=torch.int64, device="cuda")
        native.call("sufhip_packed_lt_eval", P(keys), kb, int(broadcast), num_thr, ow, P(xs), n,
                    out.data_ptr(), torch.cuda.current_stream().cuda_stream)
        exp = ol.packed_eval(keys, kb, int(broadcast), xs, ow)
        assert np.array_equal(u64(out).reshape(n, ow), exp), party


def test_oracle_lut_eval_at_matches_the_batch_slice():
    rng = np.random.default_rng(9)
    cuts = np.sort(rng.integers(0, 1 << 20, 9, dtype=np.uint64))
    payload = rng.integers(0, 1 << 63, 8 * 3, dtype=np.uint64)
    blob = ol.lut_key(0, 5, 20, 3, cuts, payload, ol.seed_from_id(5, 7))
    xs = rng.integers(0, 1 << 20, 300, dtype=np.uint64)
    whole = ol.lut_eval(blob, blob.size, 1, xs, 3)
    part = ol.lut_eval(blob, blob.size, 1, xs[100:250], 3, idx0=100)
    assert np.array_equal(whole[100:250], part)
    assert not np.array_equal(ol.lut_eval(blob, blob.size, 1, xs[100:250], 3), part)
