"""GPU parity of AES-128, the myl7 PRG and the myl7 DCF (gen + eval) with the
oracle, the reference-made golden vectors and the closed form 1[x < alpha].
All calls go through the C ABI (libsuf_hip.so)."""
import json
import os

import numpy as np
import pytest
import torch

import oracle_lib as ol
from gpu_util import dev, host, say, u64
from suf_amd import native, pfss

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "dcf_myl7.json")
MODES = {"bit": native.DCF_OUT_BIT, "bytes": native.DCF_OUT_BYTES, "packed": native.DCF_OUT_PACKED}


@pytest.fixture(scope="module", autouse=True)
def _init():
    native.call("sufhip_init", 0)


def _state(seed):
    return ol.mt64_bytes(seed, ol.PRG_STATE_BYTES).tobytes()


def test_aes_ctr_matches_oracle():
    say("aes128_ctr 1024 blocks")
    key = ol.mt64_bytes(12345, 16)
    rk = ol.aes_expand(key.tobytes())
    out = pfss.aes128_ctr(rk.tobytes(), 5, 0xDEADBEEF, 1024)
    torch.cuda.synchronize()
    ref = np.zeros(1024 * 16, dtype=np.uint8)
    ol.LIB.orc_aes128_ctr(ol.ptr(rk), 5, 0xDEADBEEF, 1024, ol.ptr(ref))
    assert np.array_equal(host(out), ref)


def test_aes_fips197():
    say("aes128 fips-197 C.1")
    rk = ol.aes_expand(bytes(range(16)))
    # CTR block 0 with ctr_lo/ctr_hi chosen so the block equals 00112233..ff
    lo = int.from_bytes(bytes.fromhex("0011223344556677"), "little")
    hi = int.from_bytes(bytes.fromhex("8899aabbccddeeff"), "little")
    out = pfss.aes128_ctr(rk.tobytes(), lo, hi, 1)
    assert host(out).tobytes().hex() == "69c4e0d86a7b0430d8cdb78070b4c55a"


@pytest.mark.parametrize("blocks,lo,hi", [(1, 5, 0xDEADBEEF), (31, 0, 7), (1024, 5, 0xDEADBEEF),
                                          (1037, 0xFFFFFFFFFFFFFFF0, 3), (4096 + 5, 96, 0)])
def test_aes_ctr_bitsliced_matches_oracle(blocks, lo, hi):
    """The bitsliced CTR kernel (32 blocks per lane as slices, tower-field
    S-box) writes the oracle's keystream: partial last groups, counters whose
    low bits carry inside a lane's group (lo mod 32 != 0) and across 2^64."""
    say("aes128_ctr bitsliced blocks=%d lo=%x" % (blocks, lo))
    key = ol.mt64_bytes(4242, 16)
    rk = ol.aes_expand(key.tobytes())
    out = pfss.aes128_ctr(rk.tobytes(), lo, hi, blocks, bitsliced=True)
    ref = np.zeros(blocks * 16, dtype=np.uint8)
    ol.LIB.orc_aes128_ctr(ol.ptr(rk), lo, hi, blocks, ol.ptr(ref))
    assert np.array_equal(host(out), ref)


def test_aes_fips197_bitsliced():
    say("aes128 bitsliced fips-197 C.1")
    rk = ol.aes_expand(bytes(range(16)))
    lo = int.from_bytes(bytes.fromhex("0011223344556677"), "little")
    hi = int.from_bytes(bytes.fromhex("8899aabbccddeeff"), "little")
    out = pfss.aes128_ctr(rk.tobytes(), lo, hi, 1, bitsliced=True)
    assert host(out).tobytes().hex() == "69c4e0d86a7b0430d8cdb78070b4c55a"


@pytest.mark.parametrize("blocks", [1, 4, 8])
def test_prg_mmo_matches_oracle(blocks):
    say("prg_mmo blocks=%d" % blocks)
    state = _state(3)
    prg = ol.Prg(state)
    seeds = ol.mt64_bytes(77, 16 * 300)
    out = host(pfss.prg_mmo(state, dev(seeds), blocks)).reshape(300, 16 * blocks)
    for i in range(300):
        ref = np.zeros(16 * blocks, dtype=np.uint8)
        ol.LIB.orc_prg(prg.buf, ol.ptr(ref), 16 * blocks, ol.ptr(seeds[16 * i:16 * i + 16]))
        assert out[i].tobytes() == ref.tobytes(), i


def _golden():
    with open(GOLDEN) as f:
        return json.load(f)


@pytest.mark.parametrize("mode", ["bit", "bytes", "packed"])
def test_eval_reproduces_reference_golden_vectors(mode):
    doc = _golden()
    state = bytes.fromhex(doc["prg_state"])
    for ci, c in enumerate(doc["cases"]):
        g = native.GROUP_XOR if c["group"] == "xor" else native.GROUP_ADD
        in_bits = c["in_bits"]
        plen = len(bytes.fromhex(c["payload"]))
        xs = np.array([int(x) for x in c["xs"]], dtype=np.uint64)
        for p in (0, 1):
            key = np.frombuffer(bytes.fromhex(c["key%d" % p]), dtype=np.uint8).copy()
            say("golden case %d party %d mode %s" % (ci, p, mode))
            keys = dev(np.tile(key, (len(xs), 1)))
            out = pfss.dcf_eval(g, in_bits, plen, state, keys, dev(xs), MODES[mode],
                                out_bytes=plen)
            exp = c["out%d" % p]
            if mode == "bit":
                assert list(host(out)) == exp["bit"], ci
            elif mode == "bytes":
                got = host(out).reshape(len(xs), plen)
                assert [r.tobytes().hex() for r in got] == exp["full"], ci
            else:
                words = u64(out)
                bits = [(int(words[j // 64]) >> (j % 64)) & 1 for j in range(len(xs))]
                assert bits == exp["bit"], ci
            # broadcast-key path gives the same answer
            outb = pfss.dcf_eval(g, in_bits, plen, state, dev(key), dev(xs), MODES[mode],
                                 out_bytes=plen, broadcast=True)
            assert torch.equal(out, outb)


@pytest.mark.parametrize("group", [native.GROUP_XOR, native.GROUP_ADD])
@pytest.mark.parametrize("in_bits,plen", [(64, 1), (64, 8), (13, 1), (16, 20), (1, 3), (37, 16)])
def test_gen_matches_oracle_bytes(group, in_bits, plen):
    say("dcf_gen group=%d in_bits=%d plen=%d" % (group, in_bits, plen))
    state = _state(3)
    prg = ol.Prg(state)
    n = 67
    rng = np.random.default_rng(in_bits * 100 + plen)
    mask = (1 << in_bits) - 1
    alphas = np.array([int(v) & mask for v in rng.integers(0, 2**63, size=n)], dtype=np.uint64)
    alphas[0] = 0
    alphas[1] = mask
    chunks = (plen + 15) // 16
    seeds = rng.integers(0, 256, size=(n, chunks * 32), dtype=np.uint8)
    payload = rng.integers(0, 256, size=plen, dtype=np.uint8)
    k0, k1 = pfss.dcf_gen(group, in_bits, state, dev(alphas), dev(payload), dev(seeds))
    k0 = host(k0)
    k1 = host(k1)
    for i in range(n):
        r0, r1 = ol.myl7_gen(prg, group, in_bits, int(alphas[i]), payload.tobytes(), seeds[i])
        assert k0[i].tobytes() == r0.tobytes(), i
        assert k1[i].tobytes() == r1.tobytes(), i


def test_gen_per_element_payload():
    say("dcf_gen per-element payload")
    state = _state(9)
    prg = ol.Prg(state)
    n, plen = 40, 8
    rng = np.random.default_rng(5)
    alphas = rng.integers(0, 2**63, size=n).astype(np.uint64)
    seeds = rng.integers(0, 256, size=(n, 32), dtype=np.uint8)
    pay = rng.integers(0, 256, size=(n, plen), dtype=np.uint8)
    k0, k1 = pfss.dcf_gen(native.GROUP_ADD, 64, state, dev(alphas), dev(pay), dev(seeds),
                          payload_broadcast=False)
    k0 = host(k0)
    for i in range(n):
        r0, _ = ol.myl7_gen(prg, native.GROUP_ADD, 64, int(alphas[i]), pay[i].tobytes(), seeds[i])
        assert k0[i].tobytes() == r0.tobytes(), i


@pytest.mark.parametrize("group", [native.GROUP_XOR, native.GROUP_ADD])
# (7, 16) and (13, 16): cw_np1 ends the key at a non-word-aligned address.
@pytest.mark.parametrize("in_bits,plen", [(64, 1), (64, 16), (13, 2), (20, 20), (7, 16), (13, 16)])
def test_eval_matches_oracle(group, in_bits, plen):
    state = _state(21)
    prg = ol.Prg(state)
    n = 1000
    rng = np.random.default_rng(in_bits + 7 * plen + group)
    mask = (1 << in_bits) - 1
    alphas = np.array([int(v) & mask for v in rng.integers(0, 2**63, size=n)], dtype=np.uint64)
    chunks = (plen + 15) // 16
    seeds = rng.integers(0, 256, size=(n, chunks * 32), dtype=np.uint8)
    payload = rng.integers(0, 256, size=plen, dtype=np.uint8)
    payload[0] |= 1
    say("dcf_eval vs oracle group=%d in_bits=%d plen=%d" % (group, in_bits, plen))
    k0, k1 = pfss.dcf_gen(group, in_bits, state, dev(alphas), dev(payload), dev(seeds))
    delta = rng.integers(-3, 4, size=n)
    xs = np.array([(int(a) + int(d)) & mask for a, d in zip(alphas, delta)], dtype=np.uint64)
    xs[::5] = [int(v) & mask for v in rng.integers(0, 2**63, size=len(xs[::5]))]
    xd = dev(xs)
    outs = {}
    for p, keys in ((0, k0), (1, k1)):
        outs[p] = host(pfss.dcf_eval(group, in_bits, plen, state, keys, xd, native.DCF_OUT_BYTES,
                                     out_bytes=plen)).reshape(n, plen)
        bits = host(pfss.dcf_eval(group, in_bits, plen, state, keys, xd, native.DCF_OUT_BIT))
        packed = u64(pfss.dcf_eval(group, in_bits, plen, state, keys, xd,
                                   native.DCF_OUT_PACKED))
        kh = host(keys)
        for i in range(0, n, 7):
            ref = ol.myl7_eval(prg, group, in_bits, kh[i], int(xs[i]), plen)
            assert outs[p][i].tobytes() == ref.tobytes(), (p, i)
        assert np.array_equal(bits, outs[p][:, 0] & 1)
        unpacked = np.array([(int(packed[j // 64]) >> (j % 64)) & 1 for j in range(n)],
                            dtype=np.uint8)
        assert np.array_equal(unpacked, bits)
    # Reconstruction closed form.
    lt = np.array([int(x) < int(a) for x, a in zip(xs, alphas)])
    if group == native.GROUP_XOR:
        rec = outs[0] ^ outs[1]
        p = payload.copy()
        if plen >= 16:
            p[15] &= 0x7F
        exp = np.where(lt[:, None], p[None, :], 0).astype(np.uint8)
        assert np.array_equal(rec, exp)
    else:
        b0 = (outs[0][:, 0].astype(np.int64) + outs[1][:, 0].astype(np.int64)) & 0xFF
        assert np.array_equal(b0, np.where(lt, payload[0], 0))


def test_eval_first_chunks_only():
    """out_bytes < payload_len evaluates only the chunks it needs."""
    state = _state(4)
    n, plen = 70, 40
    rng = np.random.default_rng(8)
    alphas = rng.integers(0, 2**63, size=n).astype(np.uint64)
    seeds = rng.integers(0, 256, size=(n, 3 * 32), dtype=np.uint8)
    payload = rng.integers(0, 256, size=plen, dtype=np.uint8)
    say("dcf_eval partial chunks")
    k0, _ = pfss.dcf_gen(native.GROUP_XOR, 64, state, dev(alphas), dev(payload), dev(seeds))
    xs = dev(rng.integers(0, 2**63, size=n).astype(np.uint64))
    full = host(pfss.dcf_eval(native.GROUP_XOR, 64, plen, state, k0, xs, native.DCF_OUT_BYTES,
                              out_bytes=plen)).reshape(n, plen)
    for ob in (1, 16, 17, 33):
        part = host(pfss.dcf_eval(native.GROUP_XOR, 64, plen, state, k0, xs,
                                  native.DCF_OUT_BYTES, out_bytes=ob)).reshape(n, ob)
        assert np.array_equal(part, full[:, :ob])


def test_empty_and_ragged_batches():
    state = _state(2)
    rng = np.random.default_rng(1)
    for n in (1, 63, 64, 65, 257):
        say("dcf ragged n=%d" % n)
        alphas = rng.integers(0, 2**63, size=n).astype(np.uint64)
        seeds = rng.integers(0, 256, size=(n, 32), dtype=np.uint8)
        k0, k1 = pfss.dcf_gen(native.GROUP_XOR, 64, state, dev(alphas),
                              dev(np.array([1], dtype=np.uint8)), dev(seeds))
        xs = rng.integers(0, 2**63, size=n).astype(np.uint64)
        xd = dev(xs)
        w0 = u64(pfss.dcf_eval(0, 64, 1, state, k0, xd, native.DCF_OUT_PACKED))
        w1 = u64(pfss.dcf_eval(0, 64, 1, state, k1, xd, native.DCF_OUT_PACKED))
        rec = w0 ^ w1
        exp = np.zeros_like(rec)
        for j in range(n):
            if int(xs[j]) < int(alphas[j]):
                exp[j // 64] |= np.uint64(1 << (j % 64))
        assert np.array_equal(rec, exp)
    # n == 0 is a no-op
    out = torch.zeros(4, dtype=torch.uint8, device="cuda")
    native.call("sufhip_dcf_eval", 0, 64, 1, pfss._state_buf(state), None, 2152, 0, None, 0, 0, 1,
                out.data_ptr(), None)


def test_full_size_batch_reconstructs():
    """N = 2^20 keys over Z_2^64 (one chunk, 1-byte payload): keygen, eval for
    both parties, XOR-reconstruct and compare with 1[xhat < r_in]."""
    n = 1 << 20
    say("dcf full-size N=2^20")
    state = _state(3)
    r_in = pfss.host_mt19937_64(1, n)
    x = pfss.host_normal_fixed(2, 1.0, 0.0, 12, n)
    xhat = (x + r_in).astype(np.uint64)
    seeds_w = pfss.host_mt19937_64(4, n * 4)
    seeds = seeds_w.view(np.uint8).reshape(n, 32)
    k0, k1 = pfss.dcf_gen(native.GROUP_XOR, 64, state, dev(r_in),
                          dev(np.array([1], dtype=np.uint8)), dev(seeds))
    xd = dev(xhat)
    b0 = pfss.dcf_eval(0, 64, 1, state, k0, xd, native.DCF_OUT_BIT)
    b1 = pfss.dcf_eval(0, 64, 1, state, k1, xd, native.DCF_OUT_BIT)
    rec = host(b0 ^ b1)
    exp = (xhat < r_in).astype(np.uint8)
    assert np.array_equal(rec, exp)
    # spot-check shares against the oracle
    prg = ol.Prg(state)
    k0h = host(k0[:: n // 16])
    for j, i in enumerate(range(0, n, n // 16)):
        ref = ol.myl7_eval(prg, 0, 64, k0h[j], int(xhat[i]), 1)[0] & 1
        assert int(host(b0[i:i + 1])[0]) == ref


@pytest.mark.parametrize("mode", ["bit", "packed"])
def test_multi_pass_ragged_batch(mode):
    """More keys than one grid-stride pass of the bit-mode kernel covers (1024
    lanes on each of 256 CUs), ending in a partial wave: both parties' bits
    XOR to 1[x < alpha], and equal bit 0 of the full-share (bytes) walk."""
    n = 256 * 1024 + 1000 + 37
    say("dcf multi-pass ragged n=%d mode=%s" % (n, mode))
    state = _state(5)
    rng = np.random.default_rng(9)
    alphas = rng.integers(0, 2**63, size=n).astype(np.uint64) * np.uint64(2)
    seeds = rng.integers(0, 256, size=(n, 32), dtype=np.uint8)
    k0, k1 = pfss.dcf_gen(native.GROUP_XOR, 64, state, dev(alphas),
                          dev(np.array([1], dtype=np.uint8)), dev(seeds))
    xs = (alphas.astype(object) + rng.integers(-2, 3, size=n).astype(object))
    xs = np.array([int(v) % (1 << 64) for v in xs], dtype=np.uint64)
    xd = dev(xs)
    got = []
    for keys in (k0, k1):
        out = pfss.dcf_eval(0, 64, 1, state, keys, xd, MODES[mode])
        if mode == "packed":
            w = u64(out)
            bits = ((w[np.arange(n) // 64] >> (np.arange(n) % 64).astype(np.uint64)) & np.uint64(1))
            bits = bits.astype(np.uint8)
        else:
            bits = host(out)[:n]
        full = host(pfss.dcf_eval(0, 64, 1, state, keys, xd, native.DCF_OUT_BYTES, out_bytes=1))
        assert np.array_equal(bits, full.reshape(-1)[:n] & 1)
        got.append(bits)
    assert np.array_equal(got[0] ^ got[1], (xs < alphas).astype(np.uint8))


def test_bytes_multi_pass_additive_group():
    """The full-share walk over several grid-stride passes (1024 lanes on each
    of 256 CUs) in the additive group with an 8-byte payload: byte 0 of the
    two shares sums to payload[0] exactly where x < alpha, and the shares at
    indices around every pass boundary equal the oracle's."""
    n = 2 * 256 * 1024 + 517
    plen = 8
    say("dcf bytes multi-pass additive n=%d" % n)
    state = _state(8)
    prg = ol.Prg(state)
    rng = np.random.default_rng(13)
    alphas = rng.integers(0, 2**63, size=n).astype(np.uint64) * np.uint64(2)
    seeds = rng.integers(0, 256, size=(n, 32), dtype=np.uint8)
    payload = rng.integers(1, 256, size=plen, dtype=np.uint8)
    k0, k1 = pfss.dcf_gen(native.GROUP_ADD, 64, state, dev(alphas), dev(payload), dev(seeds))
    xs = np.array([(int(a) + int(d)) % (1 << 64) for a, d in
                   zip(alphas, rng.integers(-2, 3, size=n))], dtype=np.uint64)
    xd = dev(xs)
    outs = [host(pfss.dcf_eval(native.GROUP_ADD, 64, plen, state, keys, xd, native.DCF_OUT_BYTES,
                               out_bytes=plen)).reshape(n, plen) for keys in (k0, k1)]
    b0 = (outs[0][:, 0].astype(np.int64) + outs[1][:, 0].astype(np.int64)) & 0xFF
    assert np.array_equal(b0, np.where(xs < alphas, int(payload[0]), 0))
    stride = 256 * 1024
    idx = sorted({0, 1, stride - 1, stride, stride + 1, 2 * stride - 1, 2 * stride, n - 1} |
                 set(range(0, n, 9973)))
    for p, keys in ((0, k0), (1, k1)):
        kh = host(keys[torch.tensor(idx, device="cuda")])
        for j, i in enumerate(idx):
            ref = ol.myl7_eval(prg, native.GROUP_ADD, 64, kh[j], int(xs[i]), plen)
            assert outs[p][i].tobytes() == ref.tobytes(), (p, i)
