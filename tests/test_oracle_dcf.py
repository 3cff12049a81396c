"""Pins the oracle's myl7 DCF (CPU only).

1. Byte parity with the reference's own myl7 code (third_party/myl7_fss/src/
   dcf.c, prg/aes128_mmo.c, group/{bytes,u128_le}.c and the SUF adapter
   include/proto/myl7_fss_backend.hpp), compiled unmodified into oracle/_ref
   by oracle/build_ref.sh.  Skipped where that build is absent (the GPU box);
   the committed golden vectors in tests/golden cover that case.
2. The closed form: share0 (+) share1 == beta * 1[x < alpha], brute force over
   every x of an 8-bit domain (test_myl7_bit_order.cpp:27-31), plus the
   alpha-2..alpha+2 band at 16 and 64 bits.
"""
import numpy as np
import pytest

import oracle_lib as ol

GROUPS = [ol.GROUP_XOR, ol.GROUP_ADD]


def _prg(seed):
    return ol.Prg(ol.mt64_bytes(seed, ol.PRG_STATE_BYTES).tobytes())


def _recon(group, a, b):
    a = bytearray(a)
    b = bytearray(b)
    if group == ol.GROUP_XOR:
        return bytes(x ^ y for x, y in zip(a, b))
    n = len(a)
    s = (int.from_bytes(a, "little") + int.from_bytes(b, "little")) % (1 << (8 * n))
    return s.to_bytes(n, "little")


@pytest.mark.parametrize("group", GROUPS)
@pytest.mark.parametrize("in_bits", [8])
def test_brute_force_closed_form(group, in_bits):
    prg = _prg(3)
    rng = np.random.default_rng(11)
    payload = bytes([0x5A, 0x01, 0x77])
    for alpha in [0, 1, 2, 77, 128, 254, 255]:
        seeds = rng.integers(0, 256, size=32, dtype=np.uint8)
        k0, k1 = ol.myl7_gen(prg, group, in_bits, alpha, payload, seeds)
        for x in range(1 << in_bits):
            o0 = ol.myl7_eval(prg, group, in_bits, k0, x, len(payload))
            o1 = ol.myl7_eval(prg, group, in_bits, k1, x, len(payload))
            expect = payload if x < alpha else bytes(len(payload))
            assert _recon(group, o0.tobytes(), o1.tobytes()) == expect, (alpha, x)


@pytest.mark.parametrize("group", GROUPS)
@pytest.mark.parametrize("in_bits", [16, 64])
def test_band_closed_form(group, in_bits):
    prg = _prg(5)
    rng = np.random.default_rng(in_bits)
    mask = (1 << in_bits) - 1
    payload = (0x0123456789ABCDEF).to_bytes(8, "little") + bytes(range(9))  # two chunks
    for trial in range(6):
        alpha = int(rng.integers(0, 2**63)) * 2 + int(rng.integers(0, 2))
        alpha &= mask
        seeds = rng.integers(0, 256, size=64, dtype=np.uint8)
        k0, k1 = ol.myl7_gen(prg, group, in_bits, alpha, payload, seeds)
        pts = [(alpha + d) & mask for d in range(-2, 3)] + [0, mask]
        for x in pts:
            o0 = ol.myl7_eval(prg, group, in_bits, k0, x, len(payload))
            o1 = ol.myl7_eval(prg, group, in_bits, k1, x, len(payload))
            p = bytearray(payload)
            p[15] &= 0x7F  # beta's MSB is cleared (myl7_fss_backend.hpp:180)
            expect = bytes(p) if x < alpha else bytes(len(payload))
            if group == ol.GROUP_ADD:
                # Each 16-byte chunk reconstructs mod 2^127; compare chunk-wise.
                got = b""
                for c in range(0, len(payload), 16):
                    s = (int.from_bytes(o0[c:c + 16].tobytes(), "little") +
                         int.from_bytes(o1[c:c + 16].tobytes(), "little")) % (1 << 127)
                    got += s.to_bytes(16, "little")[:len(payload) - c]
                assert got == expect, (trial, x)
            else:
                assert _recon(group, o0.tobytes(), o1.tobytes()) == expect, (trial, x)


def test_key_layout():
    prg = _prg(1)
    seeds = np.arange(32, dtype=np.uint8)
    k0, k1 = ol.myl7_gen(prg, ol.GROUP_XOR, 64, 12345, b"\x01", seeds)
    assert len(k0) == 2152  # 8 + 16 + 64*33 + 16
    assert list(k0[:8]) == [64, 1, 0, 0, 1, 0, 0, 0]
    assert list(k1[:8]) == [64, 1, 1, 0, 1, 0, 0, 0]
    assert k0[8:24].tobytes() == bytes(range(16))
    assert k1[8:24].tobytes() == bytes(range(16, 32))
    assert k0[24:].tobytes() == k1[24:].tobytes()


# ---------------- parity with the reference build ----------------
needs_ref = pytest.mark.skipif(not ol.ref_available(), reason="oracle/_ref not built")


@needs_ref
@pytest.mark.parametrize("group", GROUPS)
@pytest.mark.parametrize("bitlen", [1, 7, 16, 33, 64])
def test_gen_eval_bytes_match_reference(group, bitlen):
    import ctypes

    ref = ol.ref_lib(group)
    state = ol.mt64_bytes(3 + bitlen, ol.PRG_STATE_BYTES)
    ref.ref_prg_init(ol.ptr(state), ol.PRG_STATE_BYTES)
    prg = ol.Prg(state.tobytes())
    rng = np.random.default_rng(bitlen * 7 + group)
    nb = (bitlen + 7) // 8
    for trial in range(4):
        alpha = rng.integers(0, 256, size=nb, dtype=np.uint8)
        if bitlen % 8:
            alpha[-1] &= (1 << (bitlen % 8)) - 1
        beta = rng.integers(0, 256, size=16, dtype=np.uint8)
        s0 = rng.integers(0, 256, size=16, dtype=np.uint8)
        s1 = rng.integers(0, 256, size=16, dtype=np.uint8)
        cws_r = np.zeros(bitlen * 33, dtype=np.uint8)
        np1_r = np.zeros(16, dtype=np.uint8)
        ref.ref_dcf_gen(bitlen, ol.ptr(alpha), ol.ptr(beta), ol.ptr(s0.copy()), ol.ptr(s1.copy()),
                        ol.ptr(cws_r), ol.ptr(np1_r))
        cws_o = np.zeros(bitlen * 33, dtype=np.uint8)
        np1_o = np.zeros(16, dtype=np.uint8)
        ol.LIB.orc_dcf_gen(prg.buf, group, bitlen, ol.ptr(alpha), ol.ptr(beta), ol.ptr(s0),
                           ol.ptr(s1), ol.ptr(cws_o), ol.ptr(np1_o))
        assert cws_o.tobytes() == cws_r.tobytes()
        assert np1_o.tobytes() == np1_r.tobytes()
        for _ in range(8):
            x = rng.integers(0, 256, size=nb, dtype=np.uint8)
            for party, seed in ((0, s0), (1, s1)):
                out_r = np.zeros(16, dtype=np.uint8)
                out_o = np.zeros(16, dtype=np.uint8)
                ref.ref_dcf_eval(party, bitlen, ol.ptr(x), ol.ptr(seed), ol.ptr(cws_r),
                                 ol.ptr(np1_r), ol.ptr(out_r))
                ol.LIB.orc_dcf_eval(prg.buf, group, party, bitlen, ol.ptr(x), ol.ptr(seed),
                                    ol.ptr(cws_o), ol.ptr(np1_o), ol.ptr(out_o))
                assert out_o.tobytes() == out_r.tobytes(), (trial, party)
    del ctypes


@needs_ref
@pytest.mark.parametrize("group", GROUPS)
def test_adapter_blob_and_batch_match_reference(group):
    ref = ol.ref_lib(group)
    state = ol.mt64_bytes(31, ol.PRG_STATE_BYTES)
    ref.ref_prg_init(ol.ptr(state), ol.PRG_STATE_BYTES)
    prg = ol.Prg(state.tobytes())
    rng = np.random.default_rng(99)
    for in_bits, plen in [(64, 1), (16, 8), (12, 20)]:
        mask = (1 << in_bits) - 1
        # Keys from the reference adapter itself (seeds from random_device).
        kb = ol.myl7_key_bytes(in_bits, plen)
        payload = rng.integers(0, 256, size=plen, dtype=np.uint8)
        payload[0] |= 1
        alphas = [int(rng.integers(0, 2**62)) & mask for _ in range(6)]
        keys0 = np.zeros((len(alphas), kb), dtype=np.uint8)
        keys1 = np.zeros((len(alphas), kb), dtype=np.uint8)
        for i, a in enumerate(alphas):
            n = ref.ref_adapter_gen(in_bits, a, ol.ptr(payload), plen, ol.ptr(keys0[i]),
                                    ol.ptr(keys1[i]), kb)
            assert n == kb
        xs = np.array([(a + d) & mask for a in alphas for d in (-1, 0, 1)], dtype=np.uint64)
        kidx = np.repeat(np.arange(len(alphas)), 3)
        for keys in (keys0, keys1):
            flat = np.ascontiguousarray(keys[kidx])
            out_r = np.zeros(len(xs), dtype=np.uint8)
            assert ref.ref_adapter_eval_many(in_bits, kb, ol.ptr(flat), ol.ptr(xs, ol.u64p),
                                             len(xs), 1, ol.ptr(out_r)) == 0
            out_o = ol.myl7_eval_many_bit(prg, group, in_bits, flat, xs)
            assert out_o.tobytes() == out_r.tobytes()
            for j in range(len(xs)):
                full_r = np.zeros(64, dtype=np.uint8)
                m = ref.ref_adapter_eval(in_bits, ol.ptr(flat[j]), kb, int(xs[j]),
                                         ol.ptr(full_r), 64)
                assert m == plen
                full_o = ol.myl7_eval(prg, group, in_bits, flat[j], int(xs[j]), plen)
                assert full_o.tobytes() == full_r[:plen].tobytes()
        # XOR group: bit 0 reconstructs 1[x < alpha] since payload[0] is odd.
        if group == ol.GROUP_XOR:
            b0 = ol.myl7_eval_many_bit(prg, group, in_bits, np.ascontiguousarray(keys0[kidx]), xs)
            b1 = ol.myl7_eval_many_bit(prg, group, in_bits, np.ascontiguousarray(keys1[kidx]), xs)
            expect = np.array([int(x) < alphas[k] for x, k in zip(xs, kidx)], dtype=np.uint8)
            assert np.array_equal(b0 ^ b1, expect)
