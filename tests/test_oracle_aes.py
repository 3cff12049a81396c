"""Pins the oracle's AES-128 and mt19937_64 (CPU only).

AES-128 is checked against FIPS-197 Appendix B and C.1 and against the
system OpenSSL libcrypto (the library the reference links for its PRG,
third_party/myl7_fss/src/prg/aes128_mmo.c:16-52, and for its CTR test,
src/demo/test_cuda_prg.cpp:23-34).  The CTR layout (le64(ctr) || le64(hi))
follows cuda/pfss_kernels.cu:169-184.
"""
import ctypes
import ctypes.util

import numpy as np
import pytest

import oracle_lib as ol


def test_fips197_appendix_c1():
    key = bytes(range(16))
    pt = bytes.fromhex("00112233445566778899aabbccddeeff")
    assert ol.aes_encrypt(key, pt).hex() == "69c4e0d86a7b0430d8cdb78070b4c55a"


def test_fips197_appendix_b():
    key = bytes.fromhex("2b7e151628aed2a6abf7158809cf4f3c")
    pt = bytes.fromhex("3243f6a8885a308d313198a2e0370734")
    assert ol.aes_encrypt(key, pt).hex() == "3925841d02dc09fbdc118597196a0b32"


def test_key_expansion_fips197_a1():
    rk = ol.aes_expand(bytes.fromhex("2b7e151628aed2a6abf7158809cf4f3c"))
    # w[43] of FIPS-197 Appendix A.1
    assert rk[172:176].tobytes().hex() == "b6630ca6"
    # w[4]
    assert rk[16:20].tobytes().hex() == "a0fafe17"


def _openssl():
    name = ctypes.util.find_library("crypto")
    if not name:
        pytest.skip("libcrypto not found")
    lib = ctypes.CDLL(name)
    if not hasattr(lib, "AES_set_encrypt_key"):
        pytest.skip("libcrypto lacks the AES_* API")
    return lib


def test_ctr_matches_openssl():
    lib = _openssl()
    key = ol.mt64_bytes(12345, 16)  # seed of test_cuda_prg.cpp:25-26
    aes_key = ctypes.create_string_buffer(512)
    assert lib.AES_set_encrypt_key(key.ctypes.data_as(ol.u8p), 128, aes_key) == 0
    blocks = 1024
    rk = ol.aes_expand(key.tobytes())
    out = np.zeros(blocks * 16, dtype=np.uint8)
    ol.LIB.orc_aes128_ctr(ol.ptr(rk), 7, 0x1122334455667788, blocks, ol.ptr(out))
    for i in range(blocks):
        blk = (7 + i).to_bytes(8, "little") + (0x1122334455667788).to_bytes(8, "little")
        ref = ctypes.create_string_buffer(16)
        lib.AES_encrypt(blk, ref, aes_key)
        assert ref.raw == out[16 * i:16 * i + 16].tobytes(), i


def test_mt19937_64_standard_value():
    # [rand.predef]: the 10000th consecutive invocation of a default-constructed
    # std::mt19937_64 (seed 5489) produces 9981545732273789042.
    assert int(ol.mt64(5489, 10000)[-1]) == 9981545732273789042


def test_aes_ni_path_matches_fips_restatement():
    """The oracle's AES-instruction path gives the FIPS-197 restatement's
    bytes: the appendix vectors and 2000 random (key, block) pairs."""
    if not ol.aes_ni_available():
        pytest.skip("CPU without AES instructions: the oracle uses the FIPS restatement")
    prev = ol.aes_use_ni(True)
    try:
        assert ol.aes_encrypt_fast(bytes(range(16)),
                                   bytes.fromhex("00112233445566778899aabbccddeeff")).hex() == \
            "69c4e0d86a7b0430d8cdb78070b4c55a"
        g = np.random.default_rng(11)
        for _ in range(2000):
            key = g.integers(0, 256, 16, dtype=np.uint8).tobytes()
            blk = g.integers(0, 256, 16, dtype=np.uint8).tobytes()
            assert ol.aes_encrypt_fast(key, blk) == ol.aes_encrypt(key, blk)
    finally:
        ol.aes_use_ni(prev)


def test_prg_and_dcf_same_with_and_without_aes_ni():
    """myl7 PRG blocks and DCF shares are the same bytes on either AES path,
    and the oracle's threaded loops give the single-thread result."""
    if not ol.aes_ni_available():
        pytest.skip("CPU without AES instructions")
    state = ol.mt64_bytes(3, ol.PRG_STATE_BYTES).tobytes()
    prg = ol.Prg(state)
    g = np.random.default_rng(12)
    n = 300
    alphas = g.integers(0, 2**64, n, dtype=np.uint64)
    seeds = g.integers(0, 256, (n, 32), dtype=np.uint8)
    k0, k1 = ol.myl7_gen_batch(prg, ol.GROUP_XOR, 64, alphas, b"\x01", seeds)
    xs = (alphas + g.integers(-3, 4, n).astype(np.uint64)).astype(np.uint64)
    rnd = g.integers(0, 2**64, ol.TRUNC_RAND_WORDS, dtype=np.uint64)
    res = []
    prev = ol.aes_use_ni(True)
    try:
        for ni, threads in ((False, 1), (True, 1), (True, 4)):
            ol.aes_use_ni(ni)
            ol.set_threads(threads)
            res.append([ol.myl7_eval_many_bit(prg, ol.GROUP_XOR, 64, k, xs, threads=threads)
                        for k in (k0, k1)])
            tk = ol.trunc_gen(prg, ol.TRUNC_GAPARS, 12, rnd)
            res[-1].append(ol.trunc_eval(prg, ol.TRUNC_GAPARS, 12, tk[0], xs))
    finally:
        ol.aes_use_ni(prev)
        ol.set_threads(0)
    for r in res[1:]:
        for a, b in zip(res[0], r):
            assert np.array_equal(a, b)
    assert np.array_equal(res[0][0] ^ res[0][1], (xs < alphas).astype(np.uint8))
