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
