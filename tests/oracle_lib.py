"""ctypes bindings for the CPU oracle (oracle/_build/liboracle.so) and, when it
was built, the reference's own myl7 DCF (oracle/_ref/libmyl7ref_*.so).

Test infrastructure only: the product package never imports this module.
"""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "_build", "liboracle.so")
REF_DIR = os.path.join(ORACLE_DIR, "_ref")

u8p = ctypes.POINTER(ctypes.c_uint8)
u64p = ctypes.POINTER(ctypes.c_uint64)
i32p = ctypes.POINTER(ctypes.c_int)
c_sz = ctypes.c_size_t

GROUP_XOR = 0
GROUP_ADD = 1
PRG_STATE_BYTES = 128  # kBlocks (8) x lambda (16)


def ptr(a, t=u8p):
    if a is None:
        return None
    return a.ctypes.data_as(t)


def _load_oracle():
    if not os.path.exists(ORACLE_SO):
        subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)
    lib = ctypes.CDLL(ORACLE_SO)
    lib.orc_myl7_key_bytes.restype = c_sz
    lib.orc_packed_key_bytes.restype = c_sz
    lib.orc_lut_key_bytes.restype = c_sz
    lib.orc_mt64_next.restype = ctypes.c_uint64
    lib.orc_beaver_scale.restype = ctypes.c_uint64
    lib.orc_beaver_scale.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int64, ctypes.c_int]
    lib.orc_myl7_gen.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_uint64,
                                 u8p, ctypes.c_int, u8p, u8p, u8p]
    lib.orc_myl7_eval.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, u8p,
                                  ctypes.c_uint64, u8p]
    lib.orc_myl7_eval_many_bit.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, c_sz,
                                           u8p, u64p, c_sz, u8p, ctypes.c_int]
    lib.orc_seed_from_id.argtypes = [ctypes.c_uint64, ctypes.c_uint64, u8p]
    lib.orc_mt64_fill.argtypes = [ctypes.c_uint64, u64p, c_sz]
    lib.orc_aes128_ctr.argtypes = [u8p, ctypes.c_uint64, ctypes.c_uint64, c_sz, u8p]
    lib.orc_packed_build_key.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_int, u64p,
                                         ctypes.c_int, u8p, u8p]
    lib.orc_packed_eval.argtypes = [u8p, c_sz, ctypes.c_int, u64p, c_sz, u64p]
    lib.orc_lut_build_key.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_int, ctypes.c_int,
                                      u64p, ctypes.c_int, u64p, u8p, u8p]
    lib.orc_lut_eval.argtypes = [u8p, c_sz, ctypes.c_int, u64p, c_sz, u64p]
    lib.orc_lut_eval_at.argtypes = [u8p, c_sz, ctypes.c_int, u64p, c_sz, c_sz, u64p]
    lib.orc_trunc_postproc.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_uint64,
                                       ctypes.c_uint64, u64p, u64p, c_sz, ctypes.c_int, u64p,
                                       c_sz, ctypes.c_int, ctypes.c_int, ctypes.c_int, u64p, c_sz]
    lib.orc_beaver_matmul.argtypes = [ctypes.c_int, u64p, u64p, u64p, u64p, u64p, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int64, ctypes.c_int, u64p,
                                      ctypes.c_int]
    lib.orc_aes_use_ni.argtypes = [ctypes.c_int]
    lib.orc_set_threads.argtypes = [ctypes.c_int]
    lib.orc_aes128_encrypt_fast.argtypes = [u8p, u8p, u8p]
    lib.orc_matmul_public.argtypes = [u64p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, u64p]
    lib.orc_add_rout_aos.argtypes = [u64p, c_sz, ctypes.c_int, u64p, ctypes.c_int]
    lib.orc_open_add.argtypes = [u64p, u64p, ctypes.c_int, u64p, c_sz, ctypes.c_int,
                                 ctypes.c_uint64, ctypes.c_int]
    lib.orc_trunc_key_bytes.restype = c_sz
    lib.orc_trunc_key_bytes.argtypes = [ctypes.c_int, ctypes.c_int]
    lib.orc_trunc_gen.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, u64p, u8p, u8p]
    lib.orc_trunc_eval.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, u8p, u64p, c_sz,
                                   u64p]
    return lib


LIB = _load_oracle()


class Prg:
    """myl7 PRG state: eight AES-128 keys taken from a 128-byte state."""

    def __init__(self, state: bytes):
        assert len(state) == PRG_STATE_BYTES
        self.state = bytes(state)
        self.buf = ctypes.create_string_buffer(8 * 176)
        st = np.frombuffer(self.state, dtype=np.uint8).copy()
        LIB.orc_prg_init(self.buf, ptr(st), PRG_STATE_BYTES)


def mt64(seed, n):
    out = np.empty(n, dtype=np.uint64)
    LIB.orc_mt64_fill(seed, ptr(out, u64p), n)
    return out


def mt64_bytes(seed, n):
    """n bytes, each the low byte of one mt19937_64 output."""
    return (mt64(seed, n) & np.uint64(0xFF)).astype(np.uint8)


def aes_expand(key: bytes) -> np.ndarray:
    rk = np.zeros(176, dtype=np.uint8)
    k = np.frombuffer(bytes(key), dtype=np.uint8).copy()
    LIB.orc_aes128_expand(ptr(k), ptr(rk))
    return rk


def aes_encrypt(key: bytes, block: bytes) -> bytes:
    rk = aes_expand(key)
    b = np.frombuffer(bytes(block), dtype=np.uint8).copy()
    out = np.zeros(16, dtype=np.uint8)
    LIB.orc_aes128_encrypt(ptr(rk), ptr(b), ptr(out))
    return out.tobytes()


def aes_encrypt_fast(key: bytes, block: bytes) -> bytes:
    """The AES-NI path (or the FIPS restatement when it is off)."""
    rk = aes_expand(key)
    inp = np.frombuffer(block, dtype=np.uint8).copy()
    out = np.zeros(16, dtype=np.uint8)
    LIB.orc_aes128_encrypt_fast(ptr(rk), ptr(inp), ptr(out))
    return out.tobytes()


def aes_use_ni(on):
    """Selects the oracle's AES: the x86 AES instructions (when the CPU has
    them) or the FIPS-197 restatement.  Returns the previous setting."""
    prev = LIB.orc_aes_ni_active()
    LIB.orc_aes_use_ni(1 if on else 0)
    return prev


def aes_ni_available():
    return bool(LIB.orc_aes_ni_available())


def set_threads(n):
    """OpenMP threads of the oracle's per-element loops (<= 0: all processors)."""
    LIB.orc_set_threads(int(n))


def get_threads():
    return int(LIB.orc_get_threads())


def matmul_public(X, W, M, K, N):
    """X [M x K] u64 share times public int64 W [K x N], mod 2^64."""
    X = np.ascontiguousarray(X, dtype=np.uint64)
    W = np.ascontiguousarray(W, dtype=np.int64)
    out = np.empty(M * N, dtype=np.uint64)
    LIB.orc_matmul_public(ptr(X, u64p), W.ctypes.data, M, K, N, ptr(out, u64p))
    return out


def myl7_key_bytes(in_bits, payload_len):
    return LIB.orc_myl7_key_bytes(in_bits, payload_len)


def myl7_gen(prg, group, in_bits, alpha, payload: bytes, seeds: np.ndarray):
    kb = myl7_key_bytes(in_bits, len(payload))
    k0 = np.zeros(kb, dtype=np.uint8)
    k1 = np.zeros(kb, dtype=np.uint8)
    p = np.frombuffer(bytes(payload), dtype=np.uint8).copy()
    rc = LIB.orc_myl7_gen(prg.buf, group, in_bits, int(alpha) & (2**64 - 1), ptr(p), len(payload),
                          ptr(np.ascontiguousarray(seeds, dtype=np.uint8)), ptr(k0), ptr(k1))
    assert rc == 0
    return k0, k1


def myl7_gen_batch(prg, group, in_bits, alphas, payload: bytes, seeds: np.ndarray):
    """seeds: [n][chunks*32] bytes. Returns (keys0 [n][kb], keys1 [n][kb])."""
    n = len(alphas)
    kb = myl7_key_bytes(in_bits, len(payload))
    k0 = np.zeros((n, kb), dtype=np.uint8)
    k1 = np.zeros((n, kb), dtype=np.uint8)
    for i in range(n):
        a, b = myl7_gen(prg, group, in_bits, int(alphas[i]), payload, seeds[i])
        k0[i] = a
        k1[i] = b
    return k0, k1


def myl7_eval(prg, group, in_bits, key: np.ndarray, x, payload_len):
    out = np.zeros(max(payload_len, 1), dtype=np.uint8)
    rc = LIB.orc_myl7_eval(prg.buf, group, in_bits, ptr(np.ascontiguousarray(key)),
                           int(x) & (2**64 - 1), ptr(out))
    assert rc == 0
    return out[:payload_len]


def myl7_eval_many_bit(prg, group, in_bits, keys: np.ndarray, xs: np.ndarray, threads=1):
    n = xs.shape[0]
    out = np.zeros(n, dtype=np.uint8)
    keys = np.ascontiguousarray(keys)
    rc = LIB.orc_myl7_eval_many_bit(prg.buf, group, in_bits, keys.shape[1], ptr(keys),
                                    ptr(np.ascontiguousarray(xs, dtype=np.uint64), u64p), n,
                                    ptr(out), threads)
    assert rc == 0
    return out


def seed_from_id(i, tweak):
    s = np.zeros(16, dtype=np.uint8)
    LIB.orc_seed_from_id(i, tweak, ptr(s))
    return s


def packed_key(party, nonce, in_bits, thr, seed):
    thr = np.ascontiguousarray(thr, dtype=np.uint64)
    blob = np.zeros(LIB.orc_packed_key_bytes(len(thr)), dtype=np.uint8)
    LIB.orc_packed_build_key(party, nonce, in_bits, ptr(thr, u64p), len(thr), ptr(seed), ptr(blob))
    return blob


def packed_eval(keys, key_bytes, broadcast, xs, out_words):
    xs = np.ascontiguousarray(xs, dtype=np.uint64)
    out = np.zeros(len(xs) * out_words, dtype=np.uint64)
    LIB.orc_packed_eval(ptr(np.ascontiguousarray(keys)), key_bytes, int(broadcast),
                        ptr(xs, u64p), len(xs), ptr(out, u64p))
    return out.reshape(len(xs), out_words)


def lut_key(party, nonce, in_bits, out_words, cuts, payload, seed):
    cuts = np.ascontiguousarray(cuts, dtype=np.uint64)
    payload = np.ascontiguousarray(payload, dtype=np.uint64).ravel()
    intervals = len(cuts) - 1
    blob = np.zeros(LIB.orc_lut_key_bytes(intervals, out_words), dtype=np.uint8)
    LIB.orc_lut_build_key(party, nonce, in_bits, out_words, ptr(cuts, u64p), intervals,
                          ptr(payload, u64p), ptr(seed), ptr(blob))
    return blob


def lut_eval(keys, key_bytes, broadcast, xs, out_words, idx0=0):
    """idx0: index of xs[0] in the batch (the keystream counter uses it)."""
    xs = np.ascontiguousarray(xs, dtype=np.uint64)
    out = np.zeros(len(xs) * out_words, dtype=np.uint64)
    LIB.orc_lut_eval_at(ptr(np.ascontiguousarray(keys)), key_bytes, int(broadcast),
                        ptr(xs, u64p), len(xs), idx0, ptr(out, u64p))
    return out.reshape(len(xs), out_words)


# ---------------- reference build (oracle/_ref) ----------------
def ref_available(group=GROUP_XOR):
    return os.path.exists(_ref_path(group))


def _ref_path(group):
    name = "libmyl7ref_bytes.so" if group == GROUP_XOR else "libmyl7ref_u128_le.so"
    return os.path.join(REF_DIR, name)


_REF = {}


def ref_lib(group=GROUP_XOR):
    if group not in _REF:
        lib = ctypes.CDLL(_ref_path(group), mode=ctypes.RTLD_LOCAL)
        lib.ref_adapter_eval.argtypes = [ctypes.c_int, u8p, c_sz, ctypes.c_uint64, u8p, c_sz]
        lib.ref_adapter_eval_many.argtypes = [ctypes.c_int, c_sz, u8p, u64p, c_sz, ctypes.c_int,
                                              u8p]
        lib.ref_adapter_gen.argtypes = [ctypes.c_int, ctypes.c_uint64, u8p, c_sz, u8p, u8p, c_sz]
        _REF[group] = lib
    return _REF[group]


# ---------------- ring postprocessing ----------------
def _u64(a):
    return np.ascontiguousarray(a, dtype=np.uint64)


def beaver_mul(party, a, b, c, d, e):
    out = np.zeros(len(a), dtype=np.uint64)
    LIB.orc_beaver_mul(party, *(ptr(_u64(v), u64p) for v in (a, b, c, d, e)), ptr(out, u64p),
                       c_sz(len(a)))
    return out


def trunc_postproc(party, gapars, f, r_hi, m, hatx, arith, arith_stride, arith_idx, bools,
                   bool_stride, carry_idx, sign_idx, wrap_idx, n):
    out = np.zeros(n, dtype=np.uint64)
    LIB.orc_trunc_postproc(party, gapars, f, int(r_hi), int(m),
                           ptr(_u64(hatx), u64p) if hatx is not None else None,
                           ptr(_u64(arith), u64p), arith_stride, arith_idx,
                           ptr(_u64(bools), u64p) if bools is not None else None, bool_stride,
                           carry_idx, sign_idx, wrap_idx, ptr(out, u64p), n)
    return out


def horner(x, c0, c1, c2, c3):
    out = np.zeros(len(x), dtype=np.uint64)
    LIB.orc_horner_cubic(*(ptr(_u64(v), u64p) for v in (x, c0, c1, c2, c3)), ptr(out, u64p),
                         c_sz(len(x)))
    return out


def add_rout_aos(out, elems, out_words, r_out):
    out = _u64(out).copy()
    r = _u64(r_out)
    LIB.orc_add_rout_aos(ptr(out, u64p), elems, out_words, ptr(r, u64p), len(r))
    return out


def row_broadcast_mul(party, A, B_rows, C, d, e_rows, rows, cols, valid_lens=None):
    out = np.zeros(rows * cols, dtype=np.uint64)
    vl = np.ascontiguousarray(valid_lens, dtype=np.int32) if valid_lens is not None else None
    LIB.orc_row_broadcast_mul(party, *(ptr(_u64(v), u64p) for v in (A, B_rows, C, d, e_rows)),
                              rows, cols, ptr(vl, i32p) if vl is not None else None,
                              ptr(out, u64p))
    return out


def _rows_call(fn, mat, rows, cols, valid_lens, *extra):
    out = np.zeros(rows, dtype=np.uint64)
    vl = np.ascontiguousarray(valid_lens, dtype=np.int32) if valid_lens is not None else None
    args = [ptr(_u64(mat), u64p)] + [ptr(_u64(e), u64p) for e in extra]
    fn(*args, rows, cols, ptr(vl, i32p) if vl is not None else None, ptr(out, u64p))
    return out


def row_sum(mat, rows, cols, valid_lens=None):
    return _rows_call(LIB.orc_row_sum, mat, rows, cols, valid_lens)


def row_mean(mat, rows, cols, valid_lens=None):
    return _rows_call(LIB.orc_row_mean, mat, rows, cols, valid_lens)


def row_variance(mat, mean, rows, cols, valid_lens=None):
    return _rows_call(LIB.orc_row_variance, mat, rows, cols, valid_lens, mean)


def row_sum_ragged(vals, offs):
    rows = len(offs) - 1
    out = np.zeros(rows, dtype=np.uint64)
    o = np.ascontiguousarray(offs, dtype=np.int32)
    LIB.orc_row_sum_ragged(ptr(_u64(vals), u64p), ptr(o, i32p), rows, ptr(out, u64p))
    return out


def pack_eff_bits(vals, eff_bits):
    n = len(vals)
    words = (n * eff_bits + 63) // 64
    out = np.zeros(max(words, 1), dtype=np.uint64)
    LIB.orc_pack_eff_bits(ptr(_u64(vals), u64p), eff_bits, ptr(out, u64p), c_sz(n))
    return out[:words]


def unpack_eff_bits(packed, eff_bits, n):
    out = np.zeros(n, dtype=np.uint64)
    LIB.orc_unpack_eff_bits(ptr(_u64(packed), u64p), eff_bits, ptr(out, u64p), c_sz(n))
    return out


def open_add(local, remote, eff_bits, n, ring_bits, ring_mask, sign_extend):
    out = np.zeros(n, dtype=np.uint64)
    LIB.orc_open_add(ptr(_u64(local), u64p), ptr(_u64(remote), u64p), eff_bits, ptr(out, u64p),
                     c_sz(n), ring_bits, ctypes.c_uint64(ring_mask), sign_extend)
    return out


def beaver_matmul(party, D, E, A, B, C, batches, M, K, N, w_t=0, has_scale=0, mul_const=0,
                  mul_shift=0, threads=0):
    out = np.zeros(batches * M * N, dtype=np.uint64)
    LIB.orc_beaver_matmul(party, *(ptr(_u64(v), u64p) for v in (D, E, A, B, C)), batches, M, K, N,
                          w_t, has_scale, mul_const, mul_shift, ptr(out, u64p), threads)
    return out


TRUNC_TR, TRUNC_ARS, TRUNC_GAPARS = 0, 1, 2
TRUNC_RAND_WORDS = 19


def trunc_key_bytes(kind, f):
    return LIB.orc_trunc_key_bytes(kind, f)


def trunc_gen(prg, kind, f, rnd):
    rnd = _u64(rnd)
    assert rnd.size == TRUNC_RAND_WORDS
    kb = trunc_key_bytes(kind, f)
    k0 = np.zeros(kb, dtype=np.uint8)
    k1 = np.zeros(kb, dtype=np.uint8)
    assert LIB.orc_trunc_gen(prg.buf, kind, f, ptr(rnd, u64p), ptr(k0), ptr(k1)) == 0
    return k0, k1


def trunc_eval(prg, kind, f, key, xhat):
    xhat = _u64(xhat)
    y = np.zeros(xhat.size, dtype=np.uint64)
    key = np.ascontiguousarray(key, dtype=np.uint8)
    assert LIB.orc_trunc_eval(prg.buf, kind, f, ptr(key), ptr(xhat, u64p), c_sz(xhat.size),
                              ptr(y, u64p)) == 0
    return y
