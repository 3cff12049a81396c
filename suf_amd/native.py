"""ctypes binding of libsuf_hip.so (the C ABI declared in include/suf_hip.h).

The library is loaded from suf_amd/lib/libsuf_hip.so, built in-tree by
`python -m suf_amd.build`.  There is no fallback: if the library is missing
or fails to load, every entry point raises.
"""
import ctypes
import os
import re

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "lib", "libsuf_hip.so")
HEADER = os.path.join(ROOT, "include", "suf_hip.h")

OK = 0
GROUP_XOR = 0
GROUP_ADD = 1
DCF_OUT_BIT = 0
DCF_OUT_BYTES = 1
DCF_OUT_PACKED = 2
TRUNC_TR = 0
TRUNC_ARS = 1
TRUNC_GAPARS = 2
TRUNC_RAND_WORDS = 19
CHAIN_CUBIC = 0
CHAIN_RECIP = 1
CHAIN_RSQRT = 2

c_int = ctypes.c_int
c_sz = ctypes.c_size_t
c_u64 = ctypes.c_uint64
c_i64 = ctypes.c_int64
c_dbl = ctypes.c_double
c_vp = ctypes.c_void_p
c_float = ctypes.c_float

# argtypes for every exported function; pointers travel as integers (void*).
_SIGS = {
    "sufhip_abi_version": (c_int, []),
    "sufhip_last_error": (ctypes.c_char_p, []),
    "sufhip_init": (c_int, [c_int]),
    "sufhip_set_keystream_per_party": (c_int, [c_int]),
    "sufhip_keystream_per_party": (c_int, []),
    "sufhip_device_count": (c_int, [c_vp]),
    "sufhip_stream_create": (c_int, [c_vp]),
    "sufhip_stream_destroy": (c_int, [c_vp]),
    "sufhip_stream_synchronize": (c_int, [c_vp]),
    "sufhip_malloc": (c_int, [c_vp, c_sz]),
    "sufhip_free": (c_int, [c_vp]),
    "sufhip_host_alloc": (c_int, [c_vp, c_sz]),
    "sufhip_host_free": (c_int, [c_vp]),
    "sufhip_memcpy_h2d": (c_int, [c_vp, c_vp, c_sz, c_vp]),
    "sufhip_memcpy_d2h": (c_int, [c_vp, c_vp, c_sz, c_vp]),
    "sufhip_memcpy_d2d": (c_int, [c_vp, c_vp, c_sz, c_vp]),
    "sufhip_event_create": (c_int, [c_vp]),
    "sufhip_event_destroy": (c_int, [c_vp]),
    "sufhip_event_record": (c_int, [c_vp, c_vp]),
    "sufhip_event_elapsed_ms": (c_int, [c_vp, c_vp, c_vp]),
    "sufhip_event_synchronize": (c_int, [c_vp]),
    "sufhip_aes128_ctr": (c_int, [c_vp, c_vp, c_u64, c_u64, c_sz, c_vp]),
    "sufhip_aes128_ctr_bitsliced": (c_int, [c_vp, c_vp, c_u64, c_u64, c_sz, c_vp]),
    "sufhip_prg_mmo": (c_int, [c_vp, c_vp, c_sz, c_int, c_vp, c_vp]),
    "sufhip_dcf_key_bytes": (c_sz, [c_int, c_int]),
    "sufhip_dcf_gen": (c_int, [c_int, c_int, c_vp, c_vp, c_vp, c_int, c_int, c_vp, c_sz, c_vp,
                               c_vp, c_vp]),
    "sufhip_dcf_eval": (c_int, [c_int, c_int, c_int, c_vp, c_vp, c_sz, c_int, c_vp, c_sz, c_int,
                                c_int, c_vp, c_vp]),
    "sufhip_trunc_key_bytes": (c_sz, [c_int, c_int]),
    "sufhip_trunc_gen": (c_int, [c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "sufhip_trunc_work_bytes": (c_sz, [c_int, c_sz]),
    "sufhip_trunc_eval": (c_int, [c_int, c_int, c_vp, c_vp, c_sz, c_vp, c_sz, c_vp, c_vp, c_sz,
                                  c_vp]),
    "sufhip_trunc_noalloc_max_work_bytes": (c_sz, []),
    "sufhip_trunc_eval_noalloc": (c_int, [c_int, c_int, c_vp, c_vp, c_sz, c_vp, c_sz, c_vp, c_vp]),
    "sufhip_trunc_prepare": (c_int, [c_int, c_int, c_vp, c_vp, c_sz, c_sz, c_vp, c_sz, c_vp]),
    "sufhip_stage_hatx": (c_int, [c_vp, c_int, c_vp, c_sz, c_vp]),
    "sufhip_open_flush2_work_bytes": (c_sz, [c_sz, c_int]),
    "sufhip_open_flush2": (c_int, [c_vp, c_int, c_int, c_int, c_int, c_vp, c_vp, c_sz, c_vp]),
    "sufhip_composite_bool_triples": (c_sz, [c_int, c_int]),
    "sufhip_composite_bool2": (c_int, [c_vp, c_vp]),
    "sufhip_trunc_finish": (c_int, [c_int, c_int, c_vp, c_vp, c_sz, c_vp, c_sz, c_vp, c_vp, c_sz,
                                    c_vp]),
    "sufhip_beaver_matmul2d_mfma_work_bytes": (c_sz, [c_int, c_int, c_int]),
    "sufhip_beaver_matmul2d_mfma": (c_int, [c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int,
                                            c_vp, c_vp, c_sz, c_vp]),
    "sufhip_open2_masked": (c_int, [c_vp, c_vp, c_u64, c_u64, c_sz, c_vp, c_vp]),
    "sufhip_open2_diff": (c_int, [c_vp, c_vp, c_vp, c_vp, c_sz, c_vp, c_vp]),
    "sufhip_mul2": (c_int, [c_vp, c_sz, c_vp]),
    "sufhip_add_shifted": (c_int, [c_vp, c_vp, c_sz, c_sz, c_int, c_sz, c_vp, c_vp]),
    "sufhip_lin2": (c_int, [c_vp, c_sz, c_vp, c_vp, c_vp, c_u64, c_vp, c_vp]),
    "sufhip_beaver_matmul2_batched_work_bytes": (c_sz, [c_int, c_int, c_int, c_int]),
    "sufhip_beaver_matmul2_batched": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                              c_int, c_int, c_int, c_int, c_vp, c_vp, c_vp, c_sz,
                                              c_vp]),
    "sufhip_kb_planes_bytes": (c_sz, [c_int, c_int, c_int]),
    "sufhip_beaver_matmul2_mfma_ex": (c_int, [c_vp, c_vp]),
    "sufhip_kb_split_batch": (c_int, [c_vp, c_int, c_vp]),
    "sufhip_kb_open_split_batch": (c_int, [c_vp, c_int, c_vp]),
    "sufhip_kb_open_split_prepare": (c_int, [c_vp, c_int, c_vp, c_vp, c_int, c_vp]),
    "sufhip_beaver_matmul2_mfma_batched": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                                   c_vp, c_int, c_int, c_int, c_int, c_vp, c_vp,
                                                   c_vp]),
    "sufhip_public_w_digits": (c_int, [c_vp, c_sz]),
    "sufhip_public_w_planes_bytes": (c_sz, [c_int, c_int, c_int]),
    "sufhip_public_w_prepare": (c_int, [c_vp, c_int, c_int, c_int, c_vp, c_vp]),
    "sufhip_matmul_public2_work_bytes": (c_sz, [c_int, c_int, c_int]),
    "sufhip_matmul_public2_planes": (c_int, [c_vp, c_int, c_int, c_int, c_vp, c_int, c_vp, c_vp,
                                             c_vp, c_u64, c_vp, c_vp, c_sz, c_vp]),
    "sufhip_matmul_public2_slices": (c_int, [c_int, c_int, c_int]),
    "sufhip_matmul_public2_planes_partial": (c_int, [c_vp, c_int, c_int, c_int, c_vp, c_int, c_vp,
                                                     c_sz, c_vp, c_vp]),
    "sufhip_matmul_public2_planes_qkv": (c_int, [c_vp, c_int, c_int, c_int, c_vp, c_int, c_u64,
                                                 c_vp, c_vp, c_vp, c_sz, c_vp]),
    "sufhip_matmul_public2": (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_vp, c_int, c_vp, c_vp,
                                      c_vp, c_u64, c_vp, c_vp, c_sz, c_vp]),
    "sufhip_trunc_finish2": (c_int, [c_int, c_int, c_vp, c_vp, c_vp, c_sz, c_vp, c_sz, c_vp, c_vp,
                                     c_vp, c_vp, c_sz, c_vp]),
    "sufhip_trunc_prepare_batch": (c_int, [c_vp, c_vp, c_int, c_vp]),
    "sufhip_mul2x": (c_int, [c_vp, c_sz, c_vp]),
    "sufhip_row_sum2": (c_int, [c_vp, c_int, c_int, c_vp, c_u64, c_vp, c_vp, c_vp, c_u64, c_vp,
                                c_vp]),
    "sufhip_interval_lut_eval2": (c_int, [c_vp, c_vp, c_sz, c_int, c_int, c_vp, c_vp, c_u64,
                                          c_sz, c_vp, c_vp, c_vp]),
    "sufhip_gate_chain2": (c_int, [c_vp, c_vp]),
    "sufhip_lin2_batch": (c_int, [c_vp, c_int, c_vp]),
    "sufhip_layernorm2": (c_int, [c_vp, c_vp]),
    "sufhip_softmax2": (c_int, [c_vp, c_vp]),
    "sufhip_relu_max_tree2": (c_int, [c_vp, c_vp, c_int, c_vp, c_int, c_int, c_vp, c_vp, c_vp,
                                      c_vp, c_vp]),
    "sufhip_relu_max_round2": (c_int, [c_vp, c_vp, c_sz, c_vp, c_vp, c_sz, c_vp, c_vp, c_sz, c_int,
                                       c_u64, c_vp, c_vp, c_vp]),
    "sufhip_seed_from_id": (None, [c_u64, c_u64, c_vp]),
    "sufhip_interval_lut_key_bytes": (c_sz, [c_int, c_int]),
    "sufhip_interval_lut_build_key": (c_int, [c_int, c_u64, c_int, c_int, c_vp, c_int, c_vp, c_vp,
                                              c_vp]),
    "sufhip_interval_lut_eval": (c_int, [c_vp, c_sz, c_int, c_int, c_int, c_vp, c_sz, c_vp,
                                         c_vp]),
    "sufhip_packed_lt_key_bytes": (c_sz, [c_int]),
    "sufhip_packed_lt_build_key": (c_int, [c_int, c_u64, c_int, c_vp, c_int, c_vp, c_vp]),
    "sufhip_packed_lt_eval": (c_int, [c_vp, c_sz, c_int, c_int, c_int, c_vp, c_sz, c_vp, c_vp]),
    "sufhip_beaver_mul": (c_int, [c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_sz,
                                  c_vp]),
    "sufhip_beaver_mul_aos": (c_int, [c_int, c_vp, c_vp, c_vp, c_vp, c_sz, c_vp]),
    "sufhip_trunc_shift": (c_int, [c_vp, c_vp, c_int, c_sz, c_vp]),
    "sufhip_trunc_postproc": (c_int, [c_int, c_int, c_int, c_u64, c_u64, c_vp, c_vp, c_sz, c_int,
                                      c_vp, c_sz, c_int, c_int, c_int, c_vp, c_sz, c_vp]),
    "sufhip_horner_cubic": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_sz, c_vp]),
    "sufhip_add_rout_aos": (c_int, [c_vp, c_sz, c_int, c_vp, c_sz, c_vp]),
    "sufhip_row_broadcast_mul": (c_int, [c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_vp,
                                         c_vp, c_sz, c_vp]),
    "sufhip_beaver_matmul2d": (c_int, [c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int,
                                       c_int, c_int, c_i64, c_int, c_vp, c_vp]),
    "sufhip_beaver_matmul2d_batched": (c_int, [c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int,
                                               c_int, c_int, c_int, c_int, c_i64, c_int, c_vp,
                                               c_vp]),
    "sufhip_row_sum": (c_int, [c_vp, c_int, c_int, c_vp, c_vp, c_vp]),
    "sufhip_row_sum_ragged": (c_int, [c_vp, c_vp, c_int, c_vp, c_vp]),
    "sufhip_row_mean": (c_int, [c_vp, c_int, c_int, c_vp, c_vp, c_vp]),
    "sufhip_row_variance": (c_int, [c_vp, c_vp, c_int, c_int, c_vp, c_vp, c_vp]),
    "sufhip_unpack_eff_bits": (c_int, [c_vp, c_int, c_vp, c_sz, c_vp]),
    "sufhip_pack_eff_bits": (c_int, [c_vp, c_int, c_vp, c_sz, c_vp]),
    "sufhip_open_add_to_signed": (c_int, [c_vp, c_vp, c_vp, c_sz, c_int, c_u64, c_vp]),
    "sufhip_unpack_add_to_signed": (c_int, [c_vp, c_vp, c_int, c_vp, c_sz, c_int, c_u64, c_vp]),
    "sufhip_unpack_add_mod": (c_int, [c_vp, c_vp, c_int, c_vp, c_sz, c_int, c_u64, c_vp]),
    "sufhip_host_mt19937_64": (c_int, [c_u64, c_vp, c_sz]),
    "sufhip_host_normal_fixed": (c_int, [c_u64, c_dbl, c_dbl, c_int, c_vp, c_sz]),
}

_lib = None


class Mul2Args(ctypes.Structure):
    """sufhip_mul2_args (include/suf_hip.h)."""
    _fields_ = [
        ("u", c_vp * 2), ("u_stride", c_sz), ("u_off", c_sz),
        ("u_add", c_vp * 2), ("u_add_stride", c_sz), ("u_add_off", c_sz), ("u_add_shift", c_int),
        ("v", c_vp * 2), ("triples", c_vp * 2),
        ("z_add", c_vp * 2), ("z_add_stride", c_sz), ("z_add_off", c_sz), ("z_add_shift", c_int),
        ("z", c_vp * 2), ("zhat", c_vp), ("open_mask", c_u64 * 2),
    ]


class Term2(ctypes.Structure):
    """sufhip_term2 (include/suf_hip.h)."""
    _fields_ = [("p", c_vp * 2), ("index", c_vp), ("len", c_sz), ("stride", c_sz),
                ("off", c_sz), ("shift", c_int), ("negate", c_int), ("mul", c_u64)]


class Operand2(ctypes.Structure):
    """sufhip_operand2 (include/suf_hip.h)."""
    _fields_ = [("t", Term2 * 2), ("party0_const", c_u64)]


class Mul2xArgs(ctypes.Structure):
    """sufhip_mul2x_args (include/suf_hip.h)."""
    _fields_ = [("u", Operand2), ("v", Operand2), ("a", Term2), ("b", Term2), ("c", Term2),
                ("z_add", Operand2), ("z", c_vp * 2), ("zhat", c_vp), ("open_mask", c_u64),
                ("trunc", c_vp)]


class TruncEpilogue(ctypes.Structure):
    """sufhip_trunc_epilogue (include/suf_hip.h)."""
    _fields_ = [("key", c_vp * 2), ("table", c_vp * 2), ("work_bytes", c_sz),
                ("frac_bits", c_int), ("y", c_vp * 2), ("add", c_vp * 2)]


class XPlanes(ctypes.Structure):
    """sufhip_x_planes (include/suf_hip.h)."""
    _fields_ = [("planes", c_vp), ("cols", c_int)]


class Chain2Args(ctypes.Structure):
    """sufhip_chain2_args (include/suf_hip.h)."""
    _fields_ = [("kind", c_int), ("frac_bits", c_int), ("n", c_sz), ("x", Operand2),
                ("lut", c_vp * 2), ("lut_key_bytes", c_sz), ("intervals", c_int),
                ("lut_mask", c_u64), ("a", Term2 * 4), ("b", Term2 * 4), ("c", Term2 * 4),
                ("trunc", TruncEpilogue * 4), ("trunc_mask", c_u64 * 4), ("out", c_vp * 2),
                ("out_planes", XPlanes)]


class KbPlanes(ctypes.Structure):
    """sufhip_kb_planes (include/suf_hip.h)."""
    _fields_ = [("planes", c_vp), ("batches", c_int), ("rows", c_int), ("cols", c_int),
                ("k_is_col", c_int), ("planes_a0", c_vp), ("a0", c_vp)]


class QkvOpens(ctypes.Structure):
    """sufhip_qkv_opens (include/suf_hip.h)."""
    _fields_ = [("heads", c_int), ("seq", c_int), ("dh", c_int), ("sub", (c_vp * 2) * 3),
                ("out", KbPlanes * 3)]


class Lin2Job(ctypes.Structure):
    """sufhip_lin2_job (include/suf_hip.h)."""
    _fields_ = [("x", Operand2), ("n", c_sz), ("out", c_vp * 2), ("xhat", c_vp),
                ("mask", c_u64), ("trunc", c_vp), ("xhat_planes", KbPlanes)]


class BeaverMfma2Args(ctypes.Structure):
    """sufhip_beaver_mfma2_args (include/suf_hip.h)."""
    _fields_ = [("Dp", c_vp), ("Ep", c_vp), ("Ap", c_vp * 2), ("Bp", c_vp * 2), ("C", c_vp * 2),
                ("batches", c_int), ("M", c_int), ("K", c_int), ("N", c_int), ("out", c_vp * 2),
                ("merge_heads", c_int), ("trunc", ctypes.POINTER(TruncEpilogue)),
                ("mask", c_u64), ("out_planes", XPlanes), ("Xp", c_vp)]


class KbSplitJob(ctypes.Structure):
    """sufhip_kb_split_job (include/suf_hip.h)."""
    _fields_ = [("src", c_vp), ("planes", c_vp), ("batches", c_int), ("rows", c_int),
                ("cols", c_int), ("k_is_col", c_int), ("planes_a0", c_vp), ("a0", c_vp)]


class KbOpenJob(ctypes.Structure):
    """sufhip_kb_open_job (include/suf_hip.h)."""
    _fields_ = [("a", c_vp * 2), ("b", c_vp * 2), ("planes", c_vp), ("batches", c_int),
                ("rows", c_int), ("cols", c_int), ("k_is_col", c_int), ("planes_a0", c_vp),
                ("a0", c_vp), ("a_stride", ctypes.c_int64 * 3)]


class Triple2(ctypes.Structure):
    """sufhip_triple2 (include/suf_hip.h)."""
    _fields_ = [("a", c_vp * 2), ("b", c_vp * 2), ("c", c_vp * 2)]


class LayerNorm2Args(ctypes.Structure):
    """sufhip_layernorm2_args (include/suf_hip.h)."""
    _fields_ = [("x", c_vp * 2), ("rows", c_int), ("cols", c_int), ("inv_len", c_u64),
                ("eps", c_u64), ("tr_mean", TruncEpilogue), ("tr_var", TruncEpilogue * 2),
                ("tr_norm", TruncEpilogue), ("mean_mask", c_u64), ("var_mask", c_u64 * 2),
                ("norm_mask", c_u64), ("sq", Triple2), ("norm", Triple2), ("rsqrt", Chain2Args),
                ("out", c_vp * 2), ("out_planes", XPlanes), ("in_slices", c_vp),
                ("in_slice_count", c_int), ("tr_in", TruncEpilogue), ("in_mask", c_u64),
                ("walk_jobs", c_vp), ("walk_count", c_int), ("walk_prg_state", c_vp)]


class ReluRoundKey(ctypes.Structure):
    """sufhip_relu_round_key (include/suf_hip.h)."""
    _fields_ = [("key", c_vp * 2), ("key_bytes", c_sz), ("intervals", c_int), ("mask", c_u64)]


class Softmax2Args(ctypes.Structure):
    """sufhip_softmax2_args (include/suf_hip.h)."""
    _fields_ = [("x", Operand2), ("pre_truncs", c_int), ("pre", TruncEpilogue * 2),
                ("pre_mask", c_u64 * 2), ("rows", c_int), ("d_row_offsets", c_vp),
                ("max_row", c_int), ("rounds", c_int), ("d_round_offsets", c_vp),
                ("keys", ReluRoundKey * 10), ("nexp", Chain2Args), ("recip", Chain2Args),
                ("norm", Triple2), ("tr_norm", TruncEpilogue), ("norm_mask", c_u64),
                ("out", c_vp * 2), ("d_dense", c_vp), ("dense_a", c_vp * 2),
                ("dense_cols", c_int), ("dense_planes", KbPlanes)]


class TruncJob(ctypes.Structure):
    """sufhip_trunc_job (include/suf_hip.h)."""
    _fields_ = [("kind", c_int), ("frac_bits", c_int), ("d_key", c_vp), ("key_bytes", c_sz),
                ("n", c_sz), ("d_work", c_vp), ("work_bytes", c_sz)]


BOOL_VAR, BOOL_WRAP, BOOL_CONST, BOOL_NOT, BOOL_XOR, BOOL_AND, BOOL_OR = range(7)
COMPOSITE_MAX_ELL = 8
COMPOSITE_MAX_CUTS = 31
COMPOSITE_MAX_WRAP = 32
COMPOSITE_MAX_PROG = 384
STAGE_MAX_SEGS = 64


class StageSeg(ctypes.Structure):
    """sufhip_stage_seg (include/suf_hip.h)."""
    _fields_ = [("src", c_vp), ("len", c_sz), ("dst", c_sz), ("eff_bits", c_int)]


class OpenReq(ctypes.Structure):
    """sufhip_open_req (include/suf_hip.h)."""
    _fields_ = [("share", c_vp * 2), ("len", c_sz)]


class CompositeBoolArgs(ctypes.Structure):
    """sufhip_composite_bool_args (include/suf_hip.h)."""
    _fields_ = [("n", c_sz), ("queries", c_int), ("cuts", c_int), ("ell", c_int),
                ("wraps", c_int), ("and_count", c_int), ("prog_len", c_int),
                ("pred", c_vp * 2), ("cut", c_vp * 2), ("bit_tri", c_vp * 2), ("tri", c_vp * 2),
                ("out", c_vp * 2), ("wrap", (c_u64 * COMPOSITE_MAX_WRAP) * 2),
                ("prog_off", ctypes.c_int16 * ((COMPOSITE_MAX_CUTS + 1) * COMPOSITE_MAX_ELL + 1)),
                ("prog", ctypes.c_int32 * COMPOSITE_MAX_PROG)]


class SufHipError(RuntimeError):
    pass


def header_symbols():
    """Names of every function declared in include/suf_hip.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sufhip_[a-z0-9_]+)\s*\(", text)))


def load(path=LIB_PATH):
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise SufHipError("libsuf_hip.so not built: run `python -m suf_amd.build` (%s)" % path)
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc, what=""):
    if rc != OK:
        msg = load().sufhip_last_error().decode(errors="replace")
        raise SufHipError("%s failed (status %d): %s" % (what or "sufhip call", rc, msg))


def call(name, *args):
    rc = getattr(load(), name)(*args)
    check(rc, name)
    return rc
