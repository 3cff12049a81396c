// Drop-in replacement for SUF's include/runtime/cuda_primitives.hpp (reference
// lines 13-236): the same extern "C" launcher prototypes, implemented in
// suf_amd/host/cuda_primitives_shim.cpp on top of the sufhip_* C ABI
// (include/suf_hip.h), so SUF code that calls the launchers by name runs on
// the MI355X kernels unchanged.  Argument lists, names and meanings are the
// reference's; streams are hipStream_t passed as void*.  Like the reference
// launchers they return nothing: a launch the C ABI rejects throws
// std::runtime_error with sufhip_last_error().  A test compiles this header
// together with the reference's own, so any prototype that differs fails to
// compile.
#pragma once

#include <cstddef>
#include <cstdint>

extern "C" {

// :14-24  z = c + d b + e a (+ d e for party 0) mod 2^64
void launch_beaver_mul_kernel(int party, const uint64_t* d_x, const uint64_t* d_y,
                              const uint64_t* d_a, const uint64_t* d_b, const uint64_t* d_c,
                              const uint64_t* d_d_open, const uint64_t* d_e_open, uint64_t* d_out,
                              size_t n, void* stream);
// :28-34  triples {a, b, c} per element
void launch_beaver_mul_aos_kernel(int party, const void* d_triples, const uint64_t* d_d_open,
                                  const uint64_t* d_e_open, uint64_t* d_out, size_t n,
                                  void* stream);
// :38-42
void launch_trunc_shift_kernel(const uint64_t* d_in, uint64_t* d_out, int frac_bits, size_t n,
                               void* stream);
// :47-63  faithful / GapARS truncation output share
void launch_trunc_postproc_kernel(int party, int kind_gapars, int frac_bits, uint64_t r_hi_share,
                                  uint64_t m_share, const uint64_t* d_hatx_public,
                                  const uint64_t* d_arith, size_t arith_stride, int arith_idx,
                                  const uint64_t* d_bools, size_t bool_stride, int carry_idx,
                                  int sign_idx, int wrap_idx, uint64_t* d_out, size_t n,
                                  void* stream);
// :67-74
void launch_horner_cubic_kernel(const uint64_t* d_x, const uint64_t* d_c0, const uint64_t* d_c1,
                                const uint64_t* d_c2, const uint64_t* d_c3, uint64_t* d_out,
                                size_t n, void* stream);
// :78-83  r_out is a host array
void launch_add_rout_aos_kernel(uint64_t* d_out, size_t elems, int out_words,
                                const uint64_t* r_out, size_t r_out_words, void* stream);
// :90-101
void launch_row_broadcast_mul_kernel(int party, const uint64_t* d_A, const uint64_t* d_B_rows,
                                     const uint64_t* d_C, const uint64_t* d_d_open,
                                     const uint64_t* d_e_open_rows, int rows, int cols,
                                     const int* d_valid_lens, uint64_t* d_out, size_t n,
                                     void* stream);
// :105-110
void launch_row_sum_kernel(const uint64_t* d_mat, int rows, int cols, const int* d_valid_lens,
                           uint64_t* d_out_rows, void* stream);
// :116-120
void launch_row_sum_ragged_kernel(const uint64_t* d_vals, const int* d_row_offsets, int rows,
                                  uint64_t* d_out_rows, void* stream);
// :132-146
void launch_beaver_matmul2d_kernel(int party, const uint64_t* d_D_open, const uint64_t* d_E_open,
                                   const uint64_t* d_A_tri_share, const uint64_t* d_B_tri_share,
                                   const uint64_t* d_C_tri_share, int M, int K, int N,
                                   int w_transposed, int has_scale, int64_t mul_const,
                                   int mul_shift, uint64_t* d_out, void* stream);
// :150-165  the same triple shares for every batch instance
void launch_beaver_matmul2d_batched_kernel(int party, const uint64_t* d_D_open,
                                           const uint64_t* d_E_open,
                                           const uint64_t* d_A_tri_share,
                                           const uint64_t* d_B_tri_share,
                                           const uint64_t* d_C_tri_share, int batches, int M,
                                           int K, int N, int w_transposed, int has_scale,
                                           int64_t mul_const, int mul_shift, uint64_t* d_out,
                                           void* stream);
// :168-173
void launch_row_mean_kernel(const uint64_t* d_mat, int rows, int cols, const int* d_valid_lens,
                            uint64_t* d_out_rows, void* stream);
// :178-184
void launch_row_variance_kernel(const uint64_t* d_mat, const uint64_t* d_mean, int rows, int cols,
                                const int* d_valid_lens, uint64_t* d_out_rows, void* stream);
// :188-192, :196-200
void launch_unpack_eff_bits_kernel(const uint64_t* d_packed, int eff_bits, uint64_t* d_out,
                                   size_t n, void* stream);
void launch_pack_eff_bits_kernel(const uint64_t* d_in, int eff_bits, uint64_t* d_packed, size_t n,
                                 void* stream);
// :205-211, :216-223, :228-235
void launch_open_add_to_signed_kernel(const uint64_t* d_local_share,
                                      const uint64_t* d_remote_share, uint64_t* d_out_signed,
                                      size_t n, int ring_bits, uint64_t ring_mask, void* stream);
void launch_unpack_add_to_signed_kernel(const uint64_t* d_local_share,
                                        const uint64_t* d_packed_remote, int eff_bits,
                                        uint64_t* d_out_signed, size_t n, int ring_bits,
                                        uint64_t ring_mask, void* stream);
void launch_unpack_add_mod_kernel(const uint64_t* d_local_share, const uint64_t* d_packed_remote,
                                  int eff_bits, uint64_t* d_out_mod, size_t n, int ring_bits,
                                  uint64_t ring_mask, void* stream);

}  // extern "C"
