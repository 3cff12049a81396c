/*
 * Oracle: Z_2^64 postprocessing, Beaver products and row reductions.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  All arithmetic is mod 2^64
 * (unsigned wrap-around), as in cuda/cuda_primitives.cu:21-24.
 */
#include "oracle.h"

#include <string.h>

/* cuda/cuda_primitives.cu:114-135 (beaver_mul_kernel): z = c + d*b + e*a (+ d*e, party 0). */
void orc_beaver_mul(int party, const uint64_t* a, const uint64_t* b, const uint64_t* c,
                    const uint64_t* d, const uint64_t* e, uint64_t* out, size_t n) {
  for (size_t i = 0; i < n; i++) {
    uint64_t z = c[i] + d[i] * b[i] + e[i] * a[i];
    if (party == 0) z += d[i] * e[i];
    out[i] = z;
  }
}

/* cuda/cuda_primitives.cu:179-252 (trunc_postproc_kernel), the same formulas as
 * include/gates/postproc_hooks.hpp:172-373 (FaithfulTrunc/FaithfulArs/GapArs). */
void orc_trunc_postproc(int party, int kind_gapars, int f, uint64_t r_hi_share,
                        uint64_t m_share, const uint64_t* hatx, const uint64_t* arith,
                        size_t arith_stride, int arith_idx, const uint64_t* bools,
                        size_t bool_stride, int carry_idx, int sign_idx, int wrap_idx,
                        uint64_t* out, size_t n) {
  int have_c = bools && carry_idx >= 0 && carry_idx < (int)bool_stride;
  int have_s = bools && sign_idx >= 0 && sign_idx < (int)bool_stride;
  int have_w = bools && wrap_idx >= 0 && wrap_idx < (int)bool_stride;
  for (size_t i = 0; i < n; i++) {
    uint64_t y = arith[(size_t)arith_idx + i * arith_stride];
    uint64_t carry = have_c ? bools[(size_t)carry_idx + i * bool_stride] : 0;
    uint64_t sign = have_s ? bools[(size_t)sign_idx + i * bool_stride] : 0;
    uint64_t wrap = have_w ? bools[(size_t)wrap_idx + i * bool_stride] : 0;
    if (kind_gapars) {
      uint64_t hb = (hatx ? hatx[i] : 0) + (1ULL << 62);
      if (party == 0) y += f <= 0 ? hb : (f >= 64 ? 0 : hb >> f);
      y -= r_hi_share;
      y -= carry;
      if (f > 0 && f < 64 && (hb >> 63) == 0) y += m_share;
      if (party == 0 && f >= 0 && f <= 62) y -= 1ULL << (62 - f);
    } else {
      if (party == 0 && f > 0 && f < 64) y += hatx ? hatx[i] >> f : 0;
      y -= r_hi_share;
      y -= carry;
      if (f > 0 && f < 64) {
        y += wrap * (1ULL << (64 - f));
        y += sign * (~0ULL << (64 - f));
      }
    }
    out[i] = y;
  }
}

/* cuda/cuda_primitives.cu:254-269 */
void orc_horner_cubic(const uint64_t* x, const uint64_t* c0, const uint64_t* c1,
                      const uint64_t* c2, const uint64_t* c3, uint64_t* out, size_t n) {
  for (size_t i = 0; i < n; i++) {
    uint64_t y = c3[i];
    y = y * x[i] + c2[i];
    y = y * x[i] + c1[i];
    y = y * x[i] + c0[i];
    out[i] = y;
  }
}

/* cuda/cuda_primitives.cu:271-301; word j of each element gains r_out[j] for
 * j < r_out_words.  (The reference launcher, :824-850, does nothing at all when
 * out_words or r_out_words exceeds 8; this oracle states the kernel formula.) */
void orc_add_rout_aos(uint64_t* out, size_t elems, int out_words, const uint64_t* r_out,
                      int r_out_words) {
  if (out_words <= 0) return;
  for (size_t i = 0; i < elems; i++)
    for (int j = 0; j < out_words && j < r_out_words; j++)
      out[i * (size_t)out_words + (size_t)j] += r_out[j];
}

/* cuda/cuda_primitives.cu:303-336 */
void orc_row_broadcast_mul(int party, const uint64_t* A, const uint64_t* B_rows,
                           const uint64_t* C, const uint64_t* d, const uint64_t* e_rows,
                           int rows, int cols, const int* valid_lens, uint64_t* out) {
  for (int r = 0; r < rows; r++)
    for (int c = 0; c < cols; c++) {
      size_t i = (size_t)r * (size_t)cols + (size_t)c;
      if (valid_lens && c >= valid_lens[r]) {
        out[i] = 0;
        continue;
      }
      uint64_t z = C[i] + d[i] * B_rows[r] + e_rows[r] * A[i];
      if (party == 0) z += d[i] * e_rows[r];
      out[i] = z;
    }
}

/* cuda/cuda_primitives.cu:339-361 */
void orc_row_sum(const uint64_t* mat, int rows, int cols, const int* valid_lens,
                 uint64_t* out) {
  for (int r = 0; r < rows; r++) {
    int L = valid_lens ? valid_lens[r] : cols;
    uint64_t acc = 0;
    for (int c = 0; c < L; c++) acc += mat[(size_t)r * (size_t)cols + (size_t)c];
    out[r] = acc;
  }
}

/* cuda/cuda_primitives.cu:365-389 */
void orc_row_sum_ragged(const uint64_t* vals, const int* row_offsets, int rows,
                        uint64_t* out) {
  for (int r = 0; r < rows; r++) {
    int s = row_offsets ? row_offsets[r] : 0, e = row_offsets ? row_offsets[r + 1] : 0;
    if (s < 0) s = 0;
    if (e < s) e = s;
    uint64_t acc = 0;
    for (int i = s; i < e; i++) acc += vals[i];
    out[r] = acc;
  }
}

/* cuda/cuda_primitives.cu:672-707: sum of (x - mu)^2 over the active columns. */
void orc_row_variance(const uint64_t* mat, const uint64_t* mean, int rows, int cols,
                      const int* valid_lens, uint64_t* out) {
  for (int r = 0; r < rows; r++) {
    int L = valid_lens ? valid_lens[r] : cols;
    uint64_t acc = 0;
    for (int c = 0; c < L; c++) {
      uint64_t dlt = mat[(size_t)r * (size_t)cols + (size_t)c] - mean[r];
      acc += dlt * dlt;
    }
    out[r] = L <= 0 ? 0 : acc;
  }
}

/* cuda/cuda_primitives.cu:391-417: optional (acc * c) >> s on the signed 128-bit product. */
uint64_t orc_beaver_scale(uint64_t acc, int has_scale, int64_t mul_const, int mul_shift) {
  if (!has_scale) return acc;
  __int128 p = (__int128)(int64_t)acc * (__int128)mul_const;
  if (mul_shift <= 0) return (uint64_t)p;
  if (mul_shift >= 128) return (uint64_t)(p >> 127);
  return (uint64_t)(p >> mul_shift);
}

/* cuda/cuda_primitives.cu:419-506 (dense and batched): out = C + D*B + A*E (+ D*E, party 0);
 * A, B, C are shared by every batch instance (launcher comment, cuda_primitives.hpp:149-150). */
void orc_beaver_matmul(int party, const uint64_t* D, const uint64_t* E, const uint64_t* A,
                       const uint64_t* B, const uint64_t* C, int batches, int M, int K,
                       int N, int w_transposed, int has_scale, int64_t mul_const,
                       int mul_shift, uint64_t* out, int threads) {
  (void)threads;
  size_t MK = (size_t)M * K, KN = (size_t)K * N, MN = (size_t)M * N;
#pragma omp parallel for collapse(2) schedule(static) num_threads(orc_threads_or_default(threads))
  for (int b = 0; b < batches; b++)
    for (int m = 0; m < M; m++)
      for (int n = 0; n < N; n++) {
        uint64_t acc = C[(size_t)m * N + n];
        for (int k = 0; k < K; k++) {
          size_t ai = (size_t)m * K + k;
          size_t bi = w_transposed ? (size_t)n * K + k : (size_t)k * N + n;
          uint64_t d = D[b * MK + ai], e = E[b * KN + bi];
          acc += d * B[bi] + A[ai] * e;
          if (party == 0) acc += d * e;
        }
        out[b * MN + (size_t)m * N + n] = orc_beaver_scale(acc, has_scale, mul_const, mul_shift);
      }
}

/* src/nn/matmul_publicW.cpp:17-36: Y = X * W mod 2^64 for a share X [M x K]
 * and public int64 W [K x N] (the reference layer passes no bias), with the
 * reference's loop order; OpenMP over the outputs. */
void orc_matmul_public(const uint64_t* X, const int64_t* W, int M, int K, int N, uint64_t* Y) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; m++)
    for (int n = 0; n < N; n++) {
      uint64_t acc = 0;
      for (int k = 0; k < K; k++) acc += X[(size_t)m * K + k] * (uint64_t)W[(size_t)k * N + n];
      Y[(size_t)m * N + n] = acc;
    }
}

/* Bit packing of fixed-width values, LSB-first within little-endian u64 words
 * (cuda/pfss_backend_gpu.cu:118-138, cuda/pfss_kernels.cu:722-812). */
void orc_pack_eff_bits(const uint64_t* in, int eff_bits, uint64_t* packed, size_t n) {
  if (eff_bits >= 64) {
    memcpy(packed, in, n * 8);
    return;
  }
  size_t words = (n * (size_t)eff_bits + 63) / 64;
  memset(packed, 0, words * 8);
  uint64_t m = (1ULL << eff_bits) - 1;
  for (size_t i = 0; i < n; i++) {
    uint64_t v = in[i] & m;
    size_t bit = i * (size_t)eff_bits, w = bit >> 6;
    int off = (int)(bit & 63);
    packed[w] |= v << off;
    if (off + eff_bits > 64 && w + 1 < words) packed[w + 1] |= v >> (64 - off);
  }
}

void orc_unpack_eff_bits(const uint64_t* packed, int eff_bits, uint64_t* out, size_t n) {
  if (eff_bits >= 64) {
    memcpy(out, packed, n * 8);
    return;
  }
  size_t words = (n * (size_t)eff_bits + 63) / 64;
  uint64_t m = (1ULL << eff_bits) - 1;
  for (size_t i = 0; i < n; i++) {
    size_t bit = i * (size_t)eff_bits, w = bit >> 6;
    int off = (int)(bit & 63);
    uint64_t lo = packed[w], hi = w + 1 < words ? packed[w + 1] : 0;
    uint64_t v = off == 0 ? lo : (lo >> off) | (hi << (64 - off));
    out[i] = v & m;
  }
}

/* cuda/cuda_primitives.cu:630-670 (row_mean_kernel): the row sum shifted right
 * by log2(L) when L is a power of two, else the u64 sum divided by L as a plain
 * unsigned integer (the reference's formula; not a ring operation). */
void orc_row_mean(const uint64_t* mat, int rows, int cols, const int* valid_lens,
                  uint64_t* out) {
  for (int r = 0; r < rows; r++) {
    int L = valid_lens ? valid_lens[r] : cols;
    if (L <= 0) {
      out[r] = 0;
      continue;
    }
    uint64_t acc = 0;
    for (int c = 0; c < L; c++) acc += mat[(size_t)r * (size_t)cols + (size_t)c];
    if ((L & (L - 1)) == 0) {
      int sh = 0;
      while ((1 << sh) != L && sh < 63) ++sh;
      out[r] = acc >> sh;
    } else {
      out[r] = acc / (uint64_t)(unsigned)L;
    }
  }
}

static uint64_t ring_sign(uint64_t v, int ring_bits, uint64_t ring_mask) {
  if (ring_bits >= 64) return v;
  v &= ring_mask;
  if (v & (1ULL << (ring_bits - 1))) v |= ~ring_mask;
  return v;
}

/* cuda/cuda_primitives.cu:26-112: open = local + remote (remote optionally
 * eff_bits-packed), then either sign-extended from ring_bits (to_signed) or
 * masked to the ring (mod). */
void orc_open_add(const uint64_t* local, const uint64_t* remote, int eff_bits, uint64_t* out,
                  size_t n, int ring_bits, uint64_t ring_mask, int sign_extend) {
  if (ring_bits <= 0) ring_bits = 1;
  if (ring_bits > 64) ring_bits = 64;
  if (eff_bits <= 0) eff_bits = 1;
  if (eff_bits > 64) eff_bits = 64;
  size_t words = (size_t)(((unsigned __int128)n * (unsigned)eff_bits + 63) / 64);
  uint64_t m = eff_bits >= 64 ? ~0ULL : (1ULL << eff_bits) - 1;
  for (size_t i = 0; i < n; i++) {
    uint64_t r;
    if (eff_bits >= 64) {
      r = remote[i];
    } else {
      size_t bit = i * (size_t)eff_bits, w = bit >> 6;
      int off = (int)(bit & 63);
      uint64_t lo = w < words ? remote[w] : 0, hi = w + 1 < words ? remote[w + 1] : 0;
      r = (off == 0 ? lo : (lo >> off) | (hi << (64 - off))) & m;
    }
    uint64_t v = local[i] + r;
    if (sign_extend) {
      out[i] = ring_sign(v, ring_bits, ring_mask);
    } else {
      out[i] = ring_bits < 64 ? v & ring_mask : v;
    }
  }
}
