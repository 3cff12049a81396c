// Z_2^64 postprocessing, Beaver products, row reductions and open-path
// packing: the launch surface of include/runtime/cuda_primitives.hpp:13-236,
// re-implemented for CDNA4.
//
// Elementwise kernels are HBM-bound streams: grid-stride loops over 256-thread
// workgroups, one u64 per lane per array (a wave moves 512 contiguous bytes
// per array per step).  Row reductions give each row to one wave (64 lanes
// stride the row, then a 6-step xor-shuffle reduction), four rows per
// workgroup.  u64 products compile to 32-bit multiply sequences (CDNA has no
// 64-bit integer multiply); all arithmetic wraps mod 2^64.
#include <hip/hip_runtime.h>

#include <cstring>

#include "sufhip_internal.hpp"

namespace sufhip {
namespace {

constexpr int kBlock = 256;

unsigned int stream_grid(size_t n) {
  size_t g = (n + kBlock - 1) / kBlock;
  const size_t cap = 256 * 16;  // 16 workgroups per CU is plenty for a stream
  return static_cast<unsigned int>(g < cap ? g : cap);
}

#define GRID_STRIDE(i, n)                                                    \
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < (n); \
       i += size_t(gridDim.x) * blockDim.x)

__global__ void __launch_bounds__(kBlock)
    beaver_mul_kernel(int party, const uint64_t* __restrict__ a, const uint64_t* __restrict__ b,
                      const uint64_t* __restrict__ c, const uint64_t* __restrict__ d,
                      const uint64_t* __restrict__ e, uint64_t* __restrict__ out, size_t n) {
  GRID_STRIDE(i, n) {
    const uint64_t dv = d[i], ev = e[i];
    uint64_t z = c[i] + dv * b[i] + ev * a[i];
    if (party == 0) z += dv * ev;
    out[i] = z;
  }
}

struct TripleAos {
  uint64_t a, b, c;
};

__global__ void __launch_bounds__(kBlock)
    beaver_mul_aos_kernel(int party, const TripleAos* __restrict__ t,
                          const uint64_t* __restrict__ d, const uint64_t* __restrict__ e,
                          uint64_t* __restrict__ out, size_t n) {
  GRID_STRIDE(i, n) {
    const TripleAos tr = t[i];
    const uint64_t dv = d[i], ev = e[i];
    uint64_t z = tr.c + dv * tr.b + ev * tr.a;
    if (party == 0) z += dv * ev;
    out[i] = z;
  }
}

__global__ void __launch_bounds__(kBlock)
    trunc_shift_kernel(const uint64_t* __restrict__ in, uint64_t* __restrict__ out, int f,
                       size_t n) {
  GRID_STRIDE(i, n) {
    const uint64_t x = in[i];
    out[i] = f <= 0 ? x : (f >= 64 ? 0 : x >> f);
  }
}

struct TruncArgs {
  const uint64_t* hatx;
  const uint64_t* arith;
  const uint64_t* bools;
  uint64_t* out;
  size_t n;
  size_t arith_stride;
  size_t bool_stride;
  uint64_t r_hi;
  uint64_t m;
  int party;
  int gapars;
  int f;
  int arith_idx;
  int carry_idx;  // -1 when absent
  int sign_idx;
  int wrap_idx;
};

// Faithful TR / ARS and GapARS output share (cuda/cuda_primitives.cu:179-252,
// the same formulas as include/gates/postproc_hooks.hpp:172-373).
__global__ void __launch_bounds__(kBlock) trunc_postproc_kernel(TruncArgs a) {
  GRID_STRIDE(i, a.n) {
    uint64_t y = a.arith[size_t(a.arith_idx) + i * a.arith_stride];
    const uint64_t* br = a.bools + i * a.bool_stride;
    const uint64_t carry = a.carry_idx >= 0 ? br[a.carry_idx] : 0;
    const int f = a.f;
    if (a.gapars) {
      const uint64_t hb = (a.hatx ? a.hatx[i] : 0) + (uint64_t(1) << 62);
      if (a.party == 0) y += f <= 0 ? hb : (f >= 64 ? 0 : hb >> f);
      y -= a.r_hi;
      y -= carry;
      if (f > 0 && f < 64 && (hb >> 63) == 0) y += a.m;
      if (a.party == 0 && f >= 0 && f <= 62) y -= uint64_t(1) << (62 - f);
    } else {
      if (a.party == 0 && f > 0 && f < 64 && a.hatx) y += a.hatx[i] >> f;
      y -= a.r_hi;
      y -= carry;
      if (f > 0 && f < 64) {
        const uint64_t wrap = a.wrap_idx >= 0 ? br[a.wrap_idx] : 0;
        const uint64_t sign = a.sign_idx >= 0 ? br[a.sign_idx] : 0;
        y += wrap * (uint64_t(1) << (64 - f));
        y += sign * (~uint64_t(0) << (64 - f));
      }
    }
    a.out[i] = y;
  }
}

__global__ void __launch_bounds__(kBlock)
    horner_cubic_kernel(const uint64_t* __restrict__ x, const uint64_t* __restrict__ c0,
                        const uint64_t* __restrict__ c1, const uint64_t* __restrict__ c2,
                        const uint64_t* __restrict__ c3, uint64_t* __restrict__ out, size_t n) {
  GRID_STRIDE(i, n) {
    const uint64_t xv = x[i];
    uint64_t y = c3[i];
    y = y * xv + c2[i];
    y = y * xv + c1[i];
    y = y * xv + c0[i];
    out[i] = y;
  }
}

constexpr int kMaxRoutWords = 64;
struct Rout {
  uint64_t w[kMaxRoutWords];
};

__global__ void __launch_bounds__(kBlock)
    add_rout_aos_kernel(uint64_t* __restrict__ out, size_t words, int out_words, int rw, Rout r) {
  GRID_STRIDE(i, words) {
    const int j = int(i % size_t(out_words));
    if (j < rw) out[i] += r.w[j];
  }
}

__global__ void __launch_bounds__(kBlock)
    row_broadcast_mul_kernel(int party, const uint64_t* __restrict__ A,
                             const uint64_t* __restrict__ B_rows, const uint64_t* __restrict__ C,
                             const uint64_t* __restrict__ d, const uint64_t* __restrict__ e_rows,
                             int rows, int cols, const int* __restrict__ valid_lens,
                             uint64_t* __restrict__ out, size_t n) {
  GRID_STRIDE(i, n) {
    const int r = int(i / size_t(cols));
    const int c = int(i - size_t(r) * size_t(cols));
    if (r >= rows) continue;
    if (valid_lens && c >= valid_lens[r]) {
      out[i] = 0;
      continue;
    }
    const uint64_t dv = d[i], ev = e_rows[r];
    uint64_t z = C[i] + dv * B_rows[r] + ev * A[i];
    if (party == 0) z += dv * ev;
    out[i] = z;
  }
}

__device__ __forceinline__ uint64_t wave_sum(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

enum RowOp { kRowSum = 0, kRowMean = 1, kRowVar = 2 };

// One wave per row; rows [r0, r0 + 4) per workgroup, grid-stride over rows.
template <int kOp>
__global__ void __launch_bounds__(kBlock)
    row_reduce_kernel(const uint64_t* __restrict__ mat, const uint64_t* __restrict__ mean,
                      int rows, int cols, const int* __restrict__ valid_lens,
                      uint64_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (int r = blockIdx.x * (kBlock / 64) + wave; r < rows; r += gridDim.x * (kBlock / 64)) {
    int L = valid_lens ? valid_lens[r] : cols;
    if (L > cols) L = cols;
    const uint64_t* row = mat + size_t(r) * size_t(cols);
    const uint64_t mu = kOp == kRowVar ? mean[r] : 0;
    uint64_t acc = 0;
    for (int c = lane; c < L; c += 64) {
      const uint64_t v = row[c];
      if constexpr (kOp == kRowVar) {
        const uint64_t dv = v - mu;
        acc += dv * dv;
      } else {
        acc += v;
      }
    }
    acc = wave_sum(acc);
    if (lane == 0) {
      uint64_t res = acc;
      if (L <= 0) {
        res = 0;
      } else if constexpr (kOp == kRowMean) {
        if ((L & (L - 1)) == 0)
          res = acc >> (31 - __builtin_clz(unsigned(L)));
        else
          res = acc / uint64_t(unsigned(L));
      }
      out[r] = res;
    }
  }
}

__global__ void __launch_bounds__(kBlock)
    row_sum_ragged_kernel(const uint64_t* __restrict__ vals, const int* __restrict__ offs,
                          int rows, uint64_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (int r = blockIdx.x * (kBlock / 64) + wave; r < rows; r += gridDim.x * (kBlock / 64)) {
    int s = offs ? offs[r] : 0, e = offs ? offs[r + 1] : 0;
    if (s < 0) s = 0;
    if (e < s) e = s;
    uint64_t acc = 0;
    for (int i = s + lane; i < e; i += 64) acc += vals[i];
    acc = wave_sum(acc);
    if (lane == 0) out[r] = acc;
  }
}

__device__ __forceinline__ uint64_t low_mask(int bits) {
  return bits >= 64 ? ~uint64_t(0) : ((uint64_t(1) << bits) - 1);
}

// Reads element i of an eff_bits-packed LSB-first stream of `words` words.
__device__ __forceinline__ uint64_t packed_get(const uint64_t* __restrict__ p, int eff_bits,
                                               size_t words, size_t i) {
  if (eff_bits >= 64) return p[i];
  const size_t bit = i * size_t(eff_bits), w = bit >> 6;
  const int off = int(bit & 63);
  const uint64_t lo = w < words ? p[w] : 0;
  const uint64_t hi = (off + eff_bits > 64 && w + 1 < words) ? p[w + 1] : 0;
  const uint64_t v = off == 0 ? lo : (lo >> off) | (hi << (64 - off));
  return v & low_mask(eff_bits);
}

__global__ void __launch_bounds__(kBlock)
    unpack_kernel(const uint64_t* __restrict__ packed, int eff_bits, size_t words,
                  uint64_t* __restrict__ out, size_t n) {
  GRID_STRIDE(i, n) out[i] = packed_get(packed, eff_bits, words, i);
}

// Word-wise pack: each output word is assembled by one lane from the (at most
// 64 / eff_bits + 2) input elements that overlap it; no atomics, no clearing.
__global__ void __launch_bounds__(kBlock)
    pack_kernel(const uint64_t* __restrict__ in, int eff_bits, uint64_t* __restrict__ packed,
                size_t n, size_t words) {
  const uint64_t m = low_mask(eff_bits);
  GRID_STRIDE(w, words) {
    if (eff_bits >= 64) {
      packed[w] = w < n ? in[w] : 0;
      continue;
    }
    const uint64_t bit0 = uint64_t(w) * 64;
    size_t idx = size_t(bit0 / unsigned(eff_bits));
    int off = int(bit0 - uint64_t(idx) * unsigned(eff_bits));  // bits of in[idx] already used
    uint64_t word = 0;
    int filled = 0;
    while (filled < 64 && idx < n) {
      const uint64_t v = (in[idx] & m) >> off;
      const int avail = eff_bits - off;
      word |= v << filled;  // bits past 64 fall off
      filled += avail;
      ++idx;
      off = 0;
    }
    packed[w] = word;
  }
}

// open = local + remote (remote eff_bits-packed when eff_bits < 64), then
// sign-extended from ring_bits or masked to the ring
// (cuda/cuda_primitives.cu:26-112).
template <bool kSigned>
__global__ void __launch_bounds__(kBlock)
    open_add_kernel(const uint64_t* __restrict__ local, const uint64_t* __restrict__ remote,
                    int eff_bits, size_t words, uint64_t* __restrict__ out, size_t n,
                    int ring_bits, uint64_t ring_mask) {
  GRID_STRIDE(i, n) {
    uint64_t v = local[i] + packed_get(remote, eff_bits, words, i);
    if (ring_bits < 64) {
      v &= ring_mask;
      if (kSigned && (v & (uint64_t(1) << (ring_bits - 1)))) v |= ~ring_mask;
    }
    out[i] = v;
  }
}

size_t packed_words(size_t n, int eff_bits) {
  return static_cast<size_t>((static_cast<unsigned __int128>(n) * unsigned(eff_bits) + 63) / 64);
}

int clamp_bits(int b) { return b < 1 ? 1 : (b > 64 ? 64 : b); }

unsigned int row_grid(int rows) {
  const int per = kBlock / 64;
  int g = (rows + per - 1) / per;
  return static_cast<unsigned int>(g < 4096 ? g : 4096);
}

}  // namespace
}  // namespace sufhip

using namespace sufhip;

extern "C" {

int sufhip_beaver_mul(int party, const uint64_t* d_x, const uint64_t* d_y, const uint64_t* d_a,
                      const uint64_t* d_b, const uint64_t* d_c, const uint64_t* d_d_open,
                      const uint64_t* d_e_open, uint64_t* d_out, size_t n, void* stream) {
  (void)d_x;
  (void)d_y;
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_a && d_b && d_c && d_d_open && d_e_open && d_out,
                 "sufhip_beaver_mul: null pointer");
  hipLaunchKernelGGL(beaver_mul_kernel, dim3(stream_grid(n)), dim3(kBlock), 0, as_stream(stream),
                     party, d_a, d_b, d_c, d_d_open, d_e_open, d_out, n);
  return check_launch("beaver_mul_kernel");
}

int sufhip_beaver_mul_aos(int party, const void* d_triples, const uint64_t* d_d_open,
                          const uint64_t* d_e_open, uint64_t* d_out, size_t n, void* stream) {
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_triples && d_d_open && d_e_open && d_out, "sufhip_beaver_mul_aos: null pointer");
  hipLaunchKernelGGL(beaver_mul_aos_kernel, dim3(stream_grid(n)), dim3(kBlock), 0,
                     as_stream(stream), party, static_cast<const TripleAos*>(d_triples), d_d_open,
                     d_e_open, d_out, n);
  return check_launch("beaver_mul_aos_kernel");
}

int sufhip_trunc_shift(const uint64_t* d_in, uint64_t* d_out, int frac_bits, size_t n,
                       void* stream) {
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_in && d_out, "sufhip_trunc_shift: null pointer");
  hipLaunchKernelGGL(trunc_shift_kernel, dim3(stream_grid(n)), dim3(kBlock), 0, as_stream(stream),
                     d_in, d_out, frac_bits, n);
  return check_launch("trunc_shift_kernel");
}

int sufhip_trunc_postproc(int party, int kind_gapars, int frac_bits, uint64_t r_hi_share,
                          uint64_t m_share, const uint64_t* d_hatx_public, const uint64_t* d_arith,
                          size_t arith_stride, int arith_idx, const uint64_t* d_bools,
                          size_t bool_stride, int carry_idx, int sign_idx, int wrap_idx,
                          uint64_t* d_out, size_t n, void* stream) {
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_arith && d_out, "sufhip_trunc_postproc: null pointer");
  SUFHIP_REQUIRE(arith_idx >= 0 && (arith_stride > size_t(arith_idx) || (arith_stride == 0 && arith_idx == 0)),
                 "sufhip_trunc_postproc: arith_idx outside arith_stride");
  TruncArgs a{};
  a.hatx = d_hatx_public;
  a.arith = d_arith;
  a.bools = d_bools;
  a.out = d_out;
  a.n = n;
  a.arith_stride = arith_stride;
  a.bool_stride = bool_stride;
  a.r_hi = r_hi_share;
  a.m = m_share;
  a.party = party;
  a.gapars = kind_gapars ? 1 : 0;
  a.f = frac_bits;
  a.arith_idx = arith_idx;
  // Same presence rule as the reference: an index is used only when it lies in
  // [0, bool_stride) and bools are given.
  auto use = [&](int idx) { return (d_bools && idx >= 0 && size_t(idx) < bool_stride) ? idx : -1; };
  a.carry_idx = use(carry_idx);
  a.sign_idx = use(sign_idx);
  a.wrap_idx = use(wrap_idx);
  hipLaunchKernelGGL(trunc_postproc_kernel, dim3(stream_grid(n)), dim3(kBlock), 0,
                     as_stream(stream), a);
  return check_launch("trunc_postproc_kernel");
}

int sufhip_horner_cubic(const uint64_t* d_x, const uint64_t* d_c0, const uint64_t* d_c1,
                        const uint64_t* d_c2, const uint64_t* d_c3, uint64_t* d_out, size_t n,
                        void* stream) {
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_x && d_c0 && d_c1 && d_c2 && d_c3 && d_out, "sufhip_horner_cubic: null pointer");
  hipLaunchKernelGGL(horner_cubic_kernel, dim3(stream_grid(n)), dim3(kBlock), 0,
                     as_stream(stream), d_x, d_c0, d_c1, d_c2, d_c3, d_out, n);
  return check_launch("horner_cubic_kernel");
}

int sufhip_add_rout_aos(uint64_t* d_out, size_t elems, int out_words, const uint64_t* r_out,
                        size_t r_out_words, void* stream) {
  if (elems == 0 || out_words <= 0 || r_out_words == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_out && r_out, "sufhip_add_rout_aos: null pointer");
  SUFHIP_REQUIRE(out_words <= kMaxRoutWords && r_out_words <= size_t(kMaxRoutWords),
                 "sufhip_add_rout_aos: at most 64 words per element");
  Rout r{};
  std::memcpy(r.w, r_out, r_out_words * sizeof(uint64_t));
  const size_t words = elems * size_t(out_words);
  hipLaunchKernelGGL(add_rout_aos_kernel, dim3(stream_grid(words)), dim3(kBlock), 0,
                     as_stream(stream), d_out, words, out_words, int(r_out_words), r);
  return check_launch("add_rout_aos_kernel");
}

int sufhip_row_broadcast_mul(int party, const uint64_t* d_A, const uint64_t* d_B_rows,
                             const uint64_t* d_C, const uint64_t* d_d_open,
                             const uint64_t* d_e_open_rows, int rows, int cols,
                             const int* d_valid_lens, uint64_t* d_out, size_t n, void* stream) {
  if (n == 0 || rows <= 0 || cols <= 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_A && d_B_rows && d_C && d_d_open && d_e_open_rows && d_out,
                 "sufhip_row_broadcast_mul: null pointer");
  SUFHIP_REQUIRE(n <= size_t(rows) * size_t(cols), "sufhip_row_broadcast_mul: n > rows * cols");
  hipLaunchKernelGGL(row_broadcast_mul_kernel, dim3(stream_grid(n)), dim3(kBlock), 0,
                     as_stream(stream), party, d_A, d_B_rows, d_C, d_d_open, d_e_open_rows, rows,
                     cols, d_valid_lens, d_out, n);
  return check_launch("row_broadcast_mul_kernel");
}

int sufhip_row_sum(const uint64_t* d_mat, int rows, int cols, const int* d_valid_lens,
                   uint64_t* d_out_rows, void* stream) {
  if (rows <= 0 || cols <= 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_mat && d_out_rows, "sufhip_row_sum: null pointer");
  hipLaunchKernelGGL(row_reduce_kernel<kRowSum>, dim3(row_grid(rows)), dim3(kBlock), 0,
                     as_stream(stream), d_mat, nullptr, rows, cols, d_valid_lens, d_out_rows);
  return check_launch("row_sum_kernel");
}

int sufhip_row_sum_ragged(const uint64_t* d_vals, const int* d_row_offsets, int rows,
                          uint64_t* d_out_rows, void* stream) {
  if (rows <= 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_vals && d_row_offsets && d_out_rows, "sufhip_row_sum_ragged: null pointer");
  hipLaunchKernelGGL(row_sum_ragged_kernel, dim3(row_grid(rows)), dim3(kBlock), 0,
                     as_stream(stream), d_vals, d_row_offsets, rows, d_out_rows);
  return check_launch("row_sum_ragged_kernel");
}

int sufhip_row_mean(const uint64_t* d_mat, int rows, int cols, const int* d_valid_lens,
                    uint64_t* d_out_rows, void* stream) {
  if (rows <= 0 || cols <= 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_mat && d_out_rows, "sufhip_row_mean: null pointer");
  hipLaunchKernelGGL(row_reduce_kernel<kRowMean>, dim3(row_grid(rows)), dim3(kBlock), 0,
                     as_stream(stream), d_mat, nullptr, rows, cols, d_valid_lens, d_out_rows);
  return check_launch("row_mean_kernel");
}

int sufhip_row_variance(const uint64_t* d_mat, const uint64_t* d_mean, int rows, int cols,
                        const int* d_valid_lens, uint64_t* d_out_rows, void* stream) {
  if (rows <= 0 || cols <= 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_mat && d_mean && d_out_rows, "sufhip_row_variance: null pointer");
  hipLaunchKernelGGL(row_reduce_kernel<kRowVar>, dim3(row_grid(rows)), dim3(kBlock), 0,
                     as_stream(stream), d_mat, d_mean, rows, cols, d_valid_lens, d_out_rows);
  return check_launch("row_variance_kernel");
}

int sufhip_unpack_eff_bits(const uint64_t* d_packed, int eff_bits, uint64_t* d_out, size_t n,
                           void* stream) {
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(eff_bits >= 1 && eff_bits <= 64, "sufhip_unpack_eff_bits: eff_bits in [1, 64]");
  SUFHIP_REQUIRE(d_packed && d_out, "sufhip_unpack_eff_bits: null pointer");
  hipLaunchKernelGGL(unpack_kernel, dim3(stream_grid(n)), dim3(kBlock), 0, as_stream(stream),
                     d_packed, eff_bits, packed_words(n, eff_bits), d_out, n);
  return check_launch("unpack_eff_bits_kernel");
}

int sufhip_pack_eff_bits(const uint64_t* d_in, int eff_bits, uint64_t* d_packed, size_t n,
                         void* stream) {
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(eff_bits >= 1 && eff_bits <= 64, "sufhip_pack_eff_bits: eff_bits in [1, 64]");
  SUFHIP_REQUIRE(d_in && d_packed, "sufhip_pack_eff_bits: null pointer");
  const size_t words = packed_words(n, eff_bits);
  hipLaunchKernelGGL(pack_kernel, dim3(stream_grid(words)), dim3(kBlock), 0, as_stream(stream),
                     d_in, eff_bits, d_packed, n, words);
  return check_launch("pack_eff_bits_kernel");
}

int sufhip_open_add_to_signed(const uint64_t* d_local_share, const uint64_t* d_remote_share,
                              uint64_t* d_out_signed, size_t n, int ring_bits, uint64_t ring_mask,
                              void* stream) {
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_local_share && d_remote_share && d_out_signed,
                 "sufhip_open_add_to_signed: null pointer");
  hipLaunchKernelGGL(open_add_kernel<true>, dim3(stream_grid(n)), dim3(kBlock), 0,
                     as_stream(stream), d_local_share, d_remote_share, 64, n, d_out_signed, n,
                     clamp_bits(ring_bits), ring_mask);
  return check_launch("open_add_to_signed_kernel");
}

int sufhip_unpack_add_to_signed(const uint64_t* d_local_share, const uint64_t* d_packed_remote,
                                int eff_bits, uint64_t* d_out_signed, size_t n, int ring_bits,
                                uint64_t ring_mask, void* stream) {
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_local_share && d_packed_remote && d_out_signed,
                 "sufhip_unpack_add_to_signed: null pointer");
  const int eb = clamp_bits(eff_bits);
  hipLaunchKernelGGL(open_add_kernel<true>, dim3(stream_grid(n)), dim3(kBlock), 0,
                     as_stream(stream), d_local_share, d_packed_remote, eb, packed_words(n, eb),
                     d_out_signed, n, clamp_bits(ring_bits), ring_mask);
  return check_launch("unpack_add_to_signed_kernel");
}

int sufhip_unpack_add_mod(const uint64_t* d_local_share, const uint64_t* d_packed_remote,
                          int eff_bits, uint64_t* d_out_mod, size_t n, int ring_bits,
                          uint64_t ring_mask, void* stream) {
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_local_share && d_packed_remote && d_out_mod,
                 "sufhip_unpack_add_mod: null pointer");
  const int eb = clamp_bits(eff_bits);
  hipLaunchKernelGGL(open_add_kernel<false>, dim3(stream_grid(n)), dim3(kBlock), 0,
                     as_stream(stream), d_local_share, d_packed_remote, eb, packed_words(n, eb),
                     d_out_mod, n, clamp_bits(ring_bits), ring_mask);
  return check_launch("unpack_add_mod_kernel");
}

}  // extern "C"
