// Two-party step kernels for gate pipelines whose two parties share one GPU
// (the reference's local channel: both parties in one process, each "open"
// an exchange of masked shares followed by an add).  Each kernel does the
// local work of both parties for one protocol round plus the open, in one
// pass over HBM:
//   open2_masked  x^ = (x_0 + r_0) + (x_1 + r_1)          (a gate's masked open)
//   open2_diff    d = (x_0 - a_0) + (x_1 - a_1)            (a Beaver open, e.g. D, E
//                 of the Beaver matmul)
//   mul2          Beaver product of MulTask (include/runtime/phase_tasks.hpp:
//                 198-402) with the d/e open inline, optional pre-add on the
//                 left factor and post-add on the product (the affine steps
//                 of CubicPolyTask, phase_tasks.hpp:2962-3061), and optional
//                 masked open of the product for the next gate
//   add_shifted   y + (a << s), strided a (coefficient words of an AoS row)
//   lin2          a general operand (sum of up to two strided / row-indexed,
//                 shifted, signed terms plus a public constant on party 0's
//                 share) for both parties, and/or its masked open
//   mul2x         the Beaver product of two general operands, with the
//                 row-broadcast triple of MulRowBroadcastTask (phase_tasks.hpp:
//                 1810-2185) when b is row-indexed
//   row_sum2      per-row sums of a general operand for both parties, scaled
//                 by a public constant, and/or their masked open (the mean /
//                 variance / softmax-denominator steps of LayerNormTask and
//                 SoftmaxBlockTask)
// All arithmetic is mod 2^64; per party the Beaver step is exactly
// z_p = c_p + d*b_p + e*a_p + [p == 0] d*e (beaver_mul_kernel,
// cuda/cuda_primitives.cu:114-139).
#include <hip/hip_runtime.h>

#include <string>

#include "suf_hip.h"
#include "sufhip_internal.hpp"
#include "operand_device.hpp"
#include "digit_planes.hpp"
#include "reduce_device.hpp"
#include "trunc_device.hpp"

namespace sufhip {
namespace {

constexpr int kBlock = 256;
constexpr size_t kMaxElems = size_t(1) << 40;

unsigned int ew_grid(size_t n) {
  size_t g = (n + kBlock - 1) / kBlock;
  return unsigned(g > 8192 ? 8192 : g);
}

__global__ void __launch_bounds__(kBlock)
    open2_masked_kernel(const uint64_t* x0, const uint64_t* x1, uint64_t r, size_t n,
                        uint64_t* xhat) {
  const size_t stride = size_t(gridDim.x) * kBlock;
  for (size_t i = size_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
    xhat[i] = x0[i] + x1[i] + r;
}

__global__ void __launch_bounds__(kBlock)
    open2_diff_kernel(const uint64_t* x0, const uint64_t* x1, const uint64_t* a0,
                      const uint64_t* a1, size_t n, uint64_t* d) {
  const size_t stride = size_t(gridDim.x) * kBlock;
  for (size_t i = size_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
    d[i] = (x0[i] - a0[i]) + (x1[i] - a1[i]);
}

__global__ void __launch_bounds__(kBlock) mul2_kernel(sufhip_mul2_args a, size_t n) {
  const size_t stride = size_t(gridDim.x) * kBlock;
  const bool has_uadd = a.u_add[0] != nullptr;
  const bool has_zadd = a.z_add[0] != nullptr;
  const bool open = a.zhat != nullptr;
  const uint64_t mask = a.open_mask[0] + a.open_mask[1];
  for (size_t i = size_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
    uint64_t u0 = a.u[0][i * a.u_stride + a.u_off];
    uint64_t u1 = a.u[1][i * a.u_stride + a.u_off];
    if (has_uadd) {
      u0 += a.u_add[0][i * a.u_add_stride + a.u_add_off] << a.u_add_shift;
      u1 += a.u_add[1][i * a.u_add_stride + a.u_add_off] << a.u_add_shift;
    }
    const uint64_t v0 = a.v[0][i], v1 = a.v[1][i];
    const uint64_t* t0 = a.triples[0] + 3 * i;
    const uint64_t* t1 = a.triples[1] + 3 * i;
    const uint64_t a0 = t0[0], b0 = t0[1], c0 = t0[2];
    const uint64_t a1 = t1[0], b1 = t1[1], c1 = t1[2];
    // The open: each party's masked shares, summed.
    const uint64_t d = (u0 - a0) + (u1 - a1);
    const uint64_t e = (v0 - b0) + (v1 - b1);
    uint64_t z0 = c0 + d * b0 + e * a0 + d * e;
    uint64_t z1 = c1 + d * b1 + e * a1;
    if (has_zadd) {
      z0 += a.z_add[0][i * a.z_add_stride + a.z_add_off] << a.z_add_shift;
      z1 += a.z_add[1][i * a.z_add_stride + a.z_add_off] << a.z_add_shift;
    }
    if (open) {
      a.zhat[i] = z0 + z1 + mask;
    } else {
      a.z[0][i] = z0;
      a.z[1][i] = z1;
    }
  }
}

__global__ void __launch_bounds__(kBlock)
    add_shifted_kernel(const uint64_t* y, const uint64_t* add, size_t stride_a, size_t off,
                       int shift, size_t n, uint64_t* out) {
  const size_t stride = size_t(gridDim.x) * kBlock;
  for (size_t i = size_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
    out[i] = y[i] + (add[i * stride_a + off] << shift);
}

__global__ void __launch_bounds__(kBlock)
    lin2_kernel(sufhip_operand2 x, size_t n, uint64_t* out0, uint64_t* out1, uint64_t* xhat,
                uint64_t mask, TruncEpi epi) {
  const size_t stride = size_t(gridDim.x) * kBlock;
  const EpiHdrs eh = epi_hdrs(epi);
  for (size_t i = size_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
    const uint64_t x0 = operand_at(x, 0, i), x1 = operand_at(x, 1, i);
    if (out0) out0[i] = x0;
    if (out1) out1[i] = x1;
    put_open(epi, eh, xhat, i, x0 + x1 + mask);
  }
}

constexpr int kLin2Jobs = 4;

struct Lin2Batch {
  sufhip_operand2 x[kLin2Jobs];
  size_t n[kLin2Jobs];
  uint64_t* out[kLin2Jobs][2];
  uint64_t* xhat[kLin2Jobs];
  uint64_t mask[kLin2Jobs];
  TruncEpi epi[kLin2Jobs];
  sufhip_kb_planes kb[kLin2Jobs];
  unsigned begin[kLin2Jobs + 1];  // each job's first workgroup
  int count;
};

// Workgroups [begin[j], begin[j + 1]) grid-stride over job j's elements.
__global__ void __launch_bounds__(kBlock) lin2_batch_kernel(Lin2Batch b) {
  int j = 0;
  while (j + 1 < b.count && blockIdx.x >= b.begin[j + 1]) ++j;
  const unsigned groups = b.begin[j + 1] - b.begin[j];
  const size_t stride = size_t(groups) * kBlock;
  const EpiHdrs eh = epi_hdrs(b.epi[j]);
  for (size_t i = size_t(blockIdx.x - b.begin[j]) * kBlock + threadIdx.x; i < b.n[j];
       i += stride) {
    const uint64_t x0 = operand_at(b.x[j], 0, i), x1 = operand_at(b.x[j], 1, i);
    if (b.out[j][0]) b.out[j][0][i] = x0;
    if (b.out[j][1]) b.out[j][1][i] = x1;
    put_open(b.epi[j], eh, b.xhat[j], i, x0 + x1 + b.mask[j]);
    if (b.kb[j].planes) put_kb_digits(b.kb[j], i, x0 + x1 + b.mask[j]);
  }
}

__global__ void __launch_bounds__(kBlock) mul2x_kernel(sufhip_mul2x_args a, size_t n, TruncEpi epi) {
  const size_t stride = size_t(gridDim.x) * kBlock;
  const bool open = a.zhat != nullptr || epi.on;
  for (size_t i = size_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
    const uint64_t u0 = operand_at(a.u, 0, i), u1 = operand_at(a.u, 1, i);
    const uint64_t v0 = operand_at(a.v, 0, i), v1 = operand_at(a.v, 1, i);
    const uint64_t a0 = term_at(a.a, 0, i), a1 = term_at(a.a, 1, i);
    const uint64_t b0 = term_at(a.b, 0, i), b1 = term_at(a.b, 1, i);
    const uint64_t c0 = term_at(a.c, 0, i), c1 = term_at(a.c, 1, i);
    // The open: each party's masked shares, summed.
    const uint64_t d = (u0 - a0) + (u1 - a1);
    const uint64_t e = (v0 - b0) + (v1 - b1);
    const uint64_t z0 = c0 + d * b0 + e * a0 + d * e + operand_at(a.z_add, 0, i);
    const uint64_t z1 = c1 + d * b1 + e * a1 + operand_at(a.z_add, 1, i);
    if (open) {
      // Headers read per element: hoisted, they would join the operands'
      // wave-uniform registers and spill them.
      put_open(epi, epi_hdrs(epi), a.zhat, i, z0 + z1 + a.open_mask);
    } else {
      a.z[0][i] = z0;
      a.z[1][i] = z1;
    }
  }
}

// One wave per row, four rows per workgroup.
__global__ void __launch_bounds__(kBlock)
    row_sum2_kernel(sufhip_operand2 x, int rows, int cols, const int32_t* offs,
                    uint64_t mul_const, uint64_t* sum0, uint64_t* sum1, uint64_t* hat,
                    uint64_t mask, TruncEpi epi) {
  const int lane = threadIdx.x & 63;
  const EpiHdrs eh = epi_hdrs(epi);
  for (int r = blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6); r < rows;
       r += gridDim.x * (kBlock / 64)) {
    const size_t b = offs ? size_t(offs[r]) : size_t(r) * size_t(cols);
    const size_t e = offs ? size_t(offs[r + 1]) : b + size_t(cols);
    uint64_t s0 = 0, s1 = 0;
    for (size_t i = b + lane; i < e; i += 64) {
      s0 += operand_at(x, 0, i);
      s1 += operand_at(x, 1, i);
    }
    s0 = wave_sum_u64(s0) * mul_const;
    s1 = wave_sum_u64(s1) * mul_const;
    if (lane == 0) {
      if (sum0) sum0[r] = s0;
      if (sum1) sum1[r] = s1;
      put_open(epi, eh, hat, size_t(r), s0 + s1 + mask);
    }
  }
}

}  // namespace
}  // namespace sufhip

using namespace sufhip;

extern "C" {

int sufhip_open2_masked(const uint64_t* d_x0, const uint64_t* d_x1, uint64_t r0, uint64_t r1,
                        size_t n, uint64_t* d_xhat, void* stream) {
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(n < kMaxElems, "sufhip_open2_masked: n too large");
  SUFHIP_REQUIRE(d_x0 && d_x1 && d_xhat, "sufhip_open2_masked: null pointer");
  hipLaunchKernelGGL(open2_masked_kernel, dim3(ew_grid(n)), dim3(kBlock), 0, as_stream(stream),
                     d_x0, d_x1, r0 + r1, n, d_xhat);
  return check_launch("open2_masked_kernel");
}

int sufhip_open2_diff(const uint64_t* d_x0, const uint64_t* d_x1, const uint64_t* d_a0,
                      const uint64_t* d_a1, size_t n, uint64_t* d_open, void* stream) {
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(n < kMaxElems, "sufhip_open2_diff: n too large");
  SUFHIP_REQUIRE(d_x0 && d_x1 && d_a0 && d_a1 && d_open, "sufhip_open2_diff: null pointer");
  hipLaunchKernelGGL(open2_diff_kernel, dim3(ew_grid(n)), dim3(kBlock), 0, as_stream(stream),
                     d_x0, d_x1, d_a0, d_a1, n, d_open);
  return check_launch("open2_diff_kernel");
}

int sufhip_mul2(const sufhip_mul2_args* args, size_t n, void* stream) {
  SUFHIP_REQUIRE(args != nullptr, "sufhip_mul2: null args");
  if (n == 0) return SUFHIP_OK;
  const sufhip_mul2_args& a = *args;
  SUFHIP_REQUIRE(n < kMaxElems, "sufhip_mul2: n too large");
  SUFHIP_REQUIRE(a.u[0] && a.u[1] && a.v[0] && a.v[1] && a.triples[0] && a.triples[1],
                 "sufhip_mul2: null factor or triple pointer");
  SUFHIP_REQUIRE(a.u_stride >= 1 && a.u_off < a.u_stride, "sufhip_mul2: bad u stride/offset");
  SUFHIP_REQUIRE((a.u_add[0] == nullptr) == (a.u_add[1] == nullptr),
                 "sufhip_mul2: u_add must be given for both parties or neither");
  if (a.u_add[0])
    SUFHIP_REQUIRE(a.u_add_stride >= 1 && a.u_add_off < a.u_add_stride && a.u_add_shift >= 0 &&
                       a.u_add_shift < 64,
                   "sufhip_mul2: bad u_add stride/offset/shift");
  SUFHIP_REQUIRE((a.z_add[0] == nullptr) == (a.z_add[1] == nullptr),
                 "sufhip_mul2: z_add must be given for both parties or neither");
  if (a.z_add[0])
    SUFHIP_REQUIRE(a.z_add_stride >= 1 && a.z_add_off < a.z_add_stride && a.z_add_shift >= 0 &&
                       a.z_add_shift < 64,
                   "sufhip_mul2: bad z_add stride/offset/shift");
  SUFHIP_REQUIRE(a.zhat != nullptr || (a.z[0] && a.z[1]),
                 "sufhip_mul2: need zhat (open) or both z outputs");
  hipLaunchKernelGGL(mul2_kernel, dim3(ew_grid(n)), dim3(kBlock), 0, as_stream(stream), a, n);
  return check_launch("mul2_kernel");
}

int sufhip_add_shifted(const uint64_t* d_y, const uint64_t* d_add, size_t add_stride,
                       size_t add_off, int shift, size_t n, uint64_t* d_out, void* stream) {
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(n < kMaxElems, "sufhip_add_shifted: n too large");
  SUFHIP_REQUIRE(d_y && d_add && d_out, "sufhip_add_shifted: null pointer");
  SUFHIP_REQUIRE(add_stride >= 1 && add_off < add_stride && shift >= 0 && shift < 64,
                 "sufhip_add_shifted: bad stride/offset/shift");
  hipLaunchKernelGGL(add_shifted_kernel, dim3(ew_grid(n)), dim3(kBlock), 0, as_stream(stream),
                     d_y, d_add, add_stride, add_off, shift, n, d_out);
  return check_launch("add_shifted_kernel");
}

int sufhip_lin2(const sufhip_operand2* x, size_t n, uint64_t* d_out0, uint64_t* d_out1,
                uint64_t* d_xhat, uint64_t mask, const sufhip_trunc_epilogue* trunc,
                void* stream) {
  SUFHIP_REQUIRE(x != nullptr, "sufhip_lin2: null operand");
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(n < kMaxElems, "sufhip_lin2: n too large");
  SUFHIP_REQUIRE(d_out0 || d_out1 || d_xhat || trunc, "sufhip_lin2: no output");
  if (int rc = check_operand(*x, n, "sufhip_lin2")) return rc;
  TruncEpi epi;
  if (int rc = make_epi(trunc, n, "sufhip_lin2", &epi)) return rc;
  hipLaunchKernelGGL(lin2_kernel, dim3(ew_grid(n)), dim3(kBlock), 0, as_stream(stream), *x, n,
                     d_out0, d_out1, d_xhat, mask, epi);
  return check_launch("lin2_kernel");
}

int sufhip_lin2_batch(const sufhip_lin2_job* jobs, int count, void* stream) {
  SUFHIP_REQUIRE(count >= 0 && count <= kLin2Jobs && (count == 0 || jobs),
                 "sufhip_lin2_batch: 0..4 jobs");
  Lin2Batch b{};
  b.begin[0] = 0;
  for (int k = 0; k < count; ++k) {
    const sufhip_lin2_job& jb = jobs[k];
    if (jb.n == 0) continue;
    SUFHIP_REQUIRE(jb.n < kMaxElems, "sufhip_lin2_batch: n too large");
    SUFHIP_REQUIRE(jb.out[0] || jb.out[1] || jb.xhat || jb.trunc || jb.xhat_planes.planes,
                   "sufhip_lin2_batch: no output");
    SUFHIP_REQUIRE(kb_planes_ok(jb.xhat_planes, jb.n),
                   "sufhip_lin2_batch: xhat_planes must cover n = batches rows cols, rows and "
                   "cols multiples of 32, 16-byte aligned");
    if (int rc = check_operand(jb.x, jb.n, "sufhip_lin2_batch")) return rc;
    const int c = b.count;
    if (int rc = make_epi(jb.trunc, jb.n, "sufhip_lin2_batch", &b.epi[c])) return rc;
    b.x[c] = jb.x;
    b.n[c] = jb.n;
    b.out[c][0] = jb.out[0];
    b.out[c][1] = jb.out[1];
    b.xhat[c] = jb.xhat;
    b.mask[c] = jb.mask;
    b.kb[c] = jb.xhat_planes;
    b.begin[c + 1] = b.begin[c] + ew_grid(jb.n);
    ++b.count;
  }
  if (b.count == 0) return SUFHIP_OK;
  hipLaunchKernelGGL(lin2_batch_kernel, dim3(b.begin[b.count]), dim3(kBlock), 0,
                     as_stream(stream), b);
  return check_launch("lin2_batch_kernel");
}

int sufhip_mul2x(const sufhip_mul2x_args* args, size_t n, void* stream) {
  SUFHIP_REQUIRE(args != nullptr, "sufhip_mul2x: null args");
  if (n == 0) return SUFHIP_OK;
  const sufhip_mul2x_args& a = *args;
  SUFHIP_REQUIRE(n < kMaxElems, "sufhip_mul2x: n too large");
  if (int rc = check_operand(a.u, n, "sufhip_mul2x u")) return rc;
  if (int rc = check_operand(a.v, n, "sufhip_mul2x v")) return rc;
  if (int rc = check_operand(a.z_add, n, "sufhip_mul2x z_add")) return rc;
  SUFHIP_REQUIRE(a.a.p[0] && a.b.p[0] && a.c.p[0], "sufhip_mul2x: triple shares missing");
  if (int rc = check_term(a.a, n, false, "sufhip_mul2x a")) return rc;
  if (int rc = check_term(a.b, n, false, "sufhip_mul2x b")) return rc;
  if (int rc = check_term(a.c, n, false, "sufhip_mul2x c")) return rc;
  SUFHIP_REQUIRE(a.zhat != nullptr || a.trunc != nullptr || (a.z[0] && a.z[1]),
                 "sufhip_mul2x: need zhat (open), a truncation epilogue or both z outputs");
  TruncEpi epi;
  if (int rc = make_epi(a.trunc, n, "sufhip_mul2x", &epi)) return rc;
  hipLaunchKernelGGL(mul2x_kernel, dim3(ew_grid(n)), dim3(kBlock), 0, as_stream(stream), a, n,
                     epi);
  return check_launch("mul2x_kernel");
}

int sufhip_row_sum2(const sufhip_operand2* x, int rows, int cols, const int32_t* d_row_offsets,
                    uint64_t mul_const, uint64_t* d_sum0, uint64_t* d_sum1, uint64_t* d_hat,
                    uint64_t mask, const sufhip_trunc_epilogue* trunc, void* stream) {
  SUFHIP_REQUIRE(x != nullptr, "sufhip_row_sum2: null operand");
  SUFHIP_REQUIRE(rows >= 0 && (d_row_offsets || cols >= 0), "sufhip_row_sum2: bad shape");
  if (rows == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_sum0 || d_sum1 || d_hat || trunc, "sufhip_row_sum2: no output");
  TruncEpi epi;
  if (int rc = make_epi(trunc, size_t(rows), "sufhip_row_sum2", &epi)) return rc;
  // Without offsets every element index is < rows * cols; with offsets the
  // caller's offsets bound them (indexed terms clamp on the device).
  const size_t n = d_row_offsets ? 0 : size_t(rows) * size_t(cols);
  if (int rc = check_operand(*x, n, "sufhip_row_sum2")) return rc;
  size_t g = (size_t(rows) + kBlock / 64 - 1) / (kBlock / 64);
  if (g > 8192) g = 8192;
  hipLaunchKernelGGL(row_sum2_kernel, dim3(unsigned(g)), dim3(kBlock), 0, as_stream(stream), *x,
                     rows, cols, d_row_offsets, mul_const, d_sum0, d_sum1, d_hat, mask, epi);
  return check_launch("row_sum2_kernel");
}

}  // extern "C"
