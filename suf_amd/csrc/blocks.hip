// Row-local task blocks for two parties on one GPU, each in one launch.
//
// With both parties in one process every open is a local sum, so a task
// chain whose rounds only combine values of one row needs no grid-wide
// synchronisation: one workgroup runs all rounds of its row, holding the row
// in registers, with workgroup sums for the row reductions and one lane for
// the per-row scalar gates.  Element indices, triples and keys are those of
// the launch-per-step evaluation, so the shares are bit-identical to it.
//
//   layernorm2_kernel  LayerNormTask (include/runtime/phase_tasks.hpp:
//                      2186-2668) with RsqrtTask (:1383-1700)
#include <hip/hip_runtime.h>

#include "chain_device.hpp"
#include "reduce_device.hpp"

namespace sufhip {
namespace {

constexpr int kLnBlock = 256;
constexpr int kLnWaves = kLnBlock / 64;
constexpr int kLnMaxPer = 8;  // elements per thread: cols <= 2048
constexpr int kLnCopies = 4;  // the T table serves one lane per workgroup

struct LnArgs {
  const uint64_t* x[2];
  int rows, cols;
  uint64_t inv_len, eps;
  TruncEpi tr[4];  // mean, var0, var1, norm
  uint64_t mask[4];
  sufhip_triple2 sq, norm;
  ChainArgs rs;
  uint64_t* out[2];
};

enum { kTrMean = 0, kTrVar0 = 1, kTrVar1 = 2, kTrNorm = 3 };

// Every load that does not depend on an open is issued when the row starts:
// x, both triples' shares, and (lane 0) the rsqrt chain's triples; the key
// headers of all truncation gates sit in LDS.  What remains serial per row
// is one table read per truncation gate and the rsqrt LUT's AES.
template <int kPer>
__global__ void __launch_bounds__(kLnBlock) layernorm2_kernel(LnArgs A) {
  __shared__ __align__(16) uint32_t tab[256 * kLnCopies];
  __shared__ ChainLds L;
  __shared__ TruncHdr th[4][2];
  __shared__ uint64_t red[2][kLnWaves];
  __shared__ uint64_t bc[2];
  __shared__ ChainPre pre;
  fill_ttable<kLnCopies>(tab, kTDev.v);
  chain_stage(A.rs, 2, L);
  if (threadIdx.x < 8) th[threadIdx.x >> 1][threadIdx.x & 1] =
      read_trunc_hdr(A.tr[threadIdx.x >> 1].key[threadIdx.x & 1]);
  __syncthreads();
  const AesLds<kLnCopies> aes{tab, threadIdx.x % kLnCopies};
  const ChainKeyInfo K = chain_key_info(A.rs);
  auto gate = [&](int j, uint64_t v) {
    return Two{{trunc_table_eval_h(th[j][0], A.tr[j].table[0], A.tr[j].f, v),
                trunc_table_eval_h(th[j][1], A.tr[j].table[1], A.tr[j].f, v)}};
  };
  const int cols = A.cols;
  for (int r = blockIdx.x; r < A.rows; r += gridDim.x) {
    const size_t base = size_t(r) * size_t(cols);
    // The row's rsqrt triples, one word per lane (visible to lane 0 after
    // the row sum's barriers).
    if (threadIdx.x < 24) {
      const int k = threadIdx.x / 6, w = (threadIdx.x / 2) % 3, p = threadIdx.x & 1;
      const sufhip_term2& t = w == 0 ? A.rs.a[k] : (w == 1 ? A.rs.b[k] : A.rs.c[k]);
      const uint64_t v = term_at(t, p, size_t(r));
      (w == 0 ? pre.a : (w == 1 ? pre.b : pre.c))[k][p] = v;
    }
    // Loads in the order of use (x, the square's triple, the norm triple):
    // each step then waits only for its own words, and the norm triple's
    // arrive while lane 0 runs the rsqrt chain.
    uint64_t d[kPer][2], sa[kPer][2], sb[kPer][2], sc[kPer][2], na[kPer][2], nc[kPer][2];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int c = threadIdx.x + k * kLnBlock;
#pragma unroll
      for (int p = 0; p < 2; ++p) d[k][p] = c < cols ? A.x[p][base + c] : 0;
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int c = threadIdx.x + k * kLnBlock;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        sa[k][p] = c < cols ? A.sq.a[p][base + c] : 0;
        sb[k][p] = c < cols ? A.sq.b[p][base + c] : 0;
        sc[k][p] = c < cols ? A.sq.c[p][base + c] : 0;
      }
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int c = threadIdx.x + k * kLnBlock;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        na[k][p] = c < cols ? A.norm.a[p][base + c] : 0;
        nc[k][p] = c < cols ? A.norm.c[p][base + c] : 0;
      }
    }
    const uint64_t nb0 = A.norm.b[0][r], nb1 = A.norm.b[1][r];
    uint64_t s0 = 0, s1 = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      s0 += d[k][0];
      s1 += d[k][1];
    }
    // mu = tr_mean(inv_len * row sum).
    block_sum2_u64<kLnWaves>(s0, s1, red);
    const Two mu = gate(kTrMean, s0 * A.inv_len + s1 * A.inv_len + A.mask[kTrMean]);
    // d = x - mu; q = d * d (Beaver), summed over the row.
    uint64_t q0 = 0, q1 = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int c = threadIdx.x + k * kLnBlock;
      if (c < cols) {
        d[k][0] -= mu.v[0];
        d[k][1] -= mu.v[1];
        const uint64_t dd = (d[k][0] - sa[k][0]) + (d[k][1] - sa[k][1]);
        const uint64_t ee = (d[k][0] - sb[k][0]) + (d[k][1] - sb[k][1]);
        q0 += sc[k][0] + dd * sb[k][0] + ee * sa[k][0] + dd * ee;
        q1 += sc[k][1] + dd * sb[k][1] + ee * sa[k][1];
      }
    }
    block_sum2_u64<kLnWaves>(q0, q1, red);
    const Two va = gate(kTrVar0, q0 * A.inv_len + q1 * A.inv_len + A.mask[kTrVar0]);
    const Two var = gate(kTrVar1, va.v[0] + va.v[1] + A.mask[kTrVar1]);
    // rsqrt of the row's variance on one lane.
    if (threadIdx.x == 0) {
      const Two v{{var.v[0] + A.eps, var.v[1]}};
      const Two rs =
          chain_eval<SUFHIP_CHAIN_RSQRT, kLnCopies>(A.rs, L, K, aes, size_t(r), v, pre);
      bc[0] = rs.v[0];
      bc[1] = rs.v[1];
    }
    __syncthreads();
    // out = tr_norm(d * rs[row]) (row-broadcast Beaver).
    const uint64_t ee = (bc[0] - nb0) + (bc[1] - nb1);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int c = threadIdx.x + k * kLnBlock;
      if (c < cols) {
        const size_t i = base + c;
        const uint64_t dd = (d[k][0] - na[k][0]) + (d[k][1] - na[k][1]);
        const uint64_t z0 = nc[k][0] + dd * nb0 + ee * na[k][0] + dd * ee;
        const uint64_t z1 = nc[k][1] + dd * nb1 + ee * na[k][1];
        const Two o = gate(kTrNorm, z0 + z1 + A.mask[kTrNorm]);
        A.out[0][i] = o.v[0];
        A.out[1][i] = o.v[1];
      }
    }
    __syncthreads();  // bc is rewritten for the next row
  }
}

int triple_ok(const sufhip_triple2& t) {
  return t.a[0] && t.a[1] && t.b[0] && t.b[1] && t.c[0] && t.c[1];
}

int table_epi(const sufhip_trunc_epilogue& t, size_t n, const char* what, TruncEpi* e) {
  sufhip_trunc_epilogue c = t;
  uint64_t dummy = 0;
  c.y[0] = c.y[1] = &dummy;  // the block writes its own outputs
  return make_epi(&c, n, what, e);
}

}  // namespace
}  // namespace sufhip

using namespace sufhip;

extern "C" {

int sufhip_layernorm2(const sufhip_layernorm2_args* args, void* stream) {
  SUFHIP_REQUIRE(args != nullptr, "sufhip_layernorm2: null args");
  const sufhip_layernorm2_args& g = *args;
  SUFHIP_REQUIRE(g.rows >= 0 && g.cols >= 1 && g.cols <= kLnBlock * kLnMaxPer,
                 "sufhip_layernorm2: cols in [1, 2048]");
  if (g.rows == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(g.x[0] && g.x[1] && g.out[0] && g.out[1],
                 "sufhip_layernorm2: null input or output");
  SUFHIP_REQUIRE(triple_ok(g.sq) && triple_ok(g.norm), "sufhip_layernorm2: a triple is missing");
  SUFHIP_REQUIRE(g.rsqrt.kind == SUFHIP_CHAIN_RSQRT && g.rsqrt.n == size_t(g.rows),
                 "sufhip_layernorm2: the rsqrt chain must be RSQRT over rows elements");
  const size_t n = size_t(g.rows) * size_t(g.cols);
  LnArgs A{};
  if (int rc = make_chain_args(g.rsqrt, false, "sufhip_layernorm2 rsqrt", &A.rs)) return rc;
  if (int rc = table_epi(g.tr_mean, size_t(g.rows), "sufhip_layernorm2 tr_mean", &A.tr[kTrMean]))
    return rc;
  if (int rc = table_epi(g.tr_var[0], size_t(g.rows), "sufhip_layernorm2 tr_var", &A.tr[kTrVar0]))
    return rc;
  if (int rc = table_epi(g.tr_var[1], size_t(g.rows), "sufhip_layernorm2 tr_var", &A.tr[kTrVar1]))
    return rc;
  if (int rc = table_epi(g.tr_norm, n, "sufhip_layernorm2 tr_norm", &A.tr[kTrNorm])) return rc;
  A.x[0] = g.x[0];
  A.x[1] = g.x[1];
  A.rows = g.rows;
  A.cols = g.cols;
  A.inv_len = g.inv_len;
  A.eps = g.eps;
  A.mask[kTrMean] = g.mean_mask;
  A.mask[kTrVar0] = g.var_mask[0];
  A.mask[kTrVar1] = g.var_mask[1];
  A.mask[kTrNorm] = g.norm_mask;
  A.sq = g.sq;
  A.norm = g.norm;
  A.out[0] = g.out[0];
  A.out[1] = g.out[1];
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const int grid = g.rows < cus * 8 ? g.rows : cus * 8;
  const int per = (g.cols + kLnBlock - 1) / kLnBlock;
  hipStream_t s = as_stream(stream);
  if (per <= 1)
    hipLaunchKernelGGL(layernorm2_kernel<1>, dim3(grid), dim3(kLnBlock), 0, s, A);
  else if (per <= 2)
    hipLaunchKernelGGL(layernorm2_kernel<2>, dim3(grid), dim3(kLnBlock), 0, s, A);
  else if (per <= 4)
    hipLaunchKernelGGL(layernorm2_kernel<4>, dim3(grid), dim3(kLnBlock), 0, s, A);
  else
    hipLaunchKernelGGL(layernorm2_kernel<kLnMaxPer>, dim3(grid), dim3(kLnBlock), 0, s, A);
  return check_launch("layernorm2_kernel");
}

}  // extern "C"
