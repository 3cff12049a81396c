// Beaver matrix product over Z_2^64 (cuda/cuda_primitives.cu:391-628):
//   out = C + D*B + A*E (+ D*E for party 0), optionally (out * c) >> s on the
//   signed 128-bit product, with D = X - A and E = W - B opened.
//
// Restated as one GEMM over a concatenated inner dimension of length 2K:
//   out = C + [D | A] * [B' ; E],   B' = B + E (party 0) or B (party 1),
// so each output costs 2K multiply-adds.  CDNA4 has no 64-bit integer
// multiply; a*b mod 2^64 = lo(a)lo(b) + 2^32 (lo(a)hi(b) + hi(a)lo(b)), so each
// lane keeps a 64-bit accumulator for lo*lo (v_mad_u64_u32) and a 32-bit one
// for the two cross terms, combined once at the end.
//
// Tiling: a 256-thread workgroup computes a 32 x 64 output tile; each lane
// owns 2 rows x 4 columns.  Per k-step of 16 the workgroup stages the LHS tile
// transposed ([k][m], so a lane's two rows are one 16-byte LDS read) and the
// RHS tile ([k][n], a lane's four columns are two 16-byte reads), with B + E
// folded in while staging.  Batched launches put the batch in grid.z and
// reuse the same A, B, C for every batch instance (cuda_primitives.hpp:149-150);
// the two-party form puts (batch, party) in grid.z with one triple per batch.
#include <hip/hip_runtime.h>

#include "sufhip_internal.hpp"

namespace sufhip {
namespace {

constexpr int BM = 32, BN = 64, BK = 16;
constexpr int kMmThreads = 256;  // 16 x 16 lanes, 2 x 4 outputs each

struct MmArgs {
  const uint64_t* D;
  const uint64_t* E;
  const uint64_t* A;
  const uint64_t* B;
  const uint64_t* C;
  uint64_t* out;
  int M, K, N;
  int party;
  int has_scale;
  int64_t mul_const;
  int mul_shift;
  // Two-party form: grid.z = 2 * batch + party; each party's triple shares
  // and output, one triple per batch instance ([b][M][K], [b][K][N],
  // [b][M][N]).  A, B, C, out and party above are unused then.
  int two_party;
  const uint64_t* A2[2];
  const uint64_t* B2[2];
  const uint64_t* C2[2];
  uint64_t* out2[2];
  // Two-party form with ksplit > 1: grid.z = (2 * batch + party) * ksplit +
  // slice; slice s sums its share of the 2K inner dimension into
  // part[s][party][batch] (no C), and reduce2_kernel adds C and the slices.
  int ksplit;
  uint64_t* part;
  int batches;
};

__device__ __forceinline__ uint64_t scaled(uint64_t acc, const MmArgs& a) {
  if (!a.has_scale) return acc;
  const int64_t s = static_cast<int64_t>(acc);
  const uint64_t lo = uint64_t(s) * uint64_t(a.mul_const);
  if (a.mul_shift <= 0) return lo;
  const int64_t hi = __mul64hi(s, a.mul_const);
  if (a.mul_shift >= 64) {
    const int sh = a.mul_shift - 64;
    return uint64_t(sh >= 64 ? (hi >> 63) : (hi >> sh));
  }
  return (lo >> a.mul_shift) | (uint64_t(hi) << (64 - a.mul_shift));
}

template <bool kTrans>
__global__ void __launch_bounds__(kMmThreads) beaver_matmul_kernel(MmArgs a) {
  __shared__ uint64_t sL[BK][BM];  // [k][m]
  __shared__ uint64_t sR[BK][BN];  // [k][n]
  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int M = a.M, K = a.K, N = a.N;
  const int ks = a.two_party ? a.ksplit : 1;
  const int slice = int(blockIdx.z) % ks;
  const int bz = int(blockIdx.z) / ks;
  const int party = a.two_party ? (bz & 1) : a.party;
  const size_t b = a.two_party ? size_t(bz >> 1) : blockIdx.z;
  const uint64_t* D = a.D + b * size_t(M) * K;
  const uint64_t* E = a.E + b * size_t(K) * N;
  // Triple shares and output of this (batch, party): shared by every batch
  // in the one-party form (cuda_primitives.hpp:149-150), per batch otherwise.
  const uint64_t* TA = a.two_party ? a.A2[party] + b * size_t(M) * K : a.A;
  const uint64_t* TB = a.two_party ? a.B2[party] + b * size_t(K) * N : a.B;
  const uint64_t* TC = a.two_party ? a.C2[party] + b * size_t(M) * N : a.C;
  uint64_t* OUT = a.two_party ? a.out2[party] + b * size_t(M) * N : a.out + b * size_t(M) * N;
  const bool p0 = party == 0;

  uint64_t acc[2][4];
  uint32_t hi[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[i][j] = 0;
      hi[i][j] = 0;
    }

  const int K2 = 2 * K;
  const int steps = (K2 + BK - 1) / BK;
  const int k_first = BK * (steps * slice / ks), k_last = BK * (steps * (slice + 1) / ks);
  for (int k0 = k_first; k0 < k_last; k0 += BK) {
    // LHS tile: 32 rows x 16 k = 512 values, 2 per lane.  k < K reads D, else A.
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int idx = tid + r * kMmThreads;
      const int mm = idx >> 4, kk = idx & 15;
      const int gm = m0 + mm, gk = k0 + kk;
      uint64_t v = 0;
      if (gm < M && gk < K2) v = gk < K ? D[size_t(gm) * K + gk] : TA[size_t(gm) * K + (gk - K)];
      sL[kk][mm] = v;
    }
    // RHS tile: 16 k x 64 n = 1024 values, 4 per lane.  k < K: B (+E for party 0), else E.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int idx = tid + r * kMmThreads;
      int kk, nn;
      if (kTrans) {  // [N][K] storage: consecutive lanes walk k for one n
        nn = idx >> 4;
        kk = idx & 15;
      } else {
        kk = idx >> 6;
        nn = idx & 63;
      }
      const int gk = k0 + kk, gn = n0 + nn;
      uint64_t v = 0;
      if (gn < N && gk < K2) {
        const int kr = gk < K ? gk : gk - K;
        const size_t off = kTrans ? size_t(gn) * K + kr : size_t(kr) * N + gn;
        if (gk < K) {
          v = TB[off];
          if (p0) v += E[off];
        } else {
          v = E[off];
        }
      }
      sR[kk][nn] = v;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK; ++kk) {
      const uint64_t l0 = sL[kk][2 * ty], l1 = sL[kk][2 * ty + 1];
      const uint64_t lv[2] = {l0, l1};
      uint64_t rv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) rv[j] = sR[kk][4 * tx + j];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t alo = uint32_t(lv[i]), ahi = uint32_t(lv[i] >> 32);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t blo = uint32_t(rv[j]), bhi = uint32_t(rv[j] >> 32);
          acc[i][j] += uint64_t(alo) * blo;
          hi[i][j] += alo * bhi + ahi * blo;
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int gm = m0 + 2 * ty + i;
    if (gm >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int gn = n0 + 4 * tx + j;
      if (gn >= N) continue;
      const size_t o = size_t(gm) * N + gn;
      if (ks > 1) {
        a.part[((size_t(slice) * 2 + party) * a.batches + b) * size_t(M) * N + o] =
            acc[i][j] + (uint64_t(hi[i][j]) << 32);
        continue;
      }
      const uint64_t v = TC[o] + acc[i][j] + (uint64_t(hi[i][j]) << 32);
      OUT[o] = scaled(v, a);
    }
  }
}

// out_p = C_p + sum over slices of part[slice][p] (two-party k-split).
__global__ void __launch_bounds__(256)
    reduce2_kernel(const uint64_t* part, int ksplit, size_t per_party, const uint64_t* C0,
                   const uint64_t* C1, uint64_t* out0, uint64_t* out1) {
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < 2 * per_party;
       i += size_t(gridDim.x) * 256) {
    const int p = i < per_party ? 0 : 1;
    const size_t j = i - size_t(p) * per_party;
    uint64_t v = p == 0 ? C0[j] : C1[j];
    for (int s = 0; s < ksplit; ++s) v += part[(size_t(s) * 2 + p) * per_party + j];
    (p == 0 ? out0 : out1)[j] = v;
  }
}

// Slices of the 2K inner dimension for the two-party form: about 512
// workgroups per launch, at most 8 slices, at least one 16-deep step each.
int ksplit_for(int batches, int M, int K, int N) {
  const long base = long((N + BN - 1) / BN) * ((M + BM - 1) / BM) * 2 * batches;
  const int steps = (2 * K + BK - 1) / BK;
  long s = base >= 512 ? 1 : (512 + base - 1) / base;
  if (s > 8) s = 8;
  if (s > steps) s = steps;
  return int(s);
}

int launch(int party, const uint64_t* D, const uint64_t* E, const uint64_t* A, const uint64_t* B,
           const uint64_t* C, int batches, int M, int K, int N, int w_transposed, int has_scale,
           int64_t mul_const, int mul_shift, uint64_t* out, void* stream) {
  if (batches <= 0 || M <= 0 || K <= 0 || N <= 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(D && E && A && B && C && out, "sufhip_beaver_matmul2d: null pointer");
  SUFHIP_REQUIRE(batches <= 65535, "sufhip_beaver_matmul2d: at most 65535 batches");
  SUFHIP_REQUIRE(size_t(K) * 2 < (size_t(1) << 31), "sufhip_beaver_matmul2d: K too large");
  MmArgs a{D, E, A, B, C, out, M, K, N, party, has_scale, mul_const, mul_shift, 0,
           {nullptr, nullptr}, {nullptr, nullptr}, {nullptr, nullptr}, {nullptr, nullptr},
           1, nullptr, batches};
  const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM, batches), block(kMmThreads);
  if (w_transposed)
    hipLaunchKernelGGL(beaver_matmul_kernel<true>, grid, block, 0, as_stream(stream), a);
  else
    hipLaunchKernelGGL(beaver_matmul_kernel<false>, grid, block, 0, as_stream(stream), a);
  return check_launch("beaver_matmul_kernel");
}

size_t work2_bytes(int batches, int M, int K, int N) {
  if (batches <= 0 || M <= 0 || K <= 0 || N <= 0) return 0;
  const int ks = ksplit_for(batches, M, K, N);
  return ks > 1 ? size_t(ks) * 2 * size_t(batches) * M * N * 8 : 0;
}

int launch2(const uint64_t* D, const uint64_t* E, const uint64_t* A0, const uint64_t* A1,
            const uint64_t* B0, const uint64_t* B1, const uint64_t* C0, const uint64_t* C1,
            int batches, int M, int K, int N, uint64_t* out0, uint64_t* out1, void* work,
            size_t work_bytes, void* stream) {
  if (batches <= 0 || M <= 0 || K <= 0 || N <= 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(D && E && A0 && A1 && B0 && B1 && C0 && C1 && out0 && out1,
                 "sufhip_beaver_matmul2_batched: null pointer");
  SUFHIP_REQUIRE(batches <= 4095, "sufhip_beaver_matmul2_batched: at most 4095 batches");
  SUFHIP_REQUIRE(size_t(K) * 2 < (size_t(1) << 31), "sufhip_beaver_matmul2_batched: K too large");
  const int ks = ksplit_for(batches, M, K, N);
  const size_t need = work2_bytes(batches, M, K, N);
  SUFHIP_REQUIRE(work_bytes >= need && (need == 0 || work),
                 "sufhip_beaver_matmul2_batched: workspace smaller than its work bytes");
  MmArgs a{D, E, nullptr, nullptr, nullptr, nullptr, M, K, N, 0, 0, 0, 0, 1,
           {A0, A1}, {B0, B1}, {C0, C1}, {out0, out1}, ks, static_cast<uint64_t*>(work),
           batches};
  const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM, 2 * batches * ks), block(kMmThreads);
  hipLaunchKernelGGL(beaver_matmul_kernel<false>, grid, block, 0, as_stream(stream), a);
  if (int rc = check_launch("beaver_matmul_kernel (two-party)")) return rc;
  if (ks == 1) return SUFHIP_OK;
  const size_t per_party = size_t(batches) * M * N;
  size_t g = (2 * per_party + 255) / 256;
  if (g > 4096) g = 4096;
  hipLaunchKernelGGL(reduce2_kernel, dim3(unsigned(g)), dim3(256), 0, as_stream(stream),
                     static_cast<const uint64_t*>(work), ks, per_party, C0, C1, out0, out1);
  return check_launch("reduce2_kernel");
}

}  // namespace
}  // namespace sufhip

using namespace sufhip;

extern "C" {

int sufhip_beaver_matmul2d(int party, const uint64_t* d_D_open, const uint64_t* d_E_open,
                           const uint64_t* d_A_tri_share, const uint64_t* d_B_tri_share,
                           const uint64_t* d_C_tri_share, int M, int K, int N, int w_transposed,
                           int has_scale, int64_t mul_const, int mul_shift, uint64_t* d_out,
                           void* stream) {
  return launch(party, d_D_open, d_E_open, d_A_tri_share, d_B_tri_share, d_C_tri_share, 1, M, K, N,
                w_transposed, has_scale, mul_const, mul_shift, d_out, stream);
}

int sufhip_beaver_matmul2d_batched(int party, const uint64_t* d_D_open, const uint64_t* d_E_open,
                                   const uint64_t* d_A_tri_share, const uint64_t* d_B_tri_share,
                                   const uint64_t* d_C_tri_share, int batches, int M, int K, int N,
                                   int w_transposed, int has_scale, int64_t mul_const,
                                   int mul_shift, uint64_t* d_out, void* stream) {
  return launch(party, d_D_open, d_E_open, d_A_tri_share, d_B_tri_share, d_C_tri_share, batches, M,
                K, N, w_transposed, has_scale, mul_const, mul_shift, d_out, stream);
}

size_t sufhip_beaver_matmul2_batched_work_bytes(int batches, int M, int K, int N) {
  return work2_bytes(batches, M, K, N);
}

int sufhip_beaver_matmul2_batched(const uint64_t* d_D_open, const uint64_t* d_E_open,
                                   const uint64_t* d_A0, const uint64_t* d_A1,
                                   const uint64_t* d_B0, const uint64_t* d_B1,
                                   const uint64_t* d_C0, const uint64_t* d_C1, int batches, int M,
                                   int K, int N, uint64_t* d_out0, uint64_t* d_out1, void* d_work,
                                   size_t work_bytes, void* stream) {
  return launch2(d_D_open, d_E_open, d_A0, d_A1, d_B0, d_B1, d_C0, d_C1, batches, M, K, N, d_out0,
                 d_out1, d_work, work_bytes, stream);
}

}  // extern "C"
