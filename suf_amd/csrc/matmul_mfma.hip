// Beaver matrix product over Z_2^64 on the int8 matrix cores (gfx950
// v_mfma_i32_32x32x32_i8), exact.
//
// Same product as beaver_matmul_kernel (launch_beaver_matmul2d_kernel,
// cuda/cuda_primitives.cu:391-506): out = C + [D | A] * [B' ; E] over a 2K
// inner dimension, B' = B + E for party 0.  Every u64 operand is written in
// balanced base-256 digits, v = sum_i d_i 256^i mod 2^64 with d_i in
// [-128, 127] (d_i = low byte as a signed value, then v = (v - d_i) / 256), so
//   L * R = sum_{s=0..7} 256^s S_s  mod 2^64,   S_s = sum_{i+j=s} L_i * R_j,
// digit products with i + j >= 8 being multiples of 2^64.  That is 36 int8
// GEMMs.  |S_s| <= 8 * 2K * 2^14 < 2^31 for K < 8192, so the int32
// accumulators are exact and out = C + sum_s (int64)S_s << 8s.
//
// Passes:
//   1. split the LHS [D | A] into digit planes Lp[8][M][2K] (k contiguous);
//   2. split the RHS [B' ; E] into digit planes Rp[8][N][2K], transposed
//      through LDS so that k is contiguous per column;
//   3. one wave per 32 x 32 output tile and k-slice: per 32-deep k-step each
//      lane loads 16 bytes of each plane for its row / column (prefetched a
//      step ahead), then 36 MFMAs accumulate into 8 int32 tiles (one per s);
//      the epilogue adds C and the shifted partial sums in u64 (or, with
//      several k-slices for small grids, writes partials that a reduction
//      pass sums with C).
// MFMA operand layout (checked on the device): lane l supplies row / column
// l % 32 at k = 16 (l / 32) + byte; accumulator register r of lane l is
// row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
#include <hip/hip_runtime.h>

#include "suf_hip.h"
#include "digit_planes.hpp"
#include "sufhip_internal.hpp"

namespace sufhip {
namespace {

constexpr int kPlanes = kDigitPlanes;
constexpr int kMaxK = 8191;

// Pass 1: rows of [S0 | S1] (each rows x K, row-major) -> planes [8][rows][2K].
// One lane per 4 consecutive k of one row.
__global__ void __launch_bounds__(256)
    split_rows_kernel(const uint64_t* S0, const uint64_t* S1, int rows, int K, int8_t* planes) {
  const int K2 = 2 * K;
  const size_t quads = size_t(rows) * K2 / 4;
  const size_t plane = size_t(rows) * K2;
  for (size_t q = size_t(blockIdx.x) * 256 + threadIdx.x; q < quads; q += size_t(gridDim.x) * 256) {
    const size_t idx = 4 * q;
    const int m = int(idx / K2), k = int(idx % K2);
    const uint64_t* src = k < K ? S0 + size_t(m) * K + k : S1 + size_t(m) * K + (k - K);
    uint32_t pk[kPlanes] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      uint32_t d[kPlanes];
      digits8(src[t], d);
#pragma unroll
      for (int i = 0; i < kPlanes; ++i) pk[i] |= d[i] << (8 * t);
    }
#pragma unroll
    for (int i = 0; i < kPlanes; ++i)
      *reinterpret_cast<uint32_t*>(planes + i * plane + idx) = pk[i];
  }
}

// Pass 2: columns of [B + add_e E ; E] (K2 x N) -> planes [8][N][2K], 64 x 64
// tiles transposed through LDS.  grid = (N / 64, 2K / 64).
__global__ void __launch_bounds__(256)
    split_cols_kernel(const uint64_t* B, const uint64_t* E, int add_e, int K, int N,
                      int8_t* planes) {
  __shared__ uint64_t tile[64][65];
  const int K2 = 2 * K;
  const int n0 = blockIdx.x * 64, k0 = blockIdx.y * 64;
  const int tid = threadIdx.x;
  const int cn = tid & 63;
#pragma unroll 4
  for (int it = 0; it < 16; ++it) {
    const int kk = it * 4 + (tid >> 6);
    const int k = k0 + kk, n = n0 + cn;
    uint64_t v;
    if (k < K) {
      v = B[size_t(k) * N + n];
      if (add_e) v += E[size_t(k) * N + n];
    } else {
      v = E[size_t(k - K) * N + n];
    }
    tile[kk][cn] = v;
  }
  __syncthreads();
  // Lane: column n0 + (tid & 63), 16 consecutive k starting at 16 * (tid >> 6).
  const int kg = tid >> 6;
  uint32_t pk[kPlanes][4];
#pragma unroll
  for (int i = 0; i < kPlanes; ++i)
#pragma unroll
    for (int w = 0; w < 4; ++w) pk[i][w] = 0;
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    uint32_t d[kPlanes];
    digits8(tile[16 * kg + t][cn], d);
#pragma unroll
    for (int i = 0; i < kPlanes; ++i) pk[i][t >> 2] |= d[i] << (8 * (t & 3));
  }
  const size_t plane = size_t(N) * K2;
  const size_t off = size_t(n0 + cn) * K2 + k0 + 16 * kg;
#pragma unroll
  for (int i = 0; i < kPlanes; ++i)
    *reinterpret_cast<uint4*>(planes + i * plane + off) =
        make_uint4(pk[i][0], pk[i][1], pk[i][2], pk[i][3]);
}

// Pass 3: one wave per 32 x 32 output tile and k-slice.  grid = (N / 32,
// M / 32, slices).  The next k-step's fragments are loaded while the current
// step's 36 MFMAs run.  With one slice the wave writes C + its sum; with
// several, slice z writes its partial sum to part[z] for reduce_kernel.
__global__ void __launch_bounds__(64)
    limb_mfma_kernel(const int8_t* Lp, const int8_t* Rp, const uint64_t* C, int M, int K2, int N,
                     uint64_t* out, uint64_t* part) {
  const int l = threadIdx.x;
  const int m0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
  const int steps = K2 / 32;
  const int k_begin = 32 * (steps * int(blockIdx.z) / int(gridDim.z));
  const int k_end = 32 * (steps * (int(blockIdx.z) + 1) / int(gridDim.z));
  const size_t lplane = size_t(M) * K2, rplane = size_t(N) * K2;
  const int8_t* lrow = Lp + size_t(m0 + (l & 31)) * K2 + 16 * (l >> 5);
  const int8_t* rcol = Rp + size_t(n0 + (l & 31)) * K2 + 16 * (l >> 5);
  v16i acc[kPlanes];
#pragma unroll
  for (int s = 0; s < kPlanes; ++s)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[s][r] = 0;
  v4i a[kPlanes], b[kPlanes];
#pragma unroll
  for (int i = 0; i < kPlanes; ++i) {
    a[i] = load16(lrow + i * lplane + k_begin);
    b[i] = load16(rcol + i * rplane + k_begin);
  }
  for (int k = k_begin; k < k_end; k += 32) {
    v4i na[kPlanes], nb[kPlanes];
    const int kn = k + 32 < k_end ? k + 32 : k;  // last step reloads in bounds
#pragma unroll
    for (int i = 0; i < kPlanes; ++i) {
      na[i] = load16(lrow + i * lplane + kn);
      nb[i] = load16(rcol + i * rplane + kn);
    }
#pragma unroll
    for (int i = 0; i < kPlanes; ++i)
#pragma unroll
      for (int j = 0; i + j < kPlanes; ++j)
        acc[i + j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i + j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < kPlanes; ++i) {
      a[i] = na[i];
      b[i] = nb[i];
    }
  }
  const int col = n0 + (l & 31);
  uint64_t* dst = gridDim.z == 1 ? out : part + size_t(blockIdx.z) * M * N;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = m0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    uint64_t v = gridDim.z == 1 ? C[size_t(row) * N + col] : 0;
#pragma unroll
    for (int s = 0; s < kPlanes; ++s) v += uint64_t(int64_t(acc[s][r])) << (8 * s);
    dst[size_t(row) * N + col] = v;
  }
}

// out = C + sum_z part[z].
__global__ void __launch_bounds__(256)
    reduce_kernel(const uint64_t* part, int slices, const uint64_t* C, size_t mn, uint64_t* out) {
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < mn; i += size_t(gridDim.x) * 256) {
    uint64_t v = C[i];
    for (int z = 0; z < slices; ++z) v += part[size_t(z) * mn + i];
    out[i] = v;
  }
}

// k-slices so that a launch has about 1024 waves.
int slices_for(int M, int K, int N) {
  const int tiles = (M / 32) * (N / 32);
  const int steps = 2 * K / 32;
  int s = tiles >= 1024 ? 1 : (1024 + tiles - 1) / tiles;
  if (s > 4) s = 4;
  if (s > steps) s = steps;
  return s;
}

}  // namespace
}  // namespace sufhip

using namespace sufhip;

extern "C" {

size_t sufhip_beaver_matmul2d_mfma_work_bytes(int M, int K, int N) {
  if (M <= 0 || K <= 0 || N <= 0 || M % 32 || N % 64 || K % 32 || K > kMaxK) return 0;
  const int sl = slices_for(M, K, N);
  return size_t(kPlanes) * (size_t(M) + size_t(N)) * 2 * size_t(K) +
         (sl > 1 ? size_t(sl) * M * N * 8 : 0);
}

int sufhip_beaver_matmul2d_mfma(int party, const uint64_t* d_D_open, const uint64_t* d_E_open,
                                const uint64_t* d_A_tri_share, const uint64_t* d_B_tri_share,
                                const uint64_t* d_C_tri_share, int M, int K, int N,
                                uint64_t* d_out, void* d_work, size_t work_bytes, void* stream) {
  SUFHIP_REQUIRE(party == 0 || party == 1, "sufhip_beaver_matmul2d_mfma: party must be 0 or 1");
  SUFHIP_REQUIRE(M > 0 && K > 0 && N > 0, "sufhip_beaver_matmul2d_mfma: empty shape");
  SUFHIP_REQUIRE(M % 32 == 0 && N % 64 == 0 && K % 32 == 0 && K <= kMaxK,
                 "sufhip_beaver_matmul2d_mfma: needs M % 32 == 0, N % 64 == 0, K % 32 == 0, "
                 "K <= 8191");
  SUFHIP_REQUIRE(d_D_open && d_E_open && d_A_tri_share && d_B_tri_share && d_C_tri_share &&
                     d_out && d_work,
                 "sufhip_beaver_matmul2d_mfma: null pointer");
  const size_t need = sufhip_beaver_matmul2d_mfma_work_bytes(M, K, N);
  SUFHIP_REQUIRE(work_bytes >= need, "sufhip_beaver_matmul2d_mfma: workspace too small");
  SUFHIP_REQUIRE((reinterpret_cast<uintptr_t>(d_work) & 15) == 0,
                 "sufhip_beaver_matmul2d_mfma: workspace must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  int8_t* Lp = static_cast<int8_t*>(d_work);
  int8_t* Rp = Lp + size_t(kPlanes) * M * 2 * K;
  const size_t quads = size_t(M) * 2 * K / 4;
  size_t g1 = (quads + 255) / 256;
  if (g1 > 4096) g1 = 4096;
  hipLaunchKernelGGL(split_rows_kernel, dim3(unsigned(g1)), dim3(256), 0, s, d_D_open,
                     d_A_tri_share, M, K, Lp);
  if (int rc = check_launch("split_rows_kernel")) return rc;
  hipLaunchKernelGGL(split_cols_kernel, dim3(N / 64, 2 * K / 64), dim3(256), 0, s, d_B_tri_share,
                     d_E_open, party == 0 ? 1 : 0, K, N, Rp);
  if (int rc = check_launch("split_cols_kernel")) return rc;
  const int sl = slices_for(M, K, N);
  uint64_t* part = reinterpret_cast<uint64_t*>(Rp + size_t(kPlanes) * N * 2 * K);
  hipLaunchKernelGGL(limb_mfma_kernel, dim3(N / 32, M / 32, sl), dim3(64), 0, s, Lp, Rp,
                     d_C_tri_share, M, 2 * K, N, d_out, part);
  if (int rc = check_launch("limb_mfma_kernel")) return rc;
  if (sl == 1) return SUFHIP_OK;
  const size_t mn = size_t(M) * N;
  size_t g = (mn + 255) / 256;
  if (g > 4096) g = 4096;
  hipLaunchKernelGGL(reduce_kernel, dim3(unsigned(g)), dim3(256), 0, s, part, sl, d_C_tri_share,
                     mn, d_out);
  return check_launch("reduce_kernel");
}

}  // extern "C"
