// Share x public-weight matrix product over Z_2^64 for both parties on the
// int8 matrix cores (gfx950 v_mfma_i32_32x32x32_i8), exact.
//
// Replaces nn::matmul_publicW_gpu (src/nn/matmul_gpu.cu:388-720; CPU form
// src/nn/matmul_publicW.cpp:17-36): Y_p = X_p * W mod 2^64, X_p a party's u64
// share [M x K], W public int64 [K x N].  The reference layer passes no bias.
//
// Both operands in balanced base-256 digits (as in matmul_mfma.hip):
// X_p = sum_{i<8} x_i 256^i, W = sum_{j<J} w_j 256^j with J the digit count
// that public weights need (|w| < 2^15: J = 2).  Then
//   X_p W = sum_{s<8} 256^s S_s mod 2^64,  S_s = sum_{i+j=s, j<J} X_i W_j,
// i.e. sum_{j<J} (8 - j) int8 GEMMs (15 for J = 2).  |S_s| <= J K 2^14 < 2^31
// for K < 2^17 / J, so int32 accumulation is exact.
//
// Digit planes are k-blocked: a plane is [K / 32][rows][32] int8, so the
// 32 rows x 32 k of one MFMA step are a contiguous 1 KB block and one 16-byte
// load per lane fetches it whole.  W's planes [J][K/32][N][32] are prepared
// once (public weights are fixed: the reference caches them on the device
// too, matmul_gpu.cu:620-674).  Per call: split X_0, X_1 into planes
// [8][K/32][2M][32] (party 0's rows first), then a workgroup of two waves,
// one per party, computes a 32 x 32 output tile over a k-slice with loads
// three steps ahead, and writes either the shares, or only the masked open
// zhat = Y_0 + Y_1 + mask that the following truncation gate consumes
// (TruncTask after every public matmul: attention_block.cpp:1136-1230,
// mlp_block.cpp:378-767), the two parties' tiles summed through LDS.  Small
// grids split k over slices whose partial sums a reduction pass adds.
#include <hip/hip_runtime.h>

#include "suf_hip.h"
#include "sufhip_internal.hpp"
#include "digit_planes.hpp"
#include "trunc_device.hpp"

namespace sufhip {
namespace {

constexpr int kPlanes = kDigitPlanes;

// X_0, X_1 [M][K] -> planes [8][K/32][2M][32]; one lane per 4 consecutive k
// of a row.
__global__ void __launch_bounds__(256)
    split_x2_kernel(const uint64_t* X0, const uint64_t* X1, int M, int K, int8_t* planes) {
  const size_t quads = size_t(2) * M * K / 4;
  const size_t rows = size_t(2) * M;
  const size_t plane = rows * K;
  for (size_t q = size_t(blockIdx.x) * 256 + threadIdx.x; q < quads; q += size_t(gridDim.x) * 256) {
    const size_t idx = 4 * q;
    const size_t row = idx / size_t(K);
    const int k = int(idx % size_t(K));
    const uint64_t* src = row < size_t(M) ? X0 + row * K + k : X1 + (row - M) * K + k;
    uint32_t pk[kPlanes] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      uint32_t d[kPlanes];
      digits8(src[t], d);
#pragma unroll
      for (int i = 0; i < kPlanes; ++i) pk[i] |= d[i] << (8 * t);
    }
    const size_t off = kblock_off(row, k, rows);
#pragma unroll
    for (int i = 0; i < kPlanes; ++i)
      *reinterpret_cast<uint32_t*>(planes + i * plane + off) = pk[i];
  }
}

// W [K][N] -> planes [J][K/32][N][32]; one lane per (n, 4 consecutive k).
__global__ void __launch_bounds__(256)
    split_w_kernel(const int64_t* W, int K, int N, int J, int8_t* planes) {
  const size_t quads = size_t(N) * K / 4;
  const size_t plane = size_t(N) * K;
  for (size_t q = size_t(blockIdx.x) * 256 + threadIdx.x; q < quads; q += size_t(gridDim.x) * 256) {
    const int n = int(q / (size_t(K) / 4));
    const int k = int(q % (size_t(K) / 4)) * 4;
    uint32_t pk[kPlanes] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      uint32_t d[kPlanes];
      digits8(uint64_t(W[size_t(k + t) * N + n]), d);
#pragma unroll
      for (int i = 0; i < kPlanes; ++i) pk[i] |= d[i] << (8 * t);
    }
    const size_t off = kblock_off(size_t(n), k, size_t(N));
    for (int j = 0; j < J; ++j) *reinterpret_cast<uint32_t*>(planes + j * plane + off) = pk[j];
  }
}

struct PubArgs {
  const int8_t* Lp;  // [8][K/32][2M][32]
  const int8_t* Wp;  // [J][K/32][N][32]
  int M, K, N;
  uint64_t* out[2];  // shares (or NULL)
  uint64_t* zhat;    // masked open (or NULL)
  uint64_t mask;
  uint64_t* part;    // [slices][2][M][N] when gridDim.z > 1
  TruncEpi epi;      // the open feeds this truncation gate (replaces zhat)
};

// k-steps of loads in flight per wave: two for the 2-digit weights of the
// layer (10 fragments a step), one for 3- and 4-digit weights, whose second
// step in flight would not fit beside the 128 accumulator registers.
template <int J>
constexpr int pub_ahead() {
  return J <= 2 ? 2 : 1;
}

// Workgroup = two waves, wave p computing party p's 32 x 32 tile over one
// k-slice; grid = (N / 32, M / 32, slices).  MFMA operand layout (checked on
// the device for matmul_mfma.hip): lane l supplies row / column l % 32 at
// k = 16 (l / 32) + byte; accumulator register r of lane l is row 8 (r / 4)
// + 4 (l / 32) + r % 4, column l % 32.
template <int J>
__global__ void __launch_bounds__(128, 2) public_mfma_kernel(PubArgs a) {
  __shared__ uint64_t other[16][64];  // party 1's tile, for the open
  const int l = threadIdx.x & 63, p = threadIdx.x >> 6;
  const int M = a.M, K = a.K, N = a.N;
  // XCD-aware tile order: workgroups are dealt round-robin to the 8 XCDs
  // (each with its own L2), so workgroup id g runs on XCD g % 8.  Give XCD x
  // a contiguous range of (column tile, row tile, slice) in that nesting, so
  // that its L2 holds 1/8 of W's columns (and all of X) instead of all of W.
  const int gx = gridDim.x, gy = gridDim.y, gz = gridDim.z;
  const int total = gx * gy * gz;
  int g = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  if (total % 8 == 0) g = (g % 8) * (total / 8) + g / 8;
  const int slice = g % gz, tile_y = (g / gz) % gy, tile_x = g / (gz * gy);
  const int m0 = tile_y * 32, n0 = tile_x * 32;
  const int steps = K / 32;
  const int s_begin = steps * slice / gz;
  const int s_end = steps * (slice + 1) / gz;
  const size_t lrows = size_t(2) * M;
  const size_t lplane = lrows * K, wplane = size_t(N) * K;
  // This lane's 16 bytes of step s: row (or column) l % 32, bytes 16 (l / 32).
  const int8_t* lbase = a.Lp + size_t(p * M + m0 + (l & 31)) * 32 + 16 * (l >> 5);
  const int8_t* wbase = a.Wp + size_t(n0 + (l & 31)) * 32 + 16 * (l >> 5);
  const size_t lstep = lrows * 32, wstep = size_t(N) * 32;
  v16i acc[kPlanes];
#pragma unroll
  for (int s = 0; s < kPlanes; ++s)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[s][r] = 0;
  constexpr int kPubAhead = pub_ahead<J>();
  v4i x[kPubAhead][kPlanes], w[kPubAhead][J];
#pragma unroll
  for (int q = 0; q < kPubAhead; ++q) {
    const int st = s_begin + q < s_end ? s_begin + q : s_begin;  // in bounds
#pragma unroll
    for (int i = 0; i < kPlanes; ++i) x[q][i] = load16(lbase + i * lplane + size_t(st) * lstep);
#pragma unroll
    for (int j = 0; j < J; ++j) w[q][j] = load16(wbase + j * wplane + size_t(st) * wstep);
  }
  for (int st = s_begin; st < s_end; ++st) {
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int i = 0; i + j < kPlanes; ++i)
        acc[i + j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x[0][i], w[0][j], acc[i + j], 0, 0, 0);
#pragma unroll
    for (int q = 0; q + 1 < kPubAhead; ++q) {
#pragma unroll
      for (int i = 0; i < kPlanes; ++i) x[q][i] = x[q + 1][i];
#pragma unroll
      for (int j = 0; j < J; ++j) w[q][j] = w[q + 1][j];
    }
    const int sn = st + kPubAhead < s_end ? st + kPubAhead : s_begin;  // in bounds
#pragma unroll
    for (int i = 0; i < kPlanes; ++i)
      x[kPubAhead - 1][i] = load16(lbase + i * lplane + size_t(sn) * lstep);
#pragma unroll
    for (int j = 0; j < J; ++j)
      w[kPubAhead - 1][j] = load16(wbase + j * wplane + size_t(sn) * wstep);
  }
  const int col = n0 + (l & 31);
  uint64_t v[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    v[r] = 0;
#pragma unroll
    for (int s = 0; s < kPlanes; ++s) v[r] += uint64_t(int64_t(acc[s][r])) << (8 * s);
  }
  if (gz > 1) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
      a.part[((size_t(slice) * 2 + p) * M + row) * N + col] = v[r];
    }
    return;
  }
  if (a.out[p]) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
      a.out[p][size_t(row) * N + col] = v[r];
    }
  }
  if (a.zhat || a.epi.on) {
    if (p == 1) {
#pragma unroll
      for (int r = 0; r < 16; ++r) other[r][l] = v[r];
    }
    __syncthreads();
    if (p == 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
        put_open(a.epi, a.zhat, size_t(row) * N + col, v[r] + other[r][l] + a.mask);
      }
    }
  }
}

// Slices -> shares and/or the masked open.
__global__ void __launch_bounds__(256)
    public_reduce_kernel(const uint64_t* part, int slices, size_t mn, uint64_t* out0,
                         uint64_t* out1, uint64_t* zhat, uint64_t mask, TruncEpi epi) {
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < mn; i += size_t(gridDim.x) * 256) {
    uint64_t v0 = 0, v1 = 0;
    for (int z = 0; z < slices; ++z) {
      v0 += part[(size_t(z) * 2 + 0) * mn + i];
      v1 += part[(size_t(z) * 2 + 1) * mn + i];
    }
    if (out0) out0[i] = v0;
    if (out1) out1[i] = v1;
    put_open(epi, zhat, i, v0 + v1 + mask);
  }
}

// k-slices so that a launch has about 512 workgroups (two waves each) and a
// slice has at least four k-steps.
int pub_slices(int M, int K, int N) {
  const int tiles = (M / 32) * (N / 32);
  const int steps = K / 32;
  int s = tiles >= 512 ? 1 : (512 + tiles - 1) / tiles;
  if (s > 8) s = 8;
  if (s > steps / 4) s = steps / 4 > 0 ? steps / 4 : 1;
  return s;
}

bool shape_ok(int M, int K, int N) {
  return M > 0 && K > 0 && N > 0 && M % 32 == 0 && N % 32 == 0 && K % 32 == 0 &&
         size_t(K) < (size_t(1) << 16);
}

}  // namespace
}  // namespace sufhip

using namespace sufhip;

extern "C" {

int sufhip_public_w_digits(const int64_t* w, size_t n) {
  if (!w) return 0;
  int need = 1;
  for (size_t i = 0; i < n; ++i) {
    uint64_t v = uint64_t(w[i]);
    int last = 0;
    for (int d = 0; d < kPlanes; ++d) {
      const uint64_t b = v & 0xffu;
      if (b != 0) last = d + 1;
      v = (v >> 8) + (b >> 7);
    }
    if (last > need) need = last;
  }
  return need;
}

size_t sufhip_public_w_planes_bytes(int K, int N, int digits) {
  if (!shape_ok(32, K, N) || digits < 1 || digits > kPlanes) return 0;
  return size_t(digits) * size_t(N) * size_t(K);
}

int sufhip_public_w_prepare(const int64_t* d_W, int K, int N, int digits, int8_t* d_planes,
                            void* stream) {
  SUFHIP_REQUIRE(shape_ok(32, K, N), "sufhip_public_w_prepare: needs K % 32 == 0, N % 32 == 0");
  SUFHIP_REQUIRE(digits >= 1 && digits <= kPlanes, "sufhip_public_w_prepare: digits in [1, 8]");
  SUFHIP_REQUIRE(d_W && d_planes, "sufhip_public_w_prepare: null pointer");
  SUFHIP_REQUIRE((reinterpret_cast<uintptr_t>(d_planes) & 3) == 0,
                 "sufhip_public_w_prepare: planes must be 4-byte aligned");
  const size_t quads = size_t(N) * K / 4;
  size_t g = (quads + 255) / 256;
  if (g > 4096) g = 4096;
  hipLaunchKernelGGL(split_w_kernel, dim3(unsigned(g)), dim3(256), 0, as_stream(stream), d_W, K, N,
                     digits, d_planes);
  return check_launch("split_w_kernel");
}

size_t sufhip_matmul_public2_work_bytes(int M, int K, int N) {
  if (!shape_ok(M, K, N)) return 0;
  const int sl = pub_slices(M, K, N);
  return size_t(kPlanes) * 2 * size_t(M) * size_t(K) +
         (sl > 1 ? size_t(sl) * 2 * size_t(M) * size_t(N) * 8 : 0);
}

}  // extern "C"

namespace sufhip {
namespace {

// The product from X's planes Lp ([8][K/32][2M][32]); work holds the
// k-slices' partial tiles after the X planes region.
int launch_public2(const char* what, const int8_t* Lp, int M, int K, int N,
                   const int8_t* d_planes, int digits, uint64_t* d_out0, uint64_t* d_out1,
                   uint64_t* d_zhat, uint64_t mask, const sufhip_trunc_epilogue* trunc,
                   void* d_work, size_t work_bytes, hipStream_t s) {
  TruncEpi epi;
  if (int rc = make_epi(trunc, size_t(M) * N, what, &epi)) return rc;
  if (work_bytes < sufhip_matmul_public2_work_bytes(M, K, N)) {
    set_error(std::string(what) + ": workspace too small");
    return SUFHIP_ERR_INVALID;
  }
  const int sl = pub_slices(M, K, N);
  uint64_t* part =
      reinterpret_cast<uint64_t*>(static_cast<int8_t*>(d_work) + size_t(kPlanes) * 2 * M * K);
  PubArgs a{Lp, d_planes, M, K, N, {d_out0, d_out1}, d_zhat, mask, part, epi};
  const dim3 grid(N / 32, M / 32, sl);
  switch (digits) {
    case 1: hipLaunchKernelGGL(public_mfma_kernel<1>, grid, dim3(128), 0, s, a); break;
    case 2: hipLaunchKernelGGL(public_mfma_kernel<2>, grid, dim3(128), 0, s, a); break;
    case 3: hipLaunchKernelGGL(public_mfma_kernel<3>, grid, dim3(128), 0, s, a); break;
    default: hipLaunchKernelGGL(public_mfma_kernel<4>, grid, dim3(128), 0, s, a); break;
  }
  if (int rc = check_launch("public_mfma_kernel")) return rc;
  if (sl == 1) return SUFHIP_OK;
  const size_t mn = size_t(M) * N;
  size_t g = (mn + 255) / 256;
  if (g > 4096) g = 4096;
  hipLaunchKernelGGL(public_reduce_kernel, dim3(unsigned(g)), dim3(256), 0, s, part, sl, mn,
                     d_out0, d_out1, d_zhat, mask, epi);
  return check_launch("public_reduce_kernel");
}

int check_public2(const char* what, int M, int K, int N, const int8_t* d_planes, int digits,
                  uint64_t* d_out0, uint64_t* d_out1, uint64_t* d_zhat,
                  const sufhip_trunc_epilogue* trunc, void* d_work) {
  auto fail = [&](const char* msg) {
    set_error(std::string(what) + ": " + msg);
    return SUFHIP_ERR_INVALID;
  };
  if (!shape_ok(M, K, N)) return fail("needs M, K, N multiples of 32 and K < 65536");
  if (digits < 1 || digits > 4 || size_t(digits) * K >= (size_t(1) << 17))
    return fail("digits must be 1..4 with digits * K < 2^17");
  if (!d_planes || !d_work) return fail("null pointer");
  if ((d_out0 == nullptr) != (d_out1 == nullptr)) return fail("give both share outputs or neither");
  if (!d_out0 && !d_zhat && !trunc) return fail("no output");
  if ((reinterpret_cast<uintptr_t>(d_work) & 15) != 0 ||
      (reinterpret_cast<uintptr_t>(d_planes) & 15) != 0)
    return fail("workspace and planes must be 16-byte aligned");
  return SUFHIP_OK;
}

}  // namespace
}  // namespace sufhip

extern "C" {

int sufhip_matmul_public2(const uint64_t* d_X0, const uint64_t* d_X1, int M, int K, int N,
                          const int8_t* d_planes, int digits, uint64_t* d_out0, uint64_t* d_out1,
                          uint64_t* d_zhat, uint64_t mask, const sufhip_trunc_epilogue* trunc,
                          void* d_work, size_t work_bytes, void* stream) {
  const char* what = "sufhip_matmul_public2";
  if (int rc = check_public2(what, M, K, N, d_planes, digits, d_out0, d_out1, d_zhat, trunc,
                             d_work))
    return rc;
  SUFHIP_REQUIRE(d_X0 && d_X1, "sufhip_matmul_public2: null pointer");
  hipStream_t s = as_stream(stream);
  int8_t* Lp = static_cast<int8_t*>(d_work);
  const size_t quads = size_t(2) * M * K / 4;
  size_t g1 = (quads + 255) / 256;
  if (g1 > 4096) g1 = 4096;
  if (work_bytes < sufhip_matmul_public2_work_bytes(M, K, N)) {
    set_error("sufhip_matmul_public2: workspace too small");
    return SUFHIP_ERR_INVALID;
  }
  hipLaunchKernelGGL(split_x2_kernel, dim3(unsigned(g1)), dim3(256), 0, s, d_X0, d_X1, M, K, Lp);
  if (int rc = check_launch("split_x2_kernel")) return rc;
  return launch_public2(what, Lp, M, K, N, d_planes, digits, d_out0, d_out1, d_zhat, mask, trunc,
                        d_work, work_bytes, s);
}

int sufhip_matmul_public2_planes(const int8_t* d_Xp, int M, int K, int N, const int8_t* d_planes,
                                 int digits, uint64_t* d_out0, uint64_t* d_out1, uint64_t* d_zhat,
                                 uint64_t mask, const sufhip_trunc_epilogue* trunc, void* d_work,
                                 size_t work_bytes, void* stream) {
  const char* what = "sufhip_matmul_public2_planes";
  if (int rc = check_public2(what, M, K, N, d_planes, digits, d_out0, d_out1, d_zhat, trunc,
                             d_work))
    return rc;
  SUFHIP_REQUIRE(d_Xp && (reinterpret_cast<uintptr_t>(d_Xp) & 15) == 0,
                 "sufhip_matmul_public2_planes: X planes null or not 16-byte aligned");
  return launch_public2(what, d_Xp, M, K, N, d_planes, digits, d_out0, d_out1, d_zhat, mask,
                        trunc, d_work, work_bytes, as_stream(stream));
}

}  // extern "C"
