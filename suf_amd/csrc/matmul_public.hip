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

// The QKV product's epilogue writing the attention's opens (on != 0): for
// output element (m, col) of [seq x 3 d], d = heads dh, region j = col / d
// (Q, K, V) and head h, column k of the region's head, the truncated value
// y_0 + y_1 minus sub[j] goes to out[j]'s digit planes (Q_h - A with
// Q_h - A + A_0, K_h^T - B, V_h - B2).
struct QkvOpen {
  int on, seq, dh, d;
  sufhip_kb_planes out[3];
  const uint64_t* sub[3][2];
};

struct PubArgs {
  const int8_t* Lp;  // [8][K/32][2M][32]
  const int8_t* Wp;  // [J][K/32][N][32]
  int M, K, N;
  uint64_t* out[2];  // shares (or NULL)
  uint64_t* zhat;    // masked open (or NULL)
  uint64_t mask;
  uint64_t* part;    // [slices][2][M][N] when gridDim.z > 1
  TruncEpi epi;      // the open feeds this truncation gate (replaces zhat)
  QkvOpen qo;        // with epi: its outputs go to the attention's opens instead
};

// The epilogue's open values v[t] of rows row[t] in column col, as the
// attention's opens (QkvOpen).  A 64-column block lies in one region (d is a
// multiple of 64); the subtrahends are indexed [heads][seq][dh] in every
// region (K^T's B transposed), so a wave's loads run along its columns.
// Every table, subtrahend and A_0 read is issued before the first plane
// store.  Rows row[4 g .. 4 g + 3] are consecutive and start at a multiple
// of 4 (the accumulator layout), so V's planes, whose k is the row, take one
// 4-byte store per plane for four rows.
template <int kN>
__device__ __forceinline__ void qkv_open_n(const TruncEpi& e, const EpiHdrs& eh, const QkvOpen& q,
                                           const int (&row)[kN], int col,
                                           const uint64_t (&v)[kN]) {
  static_assert(kN % 4 == 0, "rows in groups of four");
  const int j = col / q.d;
  const int n = col - j * q.d, h = n / q.dh, k = n - h * q.dh;
  const sufhip_kb_planes& o = q.out[j];
  const size_t hb = size_t(h) * size_t(q.seq) * size_t(q.dh);
  uint64_t w[kN][2], sb[kN][2], a0[kN];
#pragma unroll
  for (int t = 0; t < kN; ++t) {
    const size_t idx = hb + size_t(row[t]) * q.dh + k;
    w[t][0] = trunc_table_word(eh.h[0], e.table[0], e.f, v[t]);
    w[t][1] = trunc_table_word(eh.h[1], e.table[1], e.f, v[t]);
    sb[t][0] = q.sub[j][0][idx];
    sb[t][1] = q.sub[j][1][idx];
    a0[t] = o.a0 ? o.a0[idx] : 0;
  }
  const size_t plane = size_t(o.batches) * size_t(q.seq) * size_t(q.dh);
  uint64_t x[kN];
#pragma unroll
  for (int t = 0; t < kN; ++t)
    x[t] = trunc_table_out(eh.h[0], e.f, v[t], w[t][0]) +
           trunc_table_out(eh.h[1], e.f, v[t], w[t][1]) - sb[t][0] - sb[t][1];
  if (j == 2) {
    // V_h - B2: k = the sequence index (R = dh); four rows per 4-byte store.
#pragma unroll
    for (int g = 0; g < kN / 4; ++g) {
      uint32_t pk[kDigitPlanes] = {};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        uint32_t dg[kDigitPlanes];
        digits8(x[4 * g + t], dg);
#pragma unroll
        for (int i = 0; i < kDigitPlanes; ++i) pk[i] |= dg[i] << (8 * t);
      }
      const size_t off = hb + kblock_off(size_t(k), row[4 * g], size_t(q.dh));
#pragma unroll
      for (int i = 0; i < kDigitPlanes; ++i)
        *reinterpret_cast<uint32_t*>(o.planes + i * plane + off) = pk[i];
    }
    return;
  }
  // Q_h - A and K_h^T - B: k = column k of the head (R = seq).
#pragma unroll
  for (int t = 0; t < kN; ++t) {
    const size_t off = hb + kblock_off(size_t(row[t]), k, size_t(q.seq));
    uint32_t dg[kDigitPlanes];
    digits8(x[t], dg);
#pragma unroll
    for (int i = 0; i < kDigitPlanes; ++i) o.planes[i * plane + off] = int8_t(dg[i]);
    if (o.planes_a0) {
      digits8(x[t] + a0[t], dg);
#pragma unroll
      for (int i = 0; i < kDigitPlanes; ++i) o.planes_a0[i * plane + off] = int8_t(dg[i]);
    }
  }
}

// k-steps in the register pipeline of a wave: step st's fragments are
// loaded pub_stages - 1 steps before its MFMAs (8 + J fragments a step).
template <int J>
constexpr int pub_stages() {
  return J <= 2 ? 5 : 3;
}

// Workgroup = two waves, wave p computing party p's 32 x 32 tile over one
// k-slice; grid = (N / 32, M / 32, slices).  MFMA operand layout (checked on
// the device for matmul_mfma.hip): lane l supplies row / column l % 32 at
// k = 16 (l / 32) + byte; accumulator register r of lane l is row 8 (r / 4)
// + 4 (l / 32) + r % 4, column l % 32.  Plane addresses are a wave-uniform
// base plus the lane's 32-bit fragment offset (the planes of X and W stay
// below 4 GB, checked on the host), and the pipeline's buffers rotate by
// unrolling, so the loads of later steps stay in flight across the MFMAs.
template <int J>
__global__ void __launch_bounds__(128, 1) __attribute__((amdgpu_waves_per_eu(1, 1)))
public_mfma_kernel(PubArgs a) {
  __shared__ uint64_t other[16][64];  // party 1's tile, for the open
  const int l = threadIdx.x & 63;
  const int p = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
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
  const uint32_t lrows = uint32_t(2) * M;
  const uint32_t lplane = lrows * K, wplane = uint32_t(N) * K;
  const uint32_t lstep = lrows * 32, wstep = uint32_t(N) * 32;
  const uint32_t fo = uint32_t(l & 31) * 32 + 16 * uint32_t(l >> 5);
  const int8_t* lbase = a.Lp + (uint32_t(p * M + m0) * 32);
  const int8_t* wbase = a.Wp + uint32_t(n0) * 32;
  v16i acc[kPlanes];
#pragma unroll
  for (int s = 0; s < kPlanes; ++s)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[s][r] = 0;
  constexpr int S = pub_stages<J>();
  constexpr int kMfmas = J * kPlanes - J * (J - 1) / 2;  // digit products i + j < 8, j < J
  v4i x[S][kPlanes], w[S][J];
  auto issue = [&](int q, int st) {
    st = st < s_end ? st : s_end - 1;  // past the slice: repeat its last step (skipped)
    const uint32_t lo = uint32_t(st) * lstep, wo = uint32_t(st) * wstep;
#pragma unroll
    for (int i = 0; i < kPlanes; ++i) x[q][i] = load16(lbase + (i * lplane + lo) + fo);
#pragma unroll
    for (int j = 0; j < J; ++j) w[q][j] = load16(wbase + (j * wplane + wo) + fo);
  };
  auto mfmas = [&](int q) {
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int i = 0; i + j < kPlanes; ++i)
        acc[i + j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x[q][i], w[q][j], acc[i + j], 0, 0, 0);
  };
  // Whole groups of S steps without branches in the loop body (so the
  // loads' waits stay counted), then the last n % S steps, whose loads the
  // pipeline already issued into buffers 0 .. n % S - 1.
#pragma unroll
  for (int q = 0; q < S - 1; ++q) issue(q, s_begin + q);
  const int n = s_end - s_begin;
  const int groups = n / S;
  for (int g2 = 0; g2 < groups; ++g2) {
    const int t0 = s_begin + g2 * S;
#pragma unroll
    for (int h = 0; h < S; ++h) {
      issue((h + S - 1) % S, t0 + h + S - 1);
      mfmas(h);
      // Order for the scheduler: this step's loads, then its MFMAs (which
      // use the fragments loaded S - 1 steps earlier).
      __builtin_amdgcn_sched_group_barrier(0x020, kPlanes + J, 0);  // VMEM reads
      __builtin_amdgcn_sched_group_barrier(0x008, kMfmas, 0);       // MFMAs
    }
  }
  const int rest = n - groups * S;
#pragma unroll
  for (int h = 0; h < S - 1; ++h)
    if (h < rest) mfmas(h);
  const EpiHdrs eh = epi_hdrs(a.epi);  // before the first global store
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
      for (int h = 0; h < 2; ++h) {
        size_t ii[8];
        uint64_t vv[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int r = 8 * h + q;
          const int row = m0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
          ii[q] = size_t(row) * N + col;
          vv[q] = v[r] + other[r][l] + a.mask;
        }
        put_open_n<8>(a.epi, eh, a.zhat, ii, vv);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// The product for N a multiple of 64: a workgroup of four waves covers a
// 32 x 64 output block for both parties, wave (p, c) party p's 32 x 32
// sub-tile c.  A k-step's operand blocks -- both parties' 8 X planes and the
// J W planes of the two sub-tiles, 1 KB each -- go once into LDS with
// global_load_lds_dwordx4 (each lane's 16 bytes land at 16 lane in the
// block, which is the MFMA fragment layout) through a kPubStages-deep ring,
// and each wave reads its 8 + J fragments from there: the workgroup loads
// each X fragment once instead of once per column tile and each W fragment
// once instead of once per party.  The DMA of step t + kPubStages - 1 is
// issued after the barrier of step t (when every wave is done with the
// stage it overwrites); every wave issues the same number of DMAs each step
// (dummy blocks pad the stage), so a fixed vmcnt waits for step t exactly.
// The LDS reads are one asm statement with their wait, so no instruction
// can touch their registers before the data is there.
constexpr int kPubStages = 3;
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;
typedef __attribute__((address_space(3))) uint8_t lds_u8_t;

__device__ __forceinline__ void dma16(const int8_t* g, uint8_t* l) {
  __builtin_amdgcn_global_load_lds((glb_void_t*)g, (lds_void_t*)l, 16, 0, 0);
}

__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((const lds_u8_t*)p));
}

// s_waitcnt with vmcnt(N) only (expcnt and lgkmcnt at their maxima).
template <int N>
constexpr int vm_wait_imm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  return (N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8);
}

// Blocks of one stage: 16 X planes (party p plane i at 8 p + i), 2 J W
// planes (sub-tile c plane j at 16 + c J + j), padded to a multiple of the
// four waves.
template <int J>
constexpr int stage_blocks() {
  return (16 + 2 * J + 3) / 4 * 4;
}

#define SUFHIP_RD(n, reg, off) "ds_read_b128 %" #n ", %" #reg " offset:" #off "\n"
#define SUFHIP_RD_X8(xr)                                                                     \
  SUFHIP_RD(0, xr, 0) SUFHIP_RD(1, xr, 1024) SUFHIP_RD(2, xr, 2048) SUFHIP_RD(3, xr, 3072)    \
  SUFHIP_RD(4, xr, 4096) SUFHIP_RD(5, xr, 5120) SUFHIP_RD(6, xr, 6144) SUFHIP_RD(7, xr, 7168)
#define SUFHIP_XOUT                                                                          \
  "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]), "=&v"(x[3]), "=&v"(x[4]), "=&v"(x[5]), "=&v"(x[6]), \
      "=&v"(x[7])

// x: the 8 X fragments at ax (1 KB apart); w: the J W fragments at aw.  The
// reads are issued without a wait: wait_frags() completes them.
template <int J>
__device__ __forceinline__ void rd_frags(v4i (&x)[kPlanes], v4i (&w)[J], uint32_t ax, uint32_t aw);
template <>
__device__ __forceinline__ void rd_frags<1>(v4i (&x)[kPlanes], v4i (&w)[1], uint32_t ax,
                                            uint32_t aw) {
  asm volatile(SUFHIP_RD_X8(9) SUFHIP_RD(8, 10, 0) : SUFHIP_XOUT, "=&v"(w[0]) : "v"(ax), "v"(aw));
}
template <>
__device__ __forceinline__ void rd_frags<2>(v4i (&x)[kPlanes], v4i (&w)[2], uint32_t ax,
                                            uint32_t aw) {
  asm volatile(SUFHIP_RD_X8(10) SUFHIP_RD(8, 11, 0) SUFHIP_RD(9, 11, 1024)
               : SUFHIP_XOUT, "=&v"(w[0]), "=&v"(w[1])
               : "v"(ax), "v"(aw));
}
template <>
__device__ __forceinline__ void rd_frags<3>(v4i (&x)[kPlanes], v4i (&w)[3], uint32_t ax,
                                            uint32_t aw) {
  asm volatile(SUFHIP_RD_X8(11) SUFHIP_RD(8, 12, 0) SUFHIP_RD(9, 12, 1024) SUFHIP_RD(10, 12, 2048)
               : SUFHIP_XOUT, "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2])
               : "v"(ax), "v"(aw));
}
template <>
__device__ __forceinline__ void rd_frags<4>(v4i (&x)[kPlanes], v4i (&w)[4], uint32_t ax,
                                            uint32_t aw) {
  asm volatile(SUFHIP_RD_X8(12) SUFHIP_RD(8, 13, 0) SUFHIP_RD(9, 13, 1024) SUFHIP_RD(10, 13, 2048)
                   SUFHIP_RD(11, 13, 3072)
               : SUFHIP_XOUT, "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3])
               : "v"(ax), "v"(aw));
}

// Waits for rd_frags' reads.  The fragments are in-out operands, so that no
// use of them can be scheduled above the wait.
#define SUFHIP_XIO                                                                           \
  "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]), \
      "+v"(x[7])
template <int J>
__device__ __forceinline__ void wait_frags(v4i (&x)[kPlanes], v4i (&w)[J]) {
  if constexpr (J == 1)
    asm volatile("s_waitcnt lgkmcnt(0)" : SUFHIP_XIO, "+v"(w[0]));
  else if constexpr (J == 2)
    asm volatile("s_waitcnt lgkmcnt(0)" : SUFHIP_XIO, "+v"(w[0]), "+v"(w[1]));
  else if constexpr (J == 3)
    asm volatile("s_waitcnt lgkmcnt(0)" : SUFHIP_XIO, "+v"(w[0]), "+v"(w[1]), "+v"(w[2]));
  else
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : SUFHIP_XIO, "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]));
}
#undef SUFHIP_XIO
#undef SUFHIP_RD
#undef SUFHIP_RD_X8
#undef SUFHIP_XOUT

template <int J>
__global__ void __launch_bounds__(256, 1) public_lds_kernel(PubArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  // The truncation's key headers (scalar loads) in flight during the k-loop.
  const EpiHdrs eh = epi_hdrs(a.epi);
  constexpr int kBlocks = stage_blocks<J>();
  constexpr int kPerWave = kBlocks / 4;
  constexpr int kStageBytes = kBlocks * 1024;
  const int l = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int p = w >> 1, c = w & 1;
  const int M = a.M, K = a.K, N = a.N;
  const int gx = gridDim.x, gy = gridDim.y, gz = gridDim.z;
  const int total = gx * gy * gz;
  int g = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  if (total % 8 == 0) g = (g % 8) * (total / 8) + g / 8;  // XCD-aware order, as above
  const int slice = g % gz, tile_y = (g / gz) % gy, tile_x = g / (gz * gy);
  const int m0 = tile_y * 32, n0 = tile_x * 64;
  const int steps = K / 32;
  const int s_begin = steps * slice / gz;
  const int s_end = steps * (slice + 1) / gz;
  const uint32_t lplane = uint32_t(2) * M * K, wplane = uint32_t(N) * K;
  const uint32_t lstep = uint32_t(2) * M * 32, wstep = uint32_t(N) * 32;
  const uint32_t fo = uint32_t(l & 31) * 32 + 16 * uint32_t(l >> 5);
  // This wave's DMA blocks: b = w kPerWave + q; block bases are uniform.
  const int8_t* gb[kPerWave];
  uint32_t gs[kPerWave];
#pragma unroll
  for (int q = 0; q < kPerWave; ++q) {
    int b = w * kPerWave + q;
    if (b >= 16 + 2 * J) b = 0;  // padding: a valid block, never read
    if (b < 16) {
      gb[q] = a.Lp + (uint32_t(b & 7) * lplane + uint32_t((b >> 3) * M + m0) * 32);
      gs[q] = lstep;
    } else {
      const int cc = (b - 16) / J, j = (b - 16) % J;
      gb[q] = a.Wp + (uint32_t(j) * wplane + uint32_t(n0 + 32 * cc) * 32);
      gs[q] = wstep;
    }
  }
  auto dma = [&](int stage, int st) {
    st = st < s_end ? st : s_end - 1;  // past the slice: its last step again (never read)
    uint8_t* dst = lds + stage * kStageBytes + (w * kPerWave) * 1024;
#pragma unroll
    for (int q = 0; q < kPerWave; ++q) dma16(gb[q] + (uint32_t(st) * gs[q] + fo), dst + q * 1024);
  };
  v16i acc[kPlanes];
#pragma unroll
  for (int s = 0; s < kPlanes; ++s)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[s][r] = 0;
  const int n = s_end - s_begin;
  const uint32_t lane_base = lds_addr(lds) + 16 * uint32_t(l);
  const uint32_t xoff = uint32_t(8 * p) * 1024, woff = uint32_t(16 + c * J) * 1024;
  auto frags = [&](int stage, v4i (&x)[kPlanes], v4i (&wf)[J]) {
    const uint32_t sb = lane_base + uint32_t(stage) * kStageBytes;
    rd_frags<J>(x, wf, sb + xoff, sb + woff);
    // The MFMAs that follow stay below the reads (issued after the last
    // MFMA, the reads would wait for the whole step's MFMA issue).
    __builtin_amdgcn_sched_barrier(0);
  };
  auto mfmas = [&](const v4i (&x)[kPlanes], const v4i (&wf)[J]) {
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int i = 0; i + j < kPlanes; ++i)
        acc[i + j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x[i], wf[j], acc[i + j], 0, 0, 0);
    // ... and above the wait for the next step's reads.
    __builtin_amdgcn_sched_barrier(0);
  };
  // Every stage filled (steps 0 .. kPubStages - 1), step 0's fragments read.
  // Then step t: wait for step t + 1's blocks (this wave's DMAs, then the
  // barrier for everyone's, which also says that every wave has read step
  // t's stage), refill step t's stage with step t + kPubStages, read step
  // t + 1's fragments into the other register set, and run step t's MFMAs
  // while those reads are in flight.  Reads of a step past the slice see a
  // stage holding its last step again (never used).
#pragma unroll
  for (int q = 0; q < kPubStages; ++q) dma(q, s_begin + q);
  v4i xa[kPlanes], wa[J], xb[kPlanes], wb[J];
  __builtin_amdgcn_s_waitcnt(vm_wait_imm<(kPubStages - 1) * kPerWave>());
  __builtin_amdgcn_s_barrier();
  frags(0, xa, wa);
  wait_frags<J>(xa, wa);
  int stage = 0;  // step t's stage
  int t = 0;
  for (; t + 1 < n; t += 2) {  // steps t (in xa) and t + 1 (in xb)
    const int s1 = stage + 1 == kPubStages ? 0 : stage + 1;
    const int s2 = s1 + 1 == kPubStages ? 0 : s1 + 1;
    __builtin_amdgcn_s_waitcnt(vm_wait_imm<(kPubStages - 2) * kPerWave>());
    __builtin_amdgcn_s_barrier();
    dma(stage, s_begin + t + kPubStages);
    frags(s1, xb, wb);
    mfmas(xa, wa);
    wait_frags<J>(xb, wb);
    __builtin_amdgcn_s_waitcnt(vm_wait_imm<(kPubStages - 2) * kPerWave>());
    __builtin_amdgcn_s_barrier();
    dma(s1, s_begin + t + 1 + kPubStages);
    frags(s2, xa, wa);
    mfmas(xb, wb);
    wait_frags<J>(xa, wa);
    stage = s2;
  }
  if (t < n) mfmas(xa, wa);  // an odd last step, already in xa
  __builtin_amdgcn_s_waitcnt(vm_wait_imm<0>());  // no DMA may land after the ring is reused
  const int col = n0 + 32 * c + (l & 31);
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
    // Both parties' sub-tiles through LDS (the ring is free); wave (p, c)
    // then opens rows r in [8 p, 8 p + 8) of sub-tile c.
    __syncthreads();
    uint64_t(*both)[2][16][64] = reinterpret_cast<uint64_t(*)[2][16][64]>(lds);
#pragma unroll
    for (int r = 0; r < 16; ++r) both[c][p][r][l] = v[r];
    __syncthreads();
    size_t ii[8];
    int rr[8];
    uint64_t vv[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int r = 8 * p + q;
      rr[q] = m0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
      ii[q] = size_t(rr[q]) * N + col;
      vv[q] = both[c][0][r][l] + both[c][1][r][l] + a.mask;
    }
    if (a.qo.on)
      qkv_open_n<8>(a.epi, eh, a.qo, rr, col, vv);
    else
      put_open_n<8>(a.epi, eh, a.zhat, ii, vv);
  }
}

// The ring's dynamic LDS (60-72 KB; above 64 KB the kernel must allow it).
template <int J>
size_t public_lds_bytes() {
  static const int allowed = [] {
    return int(hipFuncSetAttribute(reinterpret_cast<const void*>(&public_lds_kernel<J>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                   int(size_t(kPubStages) * stage_blocks<J>() * 1024)));
  }();
  (void)allowed;
  return size_t(kPubStages) * stage_blocks<J>() * 1024;
}

// Slices -> shares and/or the masked open.
__global__ void __launch_bounds__(256)
    public_reduce_kernel(const uint64_t* part, int slices, size_t mn, uint64_t* out0,
                         uint64_t* out1, uint64_t* zhat, uint64_t mask, TruncEpi epi) {
  const EpiHdrs eh = epi_hdrs(epi);
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < mn; i += size_t(gridDim.x) * 256) {
    // Slices in groups of four, then one by one, every load of a group
    // issued before its adds: a loop of single slices waits for each
    // slice's loads before it issues the next.
    uint64_t v0 = 0, v1 = 0;
    int z = 0;
    for (; z + 4 <= slices; z += 4) {
      uint64_t t[4][2];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        t[u][0] = part[(size_t(z + u) * 2 + 0) * mn + i];
        t[u][1] = part[(size_t(z + u) * 2 + 1) * mn + i];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        v0 += t[u][0];
        v1 += t[u][1];
      }
    }
    for (; z < slices; ++z) {
      v0 += part[(size_t(z) * 2 + 0) * mn + i];
      v1 += part[(size_t(z) * 2 + 1) * mn + i];
    }
    if (out0) out0[i] = v0;
    if (out1) out1[i] = v1;
    put_open(epi, eh, zhat, i, v0 + v1 + mask);
  }
}

// k-slices so that every wave of a launch is resident at once (one wave per
// SIMD: 256 four-wave workgroups of 32 x 64 blocks, or 512 two-wave ones of
// 32 x 32 tiles when N is not a multiple of 64) and a slice has at least
// four k-steps; one slice needs no reduction pass.
int pub_slices(int M, int K, int N) {
  const bool wide = N % 64 == 0;
  const int tiles = (M / 32) * (N / (wide ? 64 : 32));
  const int cap = wide ? 256 : 512;
  const int steps = K / 32;
  int s = tiles >= cap ? 1 : cap / tiles;
  if (s > 8) s = 8;
  if (s > steps / 4) s = steps / 4 > 0 ? steps / 4 : 1;
  return s;
}

bool shape_ok(int M, int K, int N) {
  // The kernel addresses the 8 X planes (2M rows) and the W planes (up to 8)
  // with 32-bit offsets.
  return M > 0 && K > 0 && N > 0 && M % 32 == 0 && N % 32 == 0 && K % 32 == 0 &&
         size_t(K) < (size_t(1) << 16) &&
         uint64_t(kPlanes) * 2 * uint64_t(M) * uint64_t(K) < (uint64_t(1) << 32) &&
         uint64_t(kPlanes) * uint64_t(N) * uint64_t(K) < (uint64_t(1) << 32);
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
// partial: stop before the reduction of the k-slices (the caller checked
// that there are several).
int launch_public2(const char* what, const int8_t* Lp, int M, int K, int N,
                   const int8_t* d_planes, int digits, uint64_t* d_out0, uint64_t* d_out1,
                   uint64_t* d_zhat, uint64_t mask, const sufhip_trunc_epilogue* trunc,
                   void* d_work, size_t work_bytes, hipStream_t s, bool partial = false,
                   const QkvOpen* qo = nullptr) {
  TruncEpi epi;
  if (int rc = make_epi(trunc, size_t(M) * N, what, &epi)) return rc;
  if (work_bytes < sufhip_matmul_public2_work_bytes(M, K, N)) {
    set_error(std::string(what) + ": workspace too small");
    return SUFHIP_ERR_INVALID;
  }
  const int sl = pub_slices(M, K, N);
  uint64_t* part =
      reinterpret_cast<uint64_t*>(static_cast<int8_t*>(d_work) + size_t(kPlanes) * 2 * M * K);
  PubArgs a{Lp, d_planes, M, K, N, {d_out0, d_out1}, d_zhat, mask, part, epi, QkvOpen{}};
  if (qo) a.qo = *qo;
  if (N % 64 == 0) {
    const dim3 grid(N / 64, M / 32, sl);
    switch (digits) {
      case 1:
        hipLaunchKernelGGL(public_lds_kernel<1>, grid, dim3(256), public_lds_bytes<1>(), s, a);
        break;
      case 2:
        hipLaunchKernelGGL(public_lds_kernel<2>, grid, dim3(256), public_lds_bytes<2>(), s, a);
        break;
      case 3:
        hipLaunchKernelGGL(public_lds_kernel<3>, grid, dim3(256), public_lds_bytes<3>(), s, a);
        break;
      default:
        hipLaunchKernelGGL(public_lds_kernel<4>, grid, dim3(256), public_lds_bytes<4>(), s, a);
        break;
    }
    if (int rc = check_launch("public_lds_kernel")) return rc;
  } else {
    const dim3 grid(N / 32, M / 32, sl);
    switch (digits) {
      case 1: hipLaunchKernelGGL(public_mfma_kernel<1>, grid, dim3(128), 0, s, a); break;
      case 2: hipLaunchKernelGGL(public_mfma_kernel<2>, grid, dim3(128), 0, s, a); break;
      case 3: hipLaunchKernelGGL(public_mfma_kernel<3>, grid, dim3(128), 0, s, a); break;
      default: hipLaunchKernelGGL(public_mfma_kernel<4>, grid, dim3(128), 0, s, a); break;
    }
    if (int rc = check_launch("public_mfma_kernel")) return rc;
  }
  if (sl == 1 || partial) return SUFHIP_OK;
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

int sufhip_matmul_public2_planes_qkv(const int8_t* d_Xp, int M, int K, int N,
                                     const int8_t* d_planes, int digits, uint64_t mask,
                                     const sufhip_trunc_epilogue* trunc,
                                     const sufhip_qkv_opens* opens, void* d_work,
                                     size_t work_bytes, void* stream) {
  const char* what = "sufhip_matmul_public2_planes_qkv";
  SUFHIP_REQUIRE(opens && trunc, "sufhip_matmul_public2_planes_qkv: opens and trunc are required");
  if (int rc = check_public2(what, M, K, N, d_planes, digits, nullptr, nullptr, nullptr, trunc,
                             d_work))
    return rc;
  SUFHIP_REQUIRE(d_Xp && (reinterpret_cast<uintptr_t>(d_Xp) & 15) == 0,
                 "sufhip_matmul_public2_planes_qkv: X planes null or not 16-byte aligned");
  const sufhip_qkv_opens& g = *opens;
  const long long d = (long long)g.heads * g.dh;
  SUFHIP_REQUIRE(g.heads >= 1 && g.dh >= 32 && g.dh % 32 == 0 && d % 64 == 0 && g.seq == M &&
                     3 * d == N && pub_slices(M, K, N) == 1,
                 "sufhip_matmul_public2_planes_qkv: needs M = seq, N = 3 heads dh, dh a "
                 "multiple of 32, heads dh of 64, and an unsliced product");
  const int shape[3][3] = {{g.seq, g.dh, 1}, {g.dh, g.seq, 0}, {g.seq, g.dh, 0}};
  QkvOpen q{};
  q.on = 1;
  q.seq = g.seq;
  q.dh = g.dh;
  q.d = int(d);
  const size_t n = size_t(g.heads) * g.seq * g.dh;
  for (int j = 0; j < 3; ++j) {
    const sufhip_kb_planes& o = g.out[j];
    SUFHIP_REQUIRE(o.planes && kb_planes_ok(o, n) && o.batches == g.heads &&
                       o.rows == shape[j][0] && o.cols == shape[j][1] &&
                       (o.k_is_col != 0) == (shape[j][2] != 0) && (j == 0 || !o.planes_a0) &&
                       g.sub[j][0] && g.sub[j][1],
                   "sufhip_matmul_public2_planes_qkv: out[j] must be the planes of Q - A "
                   "(heads, seq, dh, k_is_col 1, optionally + A_0), K^T - B (heads, dh, seq, "
                   "0) and V - B2 (heads, seq, dh, 0), with both shares of each subtrahend");
    q.out[j] = o;
    q.sub[j][0] = g.sub[j][0];
    q.sub[j][1] = g.sub[j][1];
  }
  return launch_public2(what, d_Xp, M, K, N, d_planes, digits, nullptr, nullptr, nullptr, mask,
                        trunc, d_work, work_bytes, as_stream(stream), false, &q);
}

int sufhip_matmul_public2_slices(int M, int K, int N) {
  return shape_ok(M, K, N) ? pub_slices(M, K, N) : 0;
}

int sufhip_matmul_public2_planes_partial(const int8_t* d_Xp, int M, int K, int N,
                                         const int8_t* d_planes, int digits, void* d_work,
                                         size_t work_bytes, const uint64_t** d_slices,
                                         void* stream) {
  const char* what = "sufhip_matmul_public2_planes_partial";
  SUFHIP_REQUIRE(d_slices, "sufhip_matmul_public2_planes_partial: null d_slices");
  *d_slices = nullptr;
  uint64_t dummy = 0;  // check_public2 wants an output; the slices are it
  if (int rc = check_public2(what, M, K, N, d_planes, digits, nullptr, nullptr, &dummy, nullptr,
                             d_work))
    return rc;
  SUFHIP_REQUIRE(pub_slices(M, K, N) > 1,
                 "sufhip_matmul_public2_planes_partial: this shape runs as one k-slice");
  SUFHIP_REQUIRE(d_Xp && (reinterpret_cast<uintptr_t>(d_Xp) & 15) == 0,
                 "sufhip_matmul_public2_planes_partial: X planes null or not 16-byte aligned");
  if (int rc = launch_public2(what, d_Xp, M, K, N, d_planes, digits, nullptr, nullptr, nullptr, 0,
                              nullptr, d_work, work_bytes, as_stream(stream), true))
    return rc;
  *d_slices = reinterpret_cast<const uint64_t*>(static_cast<const int8_t*>(d_work) +
                                                size_t(kPlanes) * 2 * M * K);
  return SUFHIP_OK;
}

}  // extern "C"
