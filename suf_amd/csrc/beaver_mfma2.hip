// Two-party batched Beaver matrix product over Z_2^64 on the int8 matrix
// cores (gfx950 v_mfma_i32_32x32x32_i8), exact: the per-head QK^T and PV
// products of attention_forward (src/nn/attention_block.cpp:1590-1850, the
// BatchedMatmul2DTask form; element formula of launch_beaver_matmul2d_kernel,
// cuda/cuda_primitives.cu:391-506).  For batch b and party p:
//   out_p = C_p + D B_p + A_p E (+ D E for p = 0)   mod 2^64,
// with the opens D [M x K], E [K x N] and the triple shares A_p, B_p, C_p.
//
// Every operand is in balanced base-256 digit planes (digit_planes.hpp), so
// a product L R mod 2^64 is sum_{s<8} 256^s S_s, S_s = sum_{i+j=s} L_i R_j:
// 36 int8 GEMMs per operand pair, 72 (party 1) or 108 (party 0) per k-step.
// |S_s| <= 3 * 8 * K * 2^14 < 2^31 for K < 5461: int32 accumulation is exact.
// The triple shares' planes are made once, with the triples (like public
// weights, sufhip_public_w_prepare); the opens' planes per call, all opens of
// one stage in one launch (sufhip_kb_split_batch).
//
// Kernel: a workgroup per (32 x 32 output tile, batch) of two waves per
// k-slice, wave (slice, p) computing party p's tile over its k-steps; the
// slices' tiles are added through LDS.  MFMA operand layout (checked on
// the device for matmul_mfma.hip): lane l supplies row / column l % 32 at
// k = 16 (l / 32) + byte; accumulator register r of lane l is row 8 (r / 4)
// + 4 (l / 32) + r % 4, column l % 32.
#include <hip/hip_runtime.h>

#include "digit_planes.hpp"
#include "suf_hip.h"
#include "sufhip_internal.hpp"
#include "trunc_device.hpp"
#include "walk_device.hpp"

namespace sufhip {
namespace {

constexpr int kSplitJobs = SUFHIP_KB_SPLIT_JOBS;
constexpr int kMaxBeaverK = 4096;

struct SplitArgs {
  const uint64_t* src[kSplitJobs];
  const uint64_t* add[kSplitJobs];     // optional: + add[i]
  const uint64_t* sub[kSplitJobs][2];  // optional: - sub[0][i] - sub[1][i]
  int8_t* planes[kSplitJobs];
  int8_t* planes_a0[kSplitJobs];       // optional: planes of the value + a0[i]
  const uint64_t* a0[kSplitJobs];
  int batches[kSplitJobs], rows[kSplitJobs], cols[kSplitJobs], k_is_col[kSplitJobs];
  // src and add read through a strided view (batch, row, col strides; all
  // zero: the plain [batches][rows][cols] index of the other arrays).
  size_t view[kSplitJobs][3];
  size_t begin[kSplitJobs + 1];  // lanes of the jobs before (set by launch_split)
  int count;
};

static_assert(sizeof(SplitArgs) <= 4096, "kernel argument block must fit in 4 KB");

// Row-side operands (k_is_col: k runs along a source row) take one lane per
// 4 consecutive k of one plane row: 4 adjacent words in, consecutive lanes
// writing consecutive 4-byte groups.  Column-side operands take one lane per
// kColK (4 or 16) k of one plane row: kColK words a source row apart, the
// 32 / kColK lanes of a 32-byte plane segment adjacent (k fastest, then the
// column), so that every segment of every plane is written whole by one
// wave's kColK-byte stores (never assembled from partial writes of lanes in
// other workgroups).  16 k per lane reads 32 columns of 2 row groups per
// wave; 4 k per lane gives four times the lanes, for launches too small to
// fill the chip at 16.
// Element i (plain index) whose src / add index is iv (the view's).
__device__ __forceinline__ uint64_t split_val(const SplitArgs& a, int j, size_t i, size_t iv) {
  uint64_t v = a.src[j][iv];
  if (a.add[j]) v += a.add[j][iv];
  if (a.sub[j][0]) v -= a.sub[j][0][i];
  if (a.sub[j][1]) v -= a.sub[j][1][i];
  return v;
}

// The view index of element (b, r, c), or its plain index without a view.
__device__ __forceinline__ size_t view_index(const SplitArgs& a, int j, size_t b, size_t r,
                                             size_t c, size_t plain) {
  const size_t(&st)[3] = a.view[j];
  return (st[0] | st[1] | st[2]) ? b * st[0] + r * st[1] + c * st[2] : plain;
}

// kN consecutive k of one plane row (v[t], t < kN): one kN-byte store per plane.
template <int kN>
__device__ __forceinline__ void write_k(int8_t* planes, size_t plane, size_t off,
                                        const uint64_t (&v)[kN]) {
  static_assert(kN == 1 || kN == 2 || kN == 4 || kN == 16, "1, 2, 4 or 16 k per store");
  uint32_t pk[kDigitPlanes][(kN + 3) / 4] = {};
#pragma unroll
  for (int t = 0; t < kN; ++t) {
    uint32_t d[kDigitPlanes];
    digits8(v[t], d);
#pragma unroll
    for (int i = 0; i < kDigitPlanes; ++i) pk[i][t >> 2] |= d[i] << (8 * (t & 3));
  }
#pragma unroll
  for (int i = 0; i < kDigitPlanes; ++i) {
    if constexpr (kN == 1)
      planes[i * plane + off] = int8_t(pk[i][0]);
    else if constexpr (kN == 2)
      *reinterpret_cast<uint16_t*>(planes + i * plane + off) = uint16_t(pk[i][0]);
    else if constexpr (kN == 4)
      *reinterpret_cast<uint32_t*>(planes + i * plane + off) = pk[i][0];
    else
      *reinterpret_cast<uint4*>(planes + i * plane + off) =
          make_uint4(pk[i][0], pk[i][1], pk[i][2], pk[i][3]);
  }
}

// Lanes first, first + stride, ... of a split launch over `a`.
template <int kColK, int kRowK>
__device__ __forceinline__ void split_lanes(const SplitArgs& a, size_t first, size_t stride) {
  const size_t total = a.begin[a.count];
  for (size_t g = first; g < total; g += stride) {
    int j = 0;
    while (j + 1 < a.count && g >= a.begin[j + 1]) ++j;
    const size_t q = g - a.begin[j];
    const int rows = a.rows[j], cols = a.cols[j];
    const bool kc = a.k_is_col[j] != 0;
    const int K = kc ? cols : rows, R = kc ? rows : cols;
    const size_t plane = size_t(a.batches[j]) * R * K;
    if (kc) {
      const size_t per_batch = size_t(R) * (K / kRowK);
      const size_t b = q / per_batch, rem = q % per_batch;
      const int r = int(rem / (K / kRowK)), k = kRowK * int(rem % (K / kRowK));
      const size_t src = b * size_t(rows) * cols + size_t(r) * cols + k;
      const size_t off = b * size_t(R) * K + kblock_off(size_t(r), k, size_t(R));
      const size_t sv = view_index(a, j, b, size_t(r), size_t(k), src);
      const size_t cs = (a.view[j][0] | a.view[j][1] | a.view[j][2]) ? a.view[j][2] : 1;
      uint64_t v[kRowK];
#pragma unroll
      for (int t = 0; t < kRowK; ++t) v[t] = split_val(a, j, src + t, sv + t * cs);
      write_k<kRowK>(a.planes[j], plane, off, v);
      if (a.planes_a0[j]) {
#pragma unroll
        for (int t = 0; t < kRowK; ++t) v[t] += a.a0[j][src + t];
        write_k<kRowK>(a.planes_a0[j], plane, off, v);
      }
    } else {
      constexpr int kSeg = 32 / kColK;  // lanes per 32-byte plane segment
      const size_t per_batch = size_t(R) * (K / kColK);
      const size_t b = q / per_batch, rem = q % per_batch;
      const int kq = int(rem % kSeg), kb = int(rem / (kSeg * size_t(R)));
      const int r = int((rem / kSeg) % size_t(R));
      const int k0 = 32 * kb + kColK * kq;
      const size_t src = b * size_t(rows) * cols + size_t(k0) * cols + r;
      const size_t off = b * size_t(R) * K + kblock_off(size_t(r), k0, size_t(R));
      const size_t sv = view_index(a, j, b, size_t(k0), size_t(r), src);
      const size_t rs = (a.view[j][0] | a.view[j][1] | a.view[j][2]) ? a.view[j][1] : size_t(cols);
      uint64_t v[kColK];
#pragma unroll
      for (int t = 0; t < kColK; ++t)
        v[t] = split_val(a, j, src + size_t(t) * cols, sv + size_t(t) * rs);
      write_k<kColK>(a.planes[j], plane, off, v);
      if (a.planes_a0[j]) {
#pragma unroll
        for (int t = 0; t < kColK; ++t) v[t] += a.a0[j][src + size_t(t) * cols];
        write_k<kColK>(a.planes_a0[j], plane, off, v);
      }
    }
  }
}

template <int kColK, int kRowK>
__global__ void __launch_bounds__(256) kb_split_kernel(SplitArgs a) {
  split_lanes<kColK, kRowK>(a, size_t(blockIdx.x) * 256 + threadIdx.x, size_t(gridDim.x) * 256);
}

// The opens' digit planes and the key-only walks of truncation gates in one
// launch: workgroups below walk_groups walk (a 16-copy T table in LDS, every
// level walked, 8 lanes per walk, as trunc_batch_walk_kernel with no local
// levels), the others split.  Neither role waits for the other, so the
// walks' dependent levels run under the split's memory stream.
constexpr int kFusedWalkJobs = 8;
constexpr int kFusedCopies = 16;
using FusedAes = AesLds<kFusedCopies>;

struct SplitWalkArgs {
  SplitArgs s;
  WalkJobs<kFusedWalkJobs> w;
  uint32_t walk_groups;
  // Column-side jobs split by tiles (split_tile): tiles [tbegin[t],
  // tbegin[t + 1]) belong to job tjob[t]; their workgroups follow the walk's.
  int tcount;
  int tjob[kSplitJobs];
  uint32_t tbegin[kSplitJobs + 1];
  uint32_t tile_groups;
};

// Column-side jobs (k runs along the source rows) by 32 (k) x 64 (column)
// tiles through LDS: each wave reads 64 consecutive columns of one row (512
// contiguous bytes per source array), the workgroup forms the values in LDS,
// and lane (column c, quarter q) writes bytes 8 q .. 8 q + 7 of column c's
// 32-byte plane segment, so four adjacent lanes write a segment whole and a
// wave 512 contiguous bytes per plane.  The lane form reads 16 rows per lane
// (two 256-byte runs per wave and load).
constexpr int kTileK = 32, kTileN = 64;
using SplitTile = uint64_t[kTileK][kTileN + 1];  // + 1: the column reads spread over banks

__device__ __forceinline__ void split_tile(const SplitArgs& a, int j, uint32_t tile,
                                           SplitTile& E) {
  const int K = a.rows[j], N = a.cols[j];
  const uint32_t tn = uint32_t(N / kTileN), per_b = tn * uint32_t(K / kTileK);
  const uint32_t b = tile / per_b, rem = tile - b * per_b;
  const int kb = int(rem / tn), nb = int(rem - (rem / tn) * tn);
  const size_t bk = size_t(b) * size_t(K) * size_t(N);
  const size_t base = bk + size_t(kb) * kTileK * N + size_t(nb) * kTileN;
  uint64_t v[kTileK * kTileN / 256];
#pragma unroll
  for (int i = 0; i < kTileK * kTileN / 256; ++i) {
    const int e = int(threadIdx.x) + 256 * i;
    const size_t idx = base + size_t(e / kTileN) * N + (e % kTileN);
    v[i] = split_val(a, j, idx, idx);
  }
  __syncthreads();  // the previous tile's column reads are done
#pragma unroll
  for (int i = 0; i < kTileK * kTileN / 256; ++i) {
    const int e = int(threadIdx.x) + 256 * i;
    E[e / kTileN][e % kTileN] = v[i];
  }
  __syncthreads();
  const int c = int(threadIdx.x >> 2), q = int(threadIdx.x & 3);
  uint32_t pk[kDigitPlanes][2] = {};
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    uint32_t d[kDigitPlanes];
    digits8(E[8 * q + t][c], d);
#pragma unroll
    for (int i = 0; i < kDigitPlanes; ++i) pk[i][t >> 2] |= d[i] << (8 * (t & 3));
  }
  const size_t plane = size_t(a.batches[j]) * size_t(K) * size_t(N);
  const size_t off = bk + kblock_off(size_t(nb) * kTileN + c, kTileK * kb + 8 * q, size_t(N));
#pragma unroll
  for (int i = 0; i < kDigitPlanes; ++i)
    *reinterpret_cast<uint2*>(a.planes[j] + i * plane + off) = make_uint2(pk[i][0], pk[i][1]);
}

// Walks (workgroups below walk_groups, with kWalk), tiles (the next
// tile_groups, one tile each: more tiles per workgroup measured slower), then
// the other jobs' lanes at 4 k per lane.  Beside the walks the tiles beat the
// lane form (25.7 against 26.6 us at config 3's shape); alone they do not
// (22.0 against 20.6 us for the triples' planes), so only the launch with
// walks uses them.
template <bool kWalk>
__global__ void __launch_bounds__(256) kb_split_tiled_kernel(SplitWalkArgs a) {
  __shared__ SplitTile E;
  const uint32_t wg = kWalk ? a.walk_groups : 0u;
  if constexpr (kWalk) {
    __shared__ __align__(16) uint32_t tab[FusedAes::kWords];
    __shared__ uint4 rkl[4 * 11];
    if (blockIdx.x < wg) {
      fill_ttable<kFusedCopies>(tab, kTDev.v);
      fill_round_keys(rkl, a.w.prg.rk, 4);
      __syncthreads();
      const FusedAes aes{tab, threadIdx.x % kFusedCopies};
      const uint32_t gl = blockIdx.x * 256 + threadIdx.x;
      const uint32_t g = gl >> 3;  // walk; whole 8-lane groups leave together
      if (g >= a.w.begin[a.w.count]) return;
      const int j = batch_job<kFusedWalkJobs>(a.w.begin, a.w.count, g);
      walk_leaf_path(aes, rkl, a.w.key[j], a.w.out[j], a.w.geo[j], g - a.w.begin[j], gl);
      return;
    }
  }
  if (blockIdx.x < wg + a.tile_groups) {
    const uint32_t total = a.tbegin[a.tcount];
    for (uint32_t t = blockIdx.x - wg; t < total; t += a.tile_groups) {
      int u = 0;
      while (u + 1 < a.tcount && t >= a.tbegin[u + 1]) ++u;
      split_tile(a.s, a.tjob[u], t - a.tbegin[u], E);
    }
    return;
  }
  const uint32_t first = wg + a.tile_groups;
  split_lanes<4, 4>(a.s, size_t(blockIdx.x - first) * 256 + threadIdx.x,
                    size_t(gridDim.x - first) * 256);
}

static_assert(sizeof(SplitWalkArgs) <= 4096, "kernel argument block must fit in 4 KB");

template <int kColK, int kRowK>
__global__ void __launch_bounds__(256) kb_split_walk_kernel(SplitWalkArgs a) {
  __shared__ __align__(16) uint32_t tab[FusedAes::kWords];
  __shared__ uint4 rkl[4 * 11];
  if (blockIdx.x < a.walk_groups) {
    fill_ttable<kFusedCopies>(tab, kTDev.v);
    fill_round_keys(rkl, a.w.prg.rk, 4);
    __syncthreads();
    const FusedAes aes{tab, threadIdx.x % kFusedCopies};
    const uint32_t gl = blockIdx.x * 256 + threadIdx.x;
    const uint32_t g = gl >> 3;  // walk; whole 8-lane groups leave together
    if (g >= a.w.begin[a.w.count]) return;
    const int j = batch_job<kFusedWalkJobs>(a.w.begin, a.w.count, g);
    walk_leaf_path(aes, rkl, a.w.key[j], a.w.out[j], a.w.geo[j], g - a.w.begin[j], gl);
    return;
  }
  split_lanes<kColK, kRowK>(a.s, size_t(blockIdx.x - a.walk_groups) * 256 + threadIdx.x,
                            size_t(gridDim.x - a.walk_groups) * 256);
}

struct Bm2Args {
  const int8_t* D;     // LHS planes [8][b][K/32][M][32]
  const int8_t* E;     // RHS planes [8][b][K/32][N][32]
  const int8_t* A[2];  // LHS
  const int8_t* B[2];  // RHS
  const uint64_t* C[2];
  uint64_t* out[2];
  int batches, M, K, N;
  int merge;        // outputs at [m][b N + n] instead of [b][m][n]
  TruncEpi epi;     // on: the open + mask feeds this gate, whose outputs are written
  uint64_t mask;
  sufhip_x_planes xp;  // optional digit planes of the (truncated) outputs, merged layout
  const int8_t* X;     // balanced form: LHS planes of D + A_0
};

// Party p's finished 32 x 32 tile values (lane l: column l % 32, rows of
// the accumulator layout) to out_p, and to the output digit planes.
__device__ __forceinline__ void bm2_store(const Bm2Args& a, int p, int l, int m0, int n0, size_t b,
                                          const uint64_t (&v)[16]) {
  const int M = a.M, N = a.N;
  const int col = n0 + (l & 31);
  const size_t ob = b * size_t(M) * N;
  const size_t ld = size_t(a.batches) * N;  // merged row length
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = m0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    const size_t o = a.merge ? size_t(row) * ld + b * N + col : ob + size_t(row) * N + col;
    a.out[p][o] = v[r];
    if (a.xp.planes) put_x_digits(a.xp, size_t(M), o, p, v[r]);
  }
}

// With the truncation epilogue: both parties' tiles are in LDS (both[p]);
// wave p opens rows r in [8p, 8p + 8) and writes both parties' outputs.
// eh: the gate's key headers, read before the kernel's first global store;
// every table read is issued before the first output store.
__device__ __forceinline__ void bm2_trunc_rows(const Bm2Args& a, const EpiHdrs& eh, int p, int l,
                                               int m0, int n0, size_t b,
                                               const uint64_t (*both)[16][64]) {
  const int M = a.M, N = a.N;
  const int col = n0 + (l & 31);
  const size_t ob = b * size_t(M) * N;
  const size_t ld = size_t(a.batches) * N;
  uint64_t open[8], w[8][2];
  size_t o[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int r = 8 * p + q;
    const int row = m0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    o[q] = a.merge ? size_t(row) * ld + b * N + col : ob + size_t(row) * N + col;
    open[q] = both[0][r][l] + both[1][r][l] + a.mask;
    w[q][0] = trunc_table_word(eh.h[0], a.epi.table[0], a.epi.f, open[q]);
    w[q][1] = trunc_table_word(eh.h[1], a.epi.table[1], a.epi.f, open[q]);
  }
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const uint64_t y0 = trunc_table_out(eh.h[0], a.epi.f, open[q], w[q][0]);
    const uint64_t y1 = trunc_table_out(eh.h[1], a.epi.f, open[q], w[q][1]);
    a.epi.y[0][o[q]] = y0;
    a.epi.y[1][o[q]] = y1;
    if (a.xp.planes) {
      put_x_digits(a.xp, size_t(M), o[q], 0, y0);
      put_x_digits(a.xp, size_t(M), o[q], 1, y1);
    }
  }
}

// Waves per party: k-steps st, st + kKWaves, ... go to wave st % kKWaves, so
// up to kKWaves steps' loads and MFMAs run at once; the partial tiles are
// added through LDS.
constexpr int kKWaves = 2;

__global__ void __launch_bounds__(128 * kKWaves) beaver_mfma2_kernel(Bm2Args a) {
  __shared__ uint64_t part[kKWaves - 1][2][16][64];
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int p = w & 1, kw = w >> 1, kws = blockDim.x / 128;
  const int M = a.M, K = a.K, N = a.N;
  const int n0 = blockIdx.x * 32, m0 = blockIdx.y * 32;
  const size_t b = blockIdx.z;
  const size_t lplane = size_t(a.batches) * M * K, rplane = size_t(a.batches) * N * K;
  const size_t lb = b * size_t(M) * K + size_t(m0 + (l & 31)) * 32 + 16 * (l >> 5);
  const size_t rb = b * size_t(N) * K + size_t(n0 + (l & 31)) * 32 + 16 * (l >> 5);
  const size_t lstep = size_t(M) * 32, rstep = size_t(N) * 32;
  const int8_t* Ap = a.A[p];
  const int8_t* Bp = a.B[p];
  v16i acc[kDigitPlanes];
#pragma unroll
  for (int s = 0; s < kDigitPlanes; ++s)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[s][r] = 0;
  const int steps = K / 32;
  for (int st = kw; st < steps; st += kws) {
    v4i d[kDigitPlanes], e[kDigitPlanes], x[kDigitPlanes], y[kDigitPlanes];
#pragma unroll
    for (int i = 0; i < kDigitPlanes; ++i) {
      y[i] = load16(Bp + i * rplane + rb + st * rstep);
      d[i] = load16(a.D + i * lplane + lb + st * lstep);
      e[i] = load16(a.E + i * rplane + rb + st * rstep);
      x[i] = load16(Ap + i * lplane + lb + st * lstep);
    }
#pragma unroll
    for (int i = 0; i < kDigitPlanes; ++i)
#pragma unroll
      for (int j = 0; i + j < kDigitPlanes; ++j)
        acc[i + j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(d[i], y[j], acc[i + j], 0, 0, 0);
    if (p == 0) {
#pragma unroll
      for (int i = 0; i < kDigitPlanes; ++i)
#pragma unroll
        for (int j = 0; i + j < kDigitPlanes; ++j)
          acc[i + j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(d[i], e[j], acc[i + j], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < kDigitPlanes; ++i)
#pragma unroll
      for (int j = 0; i + j < kDigitPlanes; ++j)
        acc[i + j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x[i], e[j], acc[i + j], 0, 0, 0);
  }
  const EpiHdrs eh = epi_hdrs(a.epi);
  uint64_t v[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    v[r] = 0;
#pragma unroll
    for (int s = 0; s < kDigitPlanes; ++s) v[r] += uint64_t(int64_t(acc[s][r])) << (8 * s);
  }
  if (kw > 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) part[kw - 1][p][r][l] = v[r];
  }
  __syncthreads();
  const int col = n0 + (l & 31);
  const size_t ob = b * size_t(M) * N;
  if (kw == 0) {
    for (int q = 1; q < kws; ++q) {
#pragma unroll
      for (int r = 0; r < 16; ++r) v[r] += part[q - 1][p][r][l];
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
      v[r] += a.C[p][ob + size_t(row) * N + col];
    }
  }
  if (!a.epi.on) {
    if (kw == 0) bm2_store(a, p, l, m0, n0, b, v);
    return;
  }
  // The open out_0 + out_1 + mask through LDS (the slices' buffer is free
  // again); wave p then finishes rows r in [8p, 8p + 8) for both parties.
  __syncthreads();
  uint64_t(*both)[16][64] = part[0];
  static_assert(kKWaves >= 2, "the open reuses the slices' LDS");
  if (kw == 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) both[p][r][l] = v[r];
  }
  __syncthreads();
  if (kw == 0) bm2_trunc_rows(a, eh, p, l, m0, n0, b, both);
}

// Balanced form (Xp given): wave p computes party p's tile over every
// k-step as two operand products, (L_p, E) with L_0 = D + A_0 and L_1 = A_1,
// then (D, B_p): 72 MFMAs per party and step, so the two waves of a tile
// finish together.  The operand pairs run through a register pipeline
// kStages deep (a pair's planes are loaded kStages - 1 pairs before its
// MFMAs), which keeps loads in flight while the wave -- the only one on its
// SIMD -- multiplies.  Bases are wave-uniform (scalar registers) plus each
// lane's 32-bit fragment offset.  kPrefC (short K, three stages): the
// wave's 16 C_p words are loaded with the first operand pairs, so the tile
// needs no memory round trip after the k-loop (four stages leave no
// registers for them).
template <int kStages, bool kPrefC>
__global__ void __launch_bounds__(128, 1) beaver_bal_kernel(Bm2Args a) {
  __shared__ uint64_t both[2][16][64];
  const int l = threadIdx.x & 63;
  const int p = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int M = a.M, K = a.K, N = a.N;
  const int n0 = blockIdx.x * 32, m0 = blockIdx.y * 32;
  const size_t b = blockIdx.z;
  // Byte offsets within the operands' planes fit 32 bits (checked on the host).
  const uint32_t lplane = uint32_t(a.batches) * M * K, rplane = uint32_t(a.batches) * N * K;
  const uint32_t lstep = uint32_t(M) * 32, rstep = uint32_t(N) * 32;
  const uint32_t fo = uint32_t(l & 31) * 32 + 16 * uint32_t(l >> 5);
  const uint32_t lb0 = uint32_t(b) * M * K + uint32_t(m0) * 32;
  const uint32_t rb0 = uint32_t(b) * N * K + uint32_t(n0) * 32;
  const int8_t* Lx = (p == 0 ? a.X : a.A[1]) + lb0;
  const int8_t* Ld = a.D + lb0;
  const int8_t* Re = a.E + rb0;
  const int8_t* Rb = (p == 0 ? a.B[0] : a.B[1]) + rb0;
  const int col = n0 + (l & 31);
  const size_t ob = b * size_t(M) * N;
  uint64_t cpre[16];
  if constexpr (kPrefC) {
#pragma unroll
    for (int r = 0; r < 16; ++r)
      cpre[r] = a.C[p][ob + size_t(m0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3)) * N + col];
  }
  v16i acc[kDigitPlanes];
#pragma unroll
  for (int s = 0; s < kDigitPlanes; ++s)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[s][r] = 0;
  // Operand pairs u = 2 step + (0: (L_p, E), 1: (D, B_p)).  The loop runs
  // over whole groups of kStages pairs; loads past the last pair repeat it
  // (in bounds) and their MFMAs are skipped.
  const int U = 2 * (K / 32);
  const int Ug = (U + kStages - 1) / kStages * kStages;
  v4i L[kStages][kDigitPlanes], R[kStages][kDigitPlanes];
  auto issue = [&](int q, int u) {
    u = u < U ? u : U - 1;
    const uint32_t st = uint32_t(u >> 1);
    const int8_t* lb = (u & 1) ? Ld : Lx;
    const int8_t* rb = (u & 1) ? Rb : Re;
#pragma unroll
    for (int i = 0; i < kDigitPlanes; ++i) {
      L[q][i] = load16(lb + (i * lplane + st * lstep) + fo);
      R[q][i] = load16(rb + (i * rplane + st * rstep) + fo);
    }
  };
#pragma unroll
  for (int q = 0; q < kStages - 1; ++q) issue(q, q);
  for (int u0 = 0; u0 < Ug; u0 += kStages) {
#pragma unroll
    for (int h = 0; h < kStages; ++h) {
      const int u = u0 + h;
      issue((h + kStages - 1) % kStages, u + kStages - 1);
      if (u < U) {
#pragma unroll
        for (int i = 0; i < kDigitPlanes; ++i)
#pragma unroll
          for (int j = 0; i + j < kDigitPlanes; ++j)
            acc[i + j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(L[h][i], R[h][j], acc[i + j], 0,
                                                              0, 0);
      }
    }
  }
  const EpiHdrs eh = epi_hdrs(a.epi);
  uint64_t v[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    v[r] = 0;
#pragma unroll
    for (int s = 0; s < kDigitPlanes; ++s) v[r] += uint64_t(int64_t(acc[s][r])) << (8 * s);
    const int row = m0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    v[r] += kPrefC ? cpre[r] : a.C[p][ob + size_t(row) * N + col];
  }
  if (!a.epi.on) {
    bm2_store(a, p, l, m0, n0, b, v);
    return;
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) both[p][r][l] = v[r];
  __syncthreads();
  bm2_trunc_rows(a, eh, p, l, m0, n0, b, both);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace sufhip

using namespace sufhip;

namespace sufhip {
namespace {

// Shape checks and lane count of split job j (sources already set).
int split_job(SplitArgs& a, int j, int8_t* planes, int batches, int rows, int cols,
              int k_is_col, int8_t* planes_a0, const uint64_t* a0, const char* what) {
  const bool shape = batches >= 1 && rows >= 32 && cols >= 32 && rows % 32 == 0 &&
                     cols % 32 == 0;
  if (!shape || !planes || !aligned16(planes) || !aligned16(planes_a0)) {
    set_error(std::string(what) +
              ": batches >= 1, rows and cols multiples of 32, planes 16-byte aligned");
    return SUFHIP_ERR_INVALID;
  }
  if ((planes_a0 == nullptr) != (a0 == nullptr)) {
    set_error(std::string(what) + ": planes_a0 and a0 go together");
    return SUFHIP_ERR_INVALID;
  }
  a.planes[j] = planes;
  a.planes_a0[j] = planes_a0;
  a.a0[j] = a0;
  a.batches[j] = batches;
  a.rows[j] = rows;
  a.cols[j] = cols;
  a.k_is_col[j] = k_is_col ? 1 : 0;
  return SUFHIP_OK;
}

// SplitArgs of sufhip_kb_open_split_batch's jobs.
int open_split_args(const sufhip_kb_open_job* jobs, int count, SplitArgs& a, const char* what) {
  auto fail = [&](const char* msg) {
    set_error(std::string(what) + ": " + msg);
    return SUFHIP_ERR_INVALID;
  };
  if (count < 0 || count > kSplitJobs || (count > 0 && !jobs))
    return fail("0..SUFHIP_KB_SPLIT_JOBS jobs");
  for (int j = 0; j < count; ++j) {
    const sufhip_kb_open_job& jb = jobs[j];
    if (!jb.a[0] || !jb.a[1]) return fail("null share a[0] or a[1]");
    if ((jb.b[0] == nullptr) != (jb.b[1] == nullptr)) return fail("give both shares of b or neither");
    if (jb.a_stride[0] < 0 || jb.a_stride[1] < 0 || jb.a_stride[2] < 0)
      return fail("a_stride entries must be >= 0");
    a.src[j] = jb.a[0];
    a.add[j] = jb.a[1];
    a.sub[j][0] = jb.b[0];
    a.sub[j][1] = jb.b[1];
    for (int t = 0; t < 3; ++t) a.view[j][t] = size_t(jb.a_stride[t]);
    if (int rc = split_job(a, j, jb.planes, jb.batches, jb.rows, jb.cols, jb.k_is_col,
                           jb.planes_a0, jb.a0, what))
      return rc;
  }
  return SUFHIP_OK;
}

// Column-side jobs take 16 k per lane when that still gives two waves per
// SIMD, else 4 (more lanes, shorter per-lane chains); launches of fewer than
// two waves per SIMD at 4 k per lane take one k per lane on both sides (the
// most lanes, no serial loads per lane).  Sets a.count and a.begin; *ck and
// *rk: k per lane on the column and row side.
void plan_split(SplitArgs& a, int count, int* ck, int* rk) {
  a.count = count;
  int cus = 256;
  int dev = 0;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  size_t col16 = 0;
  for (int j = 0; j < count; ++j)
    if (!a.k_is_col[j]) col16 += size_t(a.batches[j]) * a.rows[j] * a.cols[j] / 16;
  const size_t two_waves = size_t(cus) * 4 * 64 * 2;
  size_t n4 = 0;  // lanes at 4 k per lane
  for (int j = 0; j < count; ++j) n4 += size_t(a.batches[j]) * a.rows[j] * a.cols[j] / 4;
  *ck = col16 >= two_waves ? 16 : (n4 < two_waves ? 1 : 4);
  *rk = *ck == 1 ? 1 : 4;
  a.begin[0] = 0;
  for (int j = 0; j < count; ++j)
    a.begin[j + 1] = a.begin[j] + size_t(a.batches[j]) * a.rows[j] * a.cols[j] /
                                      size_t(a.k_is_col[j] ? *rk : *ck);
}

// Column-side jobs go by tiles (split_tile) when the launch is large enough
// for 16 k per lane and every such job is plain (no view), without the
// planes of + a0, and has a multiple of 64 columns.  Fills f's tile fields
// and gives those jobs no lanes in f.s.begin (the other jobs keep theirs at
// 4 k per lane); false leaves f untouched.
bool plan_tiles(SplitWalkArgs& f, int count, int ck) {
  SplitArgs& a = f.s;
  if (ck != 16) return false;
  int n = 0;
  for (int j = 0; j < count; ++j) {
    if (a.k_is_col[j]) continue;
    if ((a.view[j][0] | a.view[j][1] | a.view[j][2]) || a.planes_a0[j] || a.cols[j] % kTileN)
      return false;
    ++n;
  }
  if (n == 0) return false;
  f.tcount = 0;
  f.tbegin[0] = 0;
  a.begin[0] = 0;
  for (int j = 0; j < count; ++j) {
    const size_t elems = size_t(a.batches[j]) * a.rows[j] * a.cols[j];
    if (a.k_is_col[j]) {
      a.begin[j + 1] = a.begin[j] + elems / 4;
      continue;
    }
    a.begin[j + 1] = a.begin[j];
    f.tjob[f.tcount] = j;
    f.tbegin[f.tcount + 1] = f.tbegin[f.tcount] + uint32_t(elems / (kTileK * kTileN));
    ++f.tcount;
  }
  int cus = 256, dev = 0;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const uint32_t tiles = f.tbegin[f.tcount], cap = uint32_t(cus) * 8;
  f.tile_groups = tiles < cap ? tiles : cap;
  return true;
}

template <bool kWalk>
int launch_tiled(SplitWalkArgs& f, void* stream) {
  size_t g = (f.s.begin[f.s.count] + 255) / 256;
  if (g > 4096) g = 4096;
  const size_t wg = kWalk ? f.walk_groups : 0;
  hipLaunchKernelGGL((kb_split_tiled_kernel<kWalk>), dim3(unsigned(wg + f.tile_groups + g)),
                     dim3(256), 0, as_stream(stream), f);
  return check_launch("kb_split_tiled_kernel");
}

int launch_split(SplitArgs& a, int count, void* stream) {
  int ck = 0, rk = 0;
  plan_split(a, count, &ck, &rk);
  if (a.begin[count] == 0) return SUFHIP_OK;
  size_t g = (a.begin[count] + 255) / 256;
  if (g > 4096) g = 4096;
  if (ck == 16)
    hipLaunchKernelGGL((kb_split_kernel<16, 4>), dim3(unsigned(g)), dim3(256), 0,
                       as_stream(stream), a);
  else if (ck == 4)
    hipLaunchKernelGGL((kb_split_kernel<4, 4>), dim3(unsigned(g)), dim3(256), 0,
                       as_stream(stream), a);
  else
    hipLaunchKernelGGL((kb_split_kernel<1, 1>), dim3(unsigned(g)), dim3(256), 0,
                       as_stream(stream), a);
  return check_launch("kb_split_kernel");
}

// The split of `a` (count jobs) with the walk of `w` in one launch.
int launch_split_walk(SplitWalkArgs& f, int count, void* stream) {
  int ck = 0, rk = 0;
  plan_split(f.s, count, &ck, &rk);
  const size_t walk_lanes_n = 8 * size_t(f.w.begin[f.w.count]);
  const size_t wg = (walk_lanes_n + 255) / 256;
  f.walk_groups = uint32_t(wg);
  if (plan_tiles(f, count, ck)) return launch_tiled<true>(f, stream);
  size_t g = (f.s.begin[count] + 255) / 256;
  if (g > 4096) g = 4096;
  if (wg + g == 0) return SUFHIP_OK;
  const dim3 grid(unsigned(wg + (g > 0 ? g : 0)));
  if (ck == 16)
    hipLaunchKernelGGL((kb_split_walk_kernel<16, 4>), grid, dim3(256), 0, as_stream(stream), f);
  else if (ck == 4)
    hipLaunchKernelGGL((kb_split_walk_kernel<4, 4>), grid, dim3(256), 0, as_stream(stream), f);
  else
    hipLaunchKernelGGL((kb_split_walk_kernel<1, 1>), grid, dim3(256), 0, as_stream(stream), f);
  return check_launch("kb_split_walk_kernel");
}

}  // namespace
}  // namespace sufhip

extern "C" {

size_t sufhip_kb_planes_bytes(int batches, int rows, int cols) {
  if (batches < 1 || rows < 1 || cols < 1 || rows % 32 || cols % 32) return 0;
  return size_t(kDigitPlanes) * size_t(batches) * size_t(rows) * size_t(cols);
}

int sufhip_kb_split_batch(const sufhip_kb_split_job* jobs, int count, void* stream) {
  SUFHIP_REQUIRE(count >= 0 && count <= kSplitJobs && (count == 0 || jobs),
                 "sufhip_kb_split_batch: 0..SUFHIP_KB_SPLIT_JOBS jobs");
  SplitArgs a{};
  for (int j = 0; j < count; ++j) {
    const sufhip_kb_split_job& jb = jobs[j];
    SUFHIP_REQUIRE(jb.src, "sufhip_kb_split_batch: null source");
    a.src[j] = jb.src;
    if (int rc = split_job(a, j, jb.planes, jb.batches, jb.rows, jb.cols, jb.k_is_col,
                           jb.planes_a0, jb.a0, "sufhip_kb_split_batch"))
      return rc;
  }
  return launch_split(a, count, stream);
}

int sufhip_kb_open_split_batch(const sufhip_kb_open_job* jobs, int count, void* stream) {
  SplitArgs a{};
  if (int rc = open_split_args(jobs, count, a, "sufhip_kb_open_split_batch")) return rc;
  return launch_split(a, count, stream);
}

int sufhip_kb_open_split_prepare(const sufhip_kb_open_job* jobs, int count,
                                 const uint8_t* prg_state, const sufhip_trunc_job* tjobs,
                                 int tcount, void* stream) {
  SplitWalkArgs f{};
  if (int rc = open_split_args(jobs, count, f.s, "sufhip_kb_open_split_prepare")) return rc;
  bool one = false;
  if (int rc = trunc_walk_plan(prg_state, tjobs, tcount, kFusedWalkJobs, f.w.begin, f.w.key,
                               f.w.out, f.w.geo, &one))
    return rc;
  if (!one) {
    // Jobs that need the prepare's own launches (expansion levels, local
    // levels, more than kFusedWalkJobs jobs): those first, then the split.
    if (int rc = sufhip_trunc_prepare_batch(prg_state, tjobs, tcount, stream)) return rc;
    return launch_split(f.s, count, stream);
  }
  fill_prg4(prg_state, &f.w.prg);
  f.w.count = tcount;
  return launch_split_walk(f, count, stream);
}

int sufhip_beaver_matmul2_mfma_ex(const sufhip_beaver_mfma2_args* args, void* stream) {
  SUFHIP_REQUIRE(args != nullptr, "sufhip_beaver_matmul2_mfma_ex: null args");
  const sufhip_beaver_mfma2_args& g = *args;
  const char* what = "sufhip_beaver_matmul2_mfma_ex";
  SUFHIP_REQUIRE(g.batches >= 0 && g.batches <= 65535 && g.M >= 0 && g.N >= 0 && g.K >= 0 &&
                     g.M % 32 == 0 && g.N % 32 == 0 && g.K % 32 == 0 && g.K <= kMaxBeaverK,
                 "sufhip_beaver_matmul2_mfma_ex: M, K, N multiples of 32, K <= 4096");
  if (g.batches == 0 || g.M == 0 || g.N == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(g.Dp && g.Ep && g.Ap[0] && g.Ap[1] && g.Bp[0] && g.Bp[1] && g.C[0] && g.C[1],
                 "sufhip_beaver_matmul2_mfma_ex: null operand");
  SUFHIP_REQUIRE(aligned16(g.Dp) && aligned16(g.Ep) && aligned16(g.Ap[0]) &&
                     aligned16(g.Ap[1]) && aligned16(g.Bp[0]) && aligned16(g.Bp[1]),
                 "sufhip_beaver_matmul2_mfma_ex: planes must be 16-byte aligned");
  const size_t n = size_t(g.batches) * g.M * g.N;
  Bm2Args a{g.Dp, g.Ep, {g.Ap[0], g.Ap[1]}, {g.Bp[0], g.Bp[1]}, {g.C[0], g.C[1]},
            {g.out[0], g.out[1]}, g.batches, g.M, g.K, g.N, g.merge_heads ? 1 : 0, TruncEpi{},
            g.mask, g.out_planes, g.Xp};
  if (int rc = make_epi(g.trunc, n, what, &a.epi)) return rc;
  SUFHIP_REQUIRE(a.epi.on || (g.out[0] && g.out[1]),
                 "sufhip_beaver_matmul2_mfma_ex: outputs (or a truncation) needed");
  SUFHIP_REQUIRE(!a.epi.on || (a.epi.add[0] == nullptr),
                 "sufhip_beaver_matmul2_mfma_ex: the truncation takes no addend");
  SUFHIP_REQUIRE(!g.out_planes.planes ||
                     (g.merge_heads && g.out_planes.cols == g.batches * g.N &&
                      x_planes_ok(g.out_planes, n)),
                 "sufhip_beaver_matmul2_mfma_ex: out_planes need merge_heads, cols = batches N");
  SUFHIP_REQUIRE(aligned16(g.Xp), "sufhip_beaver_matmul2_mfma_ex: planes must be 16-byte aligned");
  const dim3 grid(g.N / 32, g.M / 32, g.batches);
  // The balanced kernel addresses a plane set with 32-bit offsets.
  const uint64_t plane_set = uint64_t(kDigitPlanes) * uint64_t(g.batches) * uint64_t(g.K) *
                             uint64_t(g.M > g.N ? g.M : g.N);
  if (g.Xp && plane_set < (uint64_t(1) << 32)) {
    if (g.K <= 128)  // at most 8 operand pairs
      hipLaunchKernelGGL((beaver_bal_kernel<3, true>), grid, dim3(128), 0, as_stream(stream), a);
    else
      hipLaunchKernelGGL((beaver_bal_kernel<4, false>), grid, dim3(128), 0, as_stream(stream), a);
    return check_launch("beaver_bal_kernel");
  }
  const int steps = g.K / 32;
  const int kws = steps < 2 ? 2 : (steps < kKWaves ? steps : kKWaves);
  hipLaunchKernelGGL(beaver_mfma2_kernel, grid, dim3(128 * kws), 0, as_stream(stream), a);
  return check_launch("beaver_mfma2_kernel");
}

int sufhip_beaver_matmul2_mfma_batched(const int8_t* d_Dp, const int8_t* d_Ep,
                                       const int8_t* d_Ap0, const int8_t* d_Ap1,
                                       const int8_t* d_Bp0, const int8_t* d_Bp1,
                                       const uint64_t* d_C0, const uint64_t* d_C1, int batches,
                                       int M, int K, int N, uint64_t* d_out0, uint64_t* d_out1,
                                       void* stream) {
  SUFHIP_REQUIRE(d_out0 && d_out1, "sufhip_beaver_matmul2_mfma_batched: null pointer");
  sufhip_beaver_mfma2_args g{};
  g.Dp = d_Dp;
  g.Ep = d_Ep;
  g.Ap[0] = d_Ap0;
  g.Ap[1] = d_Ap1;
  g.Bp[0] = d_Bp0;
  g.Bp[1] = d_Bp1;
  g.C[0] = d_C0;
  g.C[1] = d_C1;
  g.batches = batches;
  g.M = M;
  g.K = K;
  g.N = N;
  g.out[0] = d_out0;
  g.out[1] = d_out1;
  return sufhip_beaver_matmul2_mfma_ex(&g, stream);
}

}  // extern "C"
