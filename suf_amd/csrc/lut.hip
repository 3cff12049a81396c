// Interval LUT and packed multi-threshold compare with AES-CTR output masks,
// in the reference CUDA backend's key-blob format (cuda/pfss_backend_gpu.cu:
// 75-94, 189-288) and its kernel counter convention (cuda/pfss_kernels.cu:
// 240-719).
//
// LUT: iv = (upper_bound over cuts[0..intervals) of x) - 1, clamped to
// [0, intervals - 1]; words (w, w+1) of the row are masked by the two halves
// of AES_k(le64(nonce ^ idx << 32 ^ (iv * out_words + w)) || 0^64); party 0
// holds the keystream, party 1 the row minus the keystream (mod 2^64).
// Packed compare: bit j of word w is 1[x < thr_{64 w + j}]; words (w, w+1)
// are masked by AES_k(le64(nonce ^ idx << 32 ^ w / 2) || 0); party 0 holds the
// keystream, party 1 word ^ keystream.
//
// Broadcast keys (one blob for all N inputs): the workgroup stages the round
// keys, cut points / thresholds and (for the LUT) the payload table in LDS
// once, then grid-strides over elements; each lane does its binary search in
// LDS and one AES per two output words with the T table replicated 32 ways.
// Per-element keys: each lane reads its own blob (round keys, cuts, row)
// from HBM.  Geometry (intervals / thresholds, out_words) is fixed by the
// caller and checked against key_bytes on the host, so no lane reads outside
// its key whatever the blob headers hold.
#include <hip/hip_runtime.h>

#include <cstring>
#include <random>

#include "aes_lds.hpp"
#include "operand_device.hpp"
#include "relu_tree_device.hpp"
#include "sufhip_internal.hpp"

namespace sufhip {
namespace {

constexpr int kLutBlock = 256;
constexpr int kLutCopies = 32;
constexpr size_t kLutHdr = 216;
constexpr size_t kPackedHdr = 208;
// LDS staging limits for broadcast keys (u64 words).
constexpr int kMaxCutsLds = 1024;
constexpr int kMaxPayloadLds = 4096;

struct LutArgs {
  const uint8_t* keys;
  const uint64_t* xs;
  uint64_t* out;
  size_t key_bytes;
  size_t n;
  int intervals;
  int out_words;
};

__device__ __forceinline__ uint64_t mask_bits(int bits) {
  return bits <= 0 ? 0 : (bits >= 64 ? ~uint64_t(0) : (uint64_t(1) << bits) - 1);
}

__device__ __forceinline__ uint64_t ld64(const uint8_t* p) {
  return *reinterpret_cast<const uint64_t*>(p);
}

// Round keys of a per-element blob (only 8-byte aligned) into registers.
struct RegKeys {
  uint4 r[11];
};
__device__ __forceinline__ RegKeys load_round_keys(const uint8_t* p) {
  const uint2* q = reinterpret_cast<const uint2*>(p);
  RegKeys k;
#pragma unroll
  for (int i = 0; i < 11; ++i) {
    const uint2 a = q[2 * i], b = q[2 * i + 1];
    k.r[i] = make_uint4(a.x, a.y, b.x, b.y);
  }
  return k;
}

// upper_bound over cuts[0..intervals) of x, minus one, clamped (pfss_kernels.cu:556-574).
template <typename CutAt>
__device__ __forceinline__ int interval_of(uint64_t x, int intervals, uint64_t m,
                                           const CutAt& cut) {
  if (intervals <= 1) return intervals - 1 < 0 ? 0 : intervals - 1;
  int lo = 0, hi = intervals;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if ((cut(mid) & m) <= x)
      lo = mid + 1;
    else
      hi = mid;
  }
  int iv = lo - 1;
  if (iv < 0) iv = 0;
  if (iv >= intervals) iv = intervals - 1;
  return iv;
}

// Round keys in LDS (broadcast keys) or in registers (per-element keys).
__device__ __forceinline__ void keystream(const AesLds<kLutCopies>& aes, const uint4* rk,
                                          uint64_t ctr, uint64_t& k0, uint64_t& k1) {
  uint32_t s0 = uint32_t(ctr), s1 = uint32_t(ctr >> 32), s2 = 0, s3 = 0;
  aes.encrypt(s0, s1, s2, s3, rk);
  k0 = uint64_t(s0) | uint64_t(s1) << 32;
  k1 = uint64_t(s2) | uint64_t(s3) << 32;
}

__device__ __forceinline__ void keystream(const AesLds<kLutCopies>& aes, const RegKeys& rk,
                                          uint64_t ctr, uint64_t& k0, uint64_t& k1) {
  uint32_t s0 = uint32_t(ctr), s1 = uint32_t(ctr >> 32), s2 = 0, s3 = 0;
  aes.encrypt_unrolled(s0, s1, s2, s3, rk.r);
  k0 = uint64_t(s0) | uint64_t(s1) << 32;
  k1 = uint64_t(s2) | uint64_t(s3) << 32;
}

template <typename RK>
__device__ __forceinline__ void write_masked_row(const AesLds<kLutCopies>& aes, const RK& rk,
                                                 uint64_t nonce, size_t idx, int iv, int ow,
                                                 int party, const uint64_t* row, uint64_t* out) {
  for (int w = 0; w < ow; w += 2) {
    const uint64_t ctr = nonce ^ (uint64_t(idx) << 32) ^ (uint64_t(iv) * uint64_t(ow) + uint64_t(w));
    uint64_t k0, k1;
    keystream(aes, rk, ctr, k0, k1);
    out[w] = party == 0 ? k0 : row[w] - k0;
    if (w + 1 < ow) out[w + 1] = party == 0 ? k1 : row[w + 1] - k1;
  }
}

// Broadcast key: header, round keys, cuts and payload staged in LDS.
__global__ void __launch_bounds__(kLutBlock) lut_bcast_kernel(LutArgs a) {
  __shared__ __align__(16) uint32_t tab[256 * kLutCopies];
  __shared__ uint4 rk[11];
  __shared__ uint64_t cuts[kMaxCutsLds];
  __shared__ uint64_t pay[kMaxPayloadLds];
  const uint8_t* k = a.keys;
  fill_ttable<kLutCopies>(tab, kTDev.v);
  const uint32_t* rkg = reinterpret_cast<const uint32_t*>(k + 40);
  for (int i = threadIdx.x; i < 11; i += blockDim.x)
    rk[i] = make_uint4(rkg[4 * i], rkg[4 * i + 1], rkg[4 * i + 2], rkg[4 * i + 3]);
  const int nint = a.intervals, ow = a.out_words;
  const uint64_t* cg = reinterpret_cast<const uint64_t*>(k + kLutHdr);
  const uint64_t* pg = cg + (nint + 1);
  for (int i = threadIdx.x; i < nint; i += blockDim.x) cuts[i] = cg[i];
  for (int i = threadIdx.x; i < nint * ow; i += blockDim.x) pay[i] = pg[i];
  __syncthreads();
  const AesLds<kLutCopies> aes{tab, threadIdx.x % kLutCopies};
  const uint64_t m = mask_bits(*reinterpret_cast<const uint16_t*>(k));
  const int party = k[8];
  const uint64_t nonce = ld64(k + 16);
  for (size_t e = size_t(blockIdx.x) * kLutBlock + threadIdx.x; e < a.n;
       e += size_t(gridDim.x) * kLutBlock) {
    const uint64_t x = a.xs[e] & m;
    const int iv = interval_of(x, nint, m, [&](int i) { return cuts[i]; });
    write_masked_row(aes, rk, nonce, e, iv, ow, party, pay + size_t(iv) * ow,
                     a.out + e * size_t(ow));
  }
}

// Per-element keys read from HBM (also used for broadcast keys too large for LDS).
__global__ void __launch_bounds__(kLutBlock) lut_keyed_kernel(LutArgs a, int broadcast) {
  __shared__ __align__(16) uint32_t tab[256 * kLutCopies];
  fill_ttable<kLutCopies>(tab, kTDev.v);
  __syncthreads();
  const AesLds<kLutCopies> aes{tab, threadIdx.x % kLutCopies};
  const int nint = a.intervals, ow = a.out_words;
  for (size_t e = size_t(blockIdx.x) * kLutBlock + threadIdx.x; e < a.n;
       e += size_t(gridDim.x) * kLutBlock) {
    const uint8_t* k = broadcast ? a.keys : a.keys + e * a.key_bytes;
    const uint64_t m = mask_bits(*reinterpret_cast<const uint16_t*>(k));
    const int party = k[8];
    const uint64_t nonce = ld64(k + 16);
    const RegKeys rk = load_round_keys(k + 40);
    const uint64_t* cg = reinterpret_cast<const uint64_t*>(k + kLutHdr);
    const uint64_t x = a.xs[e] & m;
    const int iv = interval_of(x, nint, m, [&](int i) { return cg[i]; });
    write_masked_row(aes, rk, nonce, e, iv, ow, party, cg + (nint + 1) + size_t(iv) * ow,
                     a.out + e * size_t(ow));
  }
}

struct PackedArgs {
  const uint8_t* keys;
  const uint64_t* xs;
  uint64_t* out;
  size_t key_bytes;
  size_t n;
  int num_thr;
  int out_words;
};

// Word w of the compare mask for x (pfss_kernels.cu:255-314): the sorted form
// uses pos = first threshold above x; both forms give bit j = 1[x < thr_j].
template <typename ThrAt>
__device__ __forceinline__ uint64_t cmp_word(uint64_t x, uint64_t m, int num_thr, bool sorted,
                                             int pos, int w, const ThrAt& thr) {
  const int base = 64 * w;
  const int limit = base + 64 < num_thr ? base + 64 : num_thr;
  const int len = limit - base;
  if (len <= 0) return 0;
  if (sorted) {
    const uint64_t bits = len >= 64 ? ~uint64_t(0) : (uint64_t(1) << len) - 1;
    if (pos <= base) return bits;
    if (pos >= limit) return 0;
    return bits ^ ((uint64_t(1) << (pos - base)) - 1);
  }
  uint64_t word = 0;
  for (int b = base; b < limit; ++b)
    if (x < (thr(b) & m)) word |= uint64_t(1) << (b - base);
  return word;
}

template <typename RK, typename ThrAt>
__device__ __forceinline__ void packed_one(const AesLds<kLutCopies>& aes, const RK& rk,
                                           uint64_t nonce, int party, uint64_t x, uint64_t m,
                                           int num_thr, int ow, bool sorted, size_t idx,
                                           const ThrAt& thr, uint64_t* out) {
  int pos = 0;
  if (sorted) {
    int lo = 0, hi = num_thr;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (x < (thr(mid) & m))
        hi = mid;
      else
        lo = mid + 1;
    }
    pos = lo;
  }
  for (int w = 0; w < ow; w += 2) {
    const uint64_t w0 = cmp_word(x, m, num_thr, sorted, pos, w, thr);
    const uint64_t w1 = w + 1 < ow ? cmp_word(x, m, num_thr, sorted, pos, w + 1, thr) : 0;
    uint64_t k0, k1;
    keystream(aes, rk, nonce ^ (uint64_t(idx) << 32) ^ uint64_t(w / 2), k0, k1);
    out[w] = party == 0 ? k0 : (w0 ^ k0);
    if (w + 1 < ow) out[w + 1] = party == 0 ? k1 : (w1 ^ k1);
  }
}

__global__ void __launch_bounds__(kLutBlock) packed_bcast_kernel(PackedArgs a) {
  __shared__ __align__(16) uint32_t tab[256 * kLutCopies];
  __shared__ uint4 rk[11];
  __shared__ uint64_t thr[kMaxCutsLds];
  const uint8_t* k = a.keys;
  fill_ttable<kLutCopies>(tab, kTDev.v);
  const uint32_t* rkg = reinterpret_cast<const uint32_t*>(k + 32);
  for (int i = threadIdx.x; i < 11; i += blockDim.x)
    rk[i] = make_uint4(rkg[4 * i], rkg[4 * i + 1], rkg[4 * i + 2], rkg[4 * i + 3]);
  const uint64_t* tg = reinterpret_cast<const uint64_t*>(k + kPackedHdr);
  for (int i = threadIdx.x; i < a.num_thr; i += blockDim.x) thr[i] = tg[i];
  __syncthreads();
  const AesLds<kLutCopies> aes{tab, threadIdx.x % kLutCopies};
  const uint64_t m = mask_bits(*reinterpret_cast<const uint16_t*>(k));
  const int party = k[4];
  const bool sorted = (k[5] & 1u) != 0;
  const uint64_t nonce = ld64(k + 8);
  for (size_t e = size_t(blockIdx.x) * kLutBlock + threadIdx.x; e < a.n;
       e += size_t(gridDim.x) * kLutBlock) {
    packed_one(aes, rk, nonce, party, a.xs[e] & m, m, a.num_thr, a.out_words, sorted, e,
               [&](int i) { return thr[i]; }, a.out + e * size_t(a.out_words));
  }
}

__global__ void __launch_bounds__(kLutBlock) packed_keyed_kernel(PackedArgs a, int broadcast) {
  __shared__ __align__(16) uint32_t tab[256 * kLutCopies];
  fill_ttable<kLutCopies>(tab, kTDev.v);
  __syncthreads();
  const AesLds<kLutCopies> aes{tab, threadIdx.x % kLutCopies};
  for (size_t e = size_t(blockIdx.x) * kLutBlock + threadIdx.x; e < a.n;
       e += size_t(gridDim.x) * kLutBlock) {
    const uint8_t* k = broadcast ? a.keys : a.keys + e * a.key_bytes;
    const uint64_t m = mask_bits(*reinterpret_cast<const uint16_t*>(k));
    const uint64_t* tg = reinterpret_cast<const uint64_t*>(k + kPackedHdr);
    const RegKeys rk = load_round_keys(k + 32);
    packed_one(aes, rk, ld64(k + 8), k[4], a.xs[e] & m, m,
               a.num_thr, a.out_words, (k[5] & 1u) != 0, e, [&](int i) { return tg[i]; },
               a.out + e * size_t(a.out_words));
  }
}

// One pairwise-max round of RowMaxDiffTask for both parties: each party's
// broadcast LUT (ReLU coefficients at the public xhat, 2 words) staged in LDS.
constexpr int kReluMaxIntervals = 64;

struct ReluRoundArgs {
  const uint64_t* cur[2];
  const int32_t* src_a;
  const int32_t* src_b;
  const uint8_t* lut[2];
  uint64_t* next[2];
  size_t n_in;
  size_t n_out;
  uint64_t mask;
  int intervals;
};

__global__ void __launch_bounds__(kLutBlock) relu_max_round2_kernel(ReluRoundArgs a) {
  __shared__ __align__(16) uint32_t tab[256 * kLutCopies];
  __shared__ uint4 rk[2][11];
  __shared__ uint64_t cuts[2][kReluMaxIntervals];
  __shared__ uint64_t pay[2][2 * kReluMaxIntervals];
  fill_ttable<kLutCopies>(tab, kTDev.v);
  const int nint = a.intervals;
  for (int p = 0; p < 2; ++p) {
    const uint8_t* k = a.lut[p];
    const uint32_t* rkg = reinterpret_cast<const uint32_t*>(k + 40);
    for (int i = threadIdx.x; i < 11; i += blockDim.x)
      rk[p][i] = make_uint4(rkg[4 * i], rkg[4 * i + 1], rkg[4 * i + 2], rkg[4 * i + 3]);
    const uint64_t* cg = reinterpret_cast<const uint64_t*>(k + kLutHdr);
    const uint64_t* pg = cg + (nint + 1);
    for (int i = threadIdx.x; i < nint; i += blockDim.x) cuts[p][i] = cg[i];
    for (int i = threadIdx.x; i < 2 * nint; i += blockDim.x) pay[p][i] = pg[i];
  }
  __syncthreads();
  const AesLds<kLutCopies> aes{tab, threadIdx.x % kLutCopies};
  uint64_t m[2], nonce[2];
  int party[2];
  for (int p = 0; p < 2; ++p) {
    m[p] = mask_bits(*reinterpret_cast<const uint16_t*>(a.lut[p]));
    party[p] = a.lut[p][8];
    nonce[p] = ld64(a.lut[p] + 16);
  }
  for (size_t j = size_t(blockIdx.x) * kLutBlock + threadIdx.x; j < a.n_out;
       j += size_t(gridDim.x) * kLutBlock) {
    const int32_t ia = a.src_a[j], ib = a.src_b[j];
    const bool va = ia >= 0 && size_t(ia) < a.n_in;
    if (ib < 0) {
      a.next[0][j] = va ? a.cur[0][ia] : 0;
      a.next[1][j] = va ? a.cur[1][ia] : 0;
      continue;
    }
    const bool vb = size_t(ib) < a.n_in;
    const uint64_t xa0 = va ? a.cur[0][ia] : 0, xa1 = va ? a.cur[1][ia] : 0;
    const uint64_t xb0 = vb ? a.cur[0][ib] : 0, xb1 = vb ? a.cur[1][ib] : 0;
    const uint64_t xhat = (xa0 - xb0) + (xa1 - xb1) + a.mask;
    uint64_t q[2][2];
    for (int p = 0; p < 2; ++p) {
      const uint64_t x = xhat & m[p];
      const int iv = interval_of(x, nint, m[p], [&](int i) { return cuts[p][i]; });
      write_masked_row(aes, rk[p], nonce[p], j, iv, 2, party[p], pay[p] + 2 * iv, q[p]);
    }
    a.next[0][j] = xb0 + q[0][0] + q[0][1] * xhat;
    a.next[1][j] = xb1 + q[1][0] + q[1][1] * xhat;
  }
}

// Both parties' broadcast keys of one small gate in one launch, each staged
// in LDS, at the masked open of an operand (or a given open).
constexpr int kLut2Intervals = 64;
constexpr int kLut2Payload = 512;

struct Lut2Args {
  const uint8_t* key[2];
  sufhip_operand2 x;
  const uint64_t* xhat;  // used when x has no terms
  uint64_t mask;
  uint64_t* out[2];
  size_t n;
  int intervals;
  int out_words;
  int has_x;
};

__global__ void __launch_bounds__(kLutBlock) lut_bcast2_kernel(Lut2Args a) {
  __shared__ __align__(16) uint32_t tab[256 * kLutCopies];
  __shared__ uint4 rk[2][11];
  __shared__ uint64_t cuts[2][kLut2Intervals];
  __shared__ uint64_t pay[2][kLut2Payload];
  fill_ttable<kLutCopies>(tab, kTDev.v);
  const int nint = a.intervals, ow = a.out_words;
  for (int p = 0; p < 2; ++p) {
    const uint8_t* k = a.key[p];
    const uint32_t* rkg = reinterpret_cast<const uint32_t*>(k + 40);
    for (int i = threadIdx.x; i < 11; i += blockDim.x)
      rk[p][i] = make_uint4(rkg[4 * i], rkg[4 * i + 1], rkg[4 * i + 2], rkg[4 * i + 3]);
    const uint64_t* cg = reinterpret_cast<const uint64_t*>(k + kLutHdr);
    const uint64_t* pg = cg + (nint + 1);
    for (int i = threadIdx.x; i < nint; i += blockDim.x) cuts[p][i] = cg[i];
    for (int i = threadIdx.x; i < nint * ow; i += blockDim.x) pay[p][i] = pg[i];
  }
  __syncthreads();
  const AesLds<kLutCopies> aes{tab, threadIdx.x % kLutCopies};
  uint64_t m[2], nonce[2];
  int party[2];
  for (int p = 0; p < 2; ++p) {
    m[p] = mask_bits(*reinterpret_cast<const uint16_t*>(a.key[p]));
    party[p] = a.key[p][8];
    nonce[p] = ld64(a.key[p] + 16);
  }
  for (size_t e = size_t(blockIdx.x) * kLutBlock + threadIdx.x; e < a.n;
       e += size_t(gridDim.x) * kLutBlock) {
    const uint64_t xh = a.has_x ? operand_at(a.x, 0, e) + operand_at(a.x, 1, e) + a.mask
                                : a.xhat[e];
    for (int p = 0; p < 2; ++p) {
      const uint64_t x = xh & m[p];
      const int iv = interval_of(x, nint, m[p], [&](int i) { return cuts[p][i]; });
      write_masked_row(aes, rk[p], nonce[p], e, iv, ow, party[p], pay[p] + size_t(iv) * ow,
                       a.out[p] + e * size_t(ow));
    }
  }
}

// The whole pairwise-max tree of RowMaxDiffTask in one launch: each
// wavefront of a workgroup owns one row (groups of `waves` rows, grid-
// stride), runs every round (relu_tree_device.hpp) and writes
// delta = max - x.
constexpr int kTreeRounds = 16;
constexpr int kTreeMaxRow = 512;
constexpr int kTreeCopies = kLutCopies;
constexpr int kTreeWaves = 4;
constexpr size_t kTreeLdsCap = 65536;

struct ReluTreeArgs {
  const uint64_t* x[2];
  uint64_t* delta[2];
  const int32_t* offs;       // [rows + 1]
  const int32_t* round_off;  // [rounds][rows]: the row's first output slot per round
  TreeKeys<kTreeRounds> keys;
  int rows;
  int max_row;
  int waves;  // rows per workgroup (1, 2 or 4); blockDim.x == 64 * waves
};

struct ReluTreeStatic {
  uint32_t tab[256 * kTreeCopies];
  TreeLds<kTreeRounds> t;
  uint32_t j0[kTreeWaves][kTreeRounds];
};

__global__ void __launch_bounds__(64 * kTreeWaves) relu_max_tree2_kernel(ReluTreeArgs a) {
  __shared__ __align__(16) ReluTreeStatic st;
  extern __shared__ uint64_t rowbuf[];
  const int mr = a.max_row;
  fill_ttable<kTreeCopies>(st.tab, kTDev.v);
  tree_stage(kernarg_tree_keys<kTreeRounds>(offsetof(ReluTreeArgs, keys)), st.t);
  __syncthreads();
  tree_compare(a.keys, st.t);
  __syncthreads();
  const AesLds<kTreeCopies> aes{st.tab, threadIdx.x % kTreeCopies};
  const uint32_t shared = ~st.t.diff;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  uint64_t* even = rowbuf + size_t(wave) * tree_row_words(mr);
  uint64_t* odd = even + 2 * size_t(mr);
  for (int g = blockIdx.x; g * a.waves < a.rows; g += gridDim.x) {
    const int r = g * a.waves + wave;
    int b = 0, full = 0;
    if (r < a.rows) {
      b = a.offs[r];
      full = a.offs[r + 1] - b;
      if (full < 1 || full > mr) full = 0;  // refused on the host
    }
    tree_row_offsets(a.keys, a.round_off, a.rows, r, full, st.j0[wave]);
    for (int i = lane; i < full; i += 64) {
      even[i] = a.x[0][b + i];
      even[mr + i] = a.x[1][b + i];
    }
    __syncthreads();
    const int level =
        tree_row<kTreeRounds, AesLds<kTreeCopies>>(a.keys, st.t, aes, even, odd, mr, full, st.j0[wave],
                                           shared);
    if (full > 0) {
      const uint64_t* fin = (level & 1) ? odd : even;
      const int fw = (level & 1) ? (mr + 1) / 2 : mr;
      const uint64_t m0 = fin[0], m1 = fin[fw];
      for (int i = lane; i < full; i += 64) {
        a.delta[0][b + i] = m0 - a.x[0][b + i];
        a.delta[1][b + i] = m1 - a.x[1][b + i];
      }
    }
    __syncthreads();
  }
}

unsigned int lut_grid(size_t n) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const size_t need = (n + kLutBlock - 1) / kLutBlock;
  const size_t cap = size_t(cus) * 4;  // LDS allows several workgroups per CU
  return static_cast<unsigned int>(need < cap ? need : cap);
}

}  // namespace
}  // namespace sufhip

using namespace sufhip;

extern "C" {

void sufhip_seed_from_id(uint64_t id, uint64_t tweak, uint8_t* seed16) {
  std::mt19937_64 g(id ^ (tweak * 0x9e3779b97f4a7c15ull));
  for (int i = 0; i < 16; ++i) seed16[i] = static_cast<uint8_t>(g() & 0xFFu);
}

size_t sufhip_interval_lut_key_bytes(int intervals, int out_words) {
  if (intervals <= 0 || out_words <= 0 || out_words > 65535) return 0;
  return kLutHdr + 8 * size_t(intervals + 1) + 8 * size_t(intervals) * size_t(out_words);
}

int sufhip_interval_lut_build_key(int party, uint64_t nonce, int in_bits, int out_words,
                                  const uint64_t* cuts, int intervals, const uint64_t* payload,
                                  const uint8_t* seed16, uint8_t* blob) {
  SUFHIP_REQUIRE(out_words > 0 && out_words <= 65535, "interval_lut_build_key: out_words");
  SUFHIP_REQUIRE(intervals >= 1, "interval_lut_build_key: need >= 2 cutpoints");
  SUFHIP_REQUIRE(cuts && payload && seed16 && blob, "interval_lut_build_key: null pointer");
  std::memset(blob, 0, kLutHdr);
  const uint16_t ib = uint16_t(in_bits), ow = uint16_t(out_words);
  const uint32_t iv = uint32_t(intervals);
  std::memcpy(blob + 0, &ib, 2);
  std::memcpy(blob + 2, &ow, 2);
  std::memcpy(blob + 4, &iv, 4);
  blob[8] = uint8_t(party);
  std::memcpy(blob + 16, &nonce, 8);
  std::memcpy(blob + 24, seed16, 16);
  uint32_t rk[44];
  aes128_expand_words(seed16, rk);
  std::memcpy(blob + 40, rk, 176);
  std::memcpy(blob + kLutHdr, cuts, 8 * size_t(intervals + 1));
  std::memcpy(blob + kLutHdr + 8 * size_t(intervals + 1), payload,
              8 * size_t(intervals) * size_t(out_words));
  return SUFHIP_OK;
}

int sufhip_interval_lut_eval(const uint8_t* d_keys, size_t key_bytes, int key_broadcast,
                             int intervals, int out_words, const uint64_t* d_xs, size_t n,
                             uint64_t* d_out, void* stream) {
  SUFHIP_REQUIRE(intervals >= 1 && out_words >= 1, "sufhip_interval_lut_eval: bad geometry");
  SUFHIP_REQUIRE(key_bytes == sufhip_interval_lut_key_bytes(intervals, out_words),
                 "sufhip_interval_lut_eval: key_bytes does not match (intervals, out_words)");
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_keys && d_xs && d_out, "sufhip_interval_lut_eval: null pointer");
  SUFHIP_REQUIRE((reinterpret_cast<uintptr_t>(d_keys) & 7) == 0 && (key_bytes & 7) == 0,
                 "sufhip_interval_lut_eval: keys must be 8-byte aligned");
  LutArgs a{d_keys, d_xs, d_out, key_bytes, n, intervals, out_words};
  const dim3 grid(lut_grid(n)), block(kLutBlock);
  if (key_broadcast && intervals <= kMaxCutsLds && size_t(intervals) * out_words <= kMaxPayloadLds) {
    hipLaunchKernelGGL(lut_bcast_kernel, grid, block, 0, as_stream(stream), a);
  } else {
    hipLaunchKernelGGL(lut_keyed_kernel, grid, block, 0, as_stream(stream), a,
                       key_broadcast ? 1 : 0);
  }
  return check_launch("interval_lut kernel");
}

size_t sufhip_packed_lt_key_bytes(int num_thr) {
  if (num_thr <= 0 || num_thr > 65535) return 0;
  return kPackedHdr + 8 * size_t(num_thr);
}

int sufhip_packed_lt_build_key(int party, uint64_t nonce, int in_bits, const uint64_t* thresholds,
                               int num_thr, const uint8_t* seed16, uint8_t* blob) {
  SUFHIP_REQUIRE(in_bits >= 1 && in_bits <= 64, "packed_lt_build_key: in_bits out of range");
  SUFHIP_REQUIRE(num_thr >= 1 && num_thr <= 65535, "packed_lt_build_key: thresholds empty");
  SUFHIP_REQUIRE(thresholds && seed16 && blob, "packed_lt_build_key: null pointer");
  std::memset(blob, 0, kPackedHdr);
  const uint16_t ib = uint16_t(in_bits), nt = uint16_t(num_thr);
  std::memcpy(blob + 0, &ib, 2);
  std::memcpy(blob + 2, &nt, 2);
  blob[4] = uint8_t(party);
  std::memcpy(blob + 8, &nonce, 8);
  std::memcpy(blob + 16, seed16, 16);
  uint32_t rk[44];
  aes128_expand_words(seed16, rk);
  std::memcpy(blob + 32, rk, 176);
  const uint64_t m = in_bits >= 64 ? ~uint64_t(0) : (uint64_t(1) << in_bits) - 1;
  bool sorted = true;
  for (int i = 0; i < num_thr; ++i) {
    const uint64_t v = thresholds[i] & m;
    std::memcpy(blob + kPackedHdr + 8 * size_t(i), &v, 8);
    if (i > 0 && v < (thresholds[i - 1] & m)) sorted = false;
  }
  blob[5] = sorted ? 1u : 0u;
  return SUFHIP_OK;
}

int sufhip_packed_lt_eval(const uint8_t* d_keys, size_t key_bytes, int key_broadcast, int num_thr,
                          int out_words, const uint64_t* d_xs, size_t n, uint64_t* d_out,
                          void* stream) {
  SUFHIP_REQUIRE(num_thr >= 1 && out_words == (num_thr + 63) / 64,
                 "sufhip_packed_lt_eval: out_words must be ceil(num_thr / 64)");
  SUFHIP_REQUIRE(key_bytes == sufhip_packed_lt_key_bytes(num_thr),
                 "sufhip_packed_lt_eval: key_bytes does not match num_thr");
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_keys && d_xs && d_out, "sufhip_packed_lt_eval: null pointer");
  SUFHIP_REQUIRE((reinterpret_cast<uintptr_t>(d_keys) & 7) == 0,
                 "sufhip_packed_lt_eval: keys must be 8-byte aligned");
  PackedArgs a{d_keys, d_xs, d_out, key_bytes, n, num_thr, out_words};
  const dim3 grid(lut_grid(n)), block(kLutBlock);
  if (key_broadcast && num_thr <= kMaxCutsLds) {
    hipLaunchKernelGGL(packed_bcast_kernel, grid, block, 0, as_stream(stream), a);
  } else {
    hipLaunchKernelGGL(packed_keyed_kernel, grid, block, 0, as_stream(stream), a,
                       key_broadcast ? 1 : 0);
  }
  return check_launch("packed_lt kernel");
}

int sufhip_interval_lut_eval2(const uint8_t* d_key0, const uint8_t* d_key1, size_t key_bytes,
                              int intervals, int out_words, const sufhip_operand2* x,
                              const uint64_t* d_xhat, uint64_t mask, size_t n, uint64_t* d_out0,
                              uint64_t* d_out1, void* stream) {
  SUFHIP_REQUIRE(intervals >= 1 && intervals <= kLut2Intervals && out_words >= 1 &&
                     intervals * out_words <= kLut2Payload,
                 "sufhip_interval_lut_eval2: needs intervals <= 64 and intervals * out_words "
                 "<= 512");
  SUFHIP_REQUIRE(key_bytes == sufhip_interval_lut_key_bytes(intervals, out_words),
                 "sufhip_interval_lut_eval2: key_bytes does not match (intervals, out_words)");
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_key0 && d_key1 && d_out0 && d_out1 && (x || d_xhat),
                 "sufhip_interval_lut_eval2: null pointer");
  SUFHIP_REQUIRE((reinterpret_cast<uintptr_t>(d_key0) & 7) == 0 &&
                     (reinterpret_cast<uintptr_t>(d_key1) & 7) == 0,
                 "sufhip_interval_lut_eval2: keys must be 8-byte aligned");
  Lut2Args a{};
  a.key[0] = d_key0;
  a.key[1] = d_key1;
  if (x) {
    if (int rc = check_operand(*x, n, "sufhip_interval_lut_eval2")) return rc;
    a.x = *x;
    a.has_x = 1;
  }
  a.xhat = d_xhat;
  a.mask = mask;
  a.out[0] = d_out0;
  a.out[1] = d_out1;
  a.n = n;
  a.intervals = intervals;
  a.out_words = out_words;
  hipLaunchKernelGGL(lut_bcast2_kernel, dim3(lut_grid(n)), dim3(kLutBlock), 0, as_stream(stream),
                     a);
  return check_launch("lut_bcast2_kernel");
}

int sufhip_relu_max_tree2(const uint64_t* d_x0, const uint64_t* d_x1, int rows,
                          const int32_t* d_row_offsets, int max_row, int rounds,
                          const int32_t* d_round_offsets, const sufhip_relu_round_key* keys,
                          uint64_t* d_delta0, uint64_t* d_delta1, void* stream) {
  SUFHIP_REQUIRE(rows >= 0, "sufhip_relu_max_tree2: rows < 0");
  SUFHIP_REQUIRE(max_row >= 1 && max_row <= kTreeMaxRow,
                 "sufhip_relu_max_tree2: rows of 1..512 elements");
  ReluTreeArgs a{};
  if (int rc = make_tree_keys<kTreeRounds>(keys, rounds, max_row, "sufhip_relu_max_tree2",
                                           &a.keys))
    return rc;
  if (rows == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_x0 && d_x1 && d_row_offsets && d_delta0 && d_delta1 &&
                     (rounds == 0 || d_round_offsets),
                 "sufhip_relu_max_tree2: null pointer");
  a.x[0] = d_x0;
  a.x[1] = d_x1;
  a.delta[0] = d_delta0;
  a.delta[1] = d_delta1;
  a.offs = d_row_offsets;
  a.round_off = d_round_offsets;
  a.rows = rows;
  a.max_row = max_row;
  // Rows per workgroup: as many (4, 2, 1) as fit the LDS cap beside the
  // staged table and keys.
  const size_t row_bytes = tree_row_words(max_row) * sizeof(uint64_t);
  int waves = kTreeWaves;
  while (waves > 1 && sizeof(ReluTreeStatic) + size_t(waves) * row_bytes > kTreeLdsCap) waves /= 2;
  SUFHIP_REQUIRE(sizeof(ReluTreeStatic) + size_t(waves) * row_bytes <= kTreeLdsCap,
                 "sufhip_relu_max_tree2: rows too long for the workgroup's LDS");
  a.waves = waves;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const int groups = (rows + waves - 1) / waves;
  const int g = groups < cus * 2 ? groups : cus * 2;
  hipLaunchKernelGGL(relu_max_tree2_kernel, dim3(g), dim3(64 * waves), size_t(waves) * row_bytes,
                     as_stream(stream), a);
  return check_launch("relu_max_tree2_kernel");
}

int sufhip_relu_max_round2(const uint64_t* d_cur0, const uint64_t* d_cur1, size_t n_in,
                           const int32_t* d_src_a, const int32_t* d_src_b, size_t n_out,
                           const uint8_t* d_lut0, const uint8_t* d_lut1, size_t key_bytes,
                           int intervals, uint64_t mask, uint64_t* d_next0, uint64_t* d_next1,
                           void* stream) {
  SUFHIP_REQUIRE(intervals >= 1 && intervals <= kReluMaxIntervals,
                 "sufhip_relu_max_round2: intervals must be in [1, 64]");
  SUFHIP_REQUIRE(key_bytes == sufhip_interval_lut_key_bytes(intervals, 2),
                 "sufhip_relu_max_round2: key_bytes does not match (intervals, 2)");
  if (n_out == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(n_in > 0 && n_in < (size_t(1) << 31), "sufhip_relu_max_round2: bad n_in");
  SUFHIP_REQUIRE(d_cur0 && d_cur1 && d_src_a && d_src_b && d_lut0 && d_lut1 && d_next0 && d_next1,
                 "sufhip_relu_max_round2: null pointer");
  SUFHIP_REQUIRE((reinterpret_cast<uintptr_t>(d_lut0) & 7) == 0 &&
                     (reinterpret_cast<uintptr_t>(d_lut1) & 7) == 0,
                 "sufhip_relu_max_round2: keys must be 8-byte aligned");
  ReluRoundArgs a{{d_cur0, d_cur1}, d_src_a, d_src_b, {d_lut0, d_lut1}, {d_next0, d_next1},
                  n_in, n_out, mask, intervals};
  hipLaunchKernelGGL(relu_max_round2_kernel, dim3(lut_grid(n_out)), dim3(kLutBlock), 0,
                     as_stream(stream), a);
  return check_launch("relu_max_round2_kernel");
}

}  // extern "C"
