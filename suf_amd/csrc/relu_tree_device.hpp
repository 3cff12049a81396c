// The pairwise-max tree of RowMaxDiffTask (include/nn/row_maxdiff_task.hpp:
// 49-165) over one row per wavefront, both parties: max(a, b) = b + ReLU(a -
// b), the ReLU as an interval LUT of its public-x^ coefficients (2 words,
// AES-CTR keystream, pfss_kernels.cu:545-719).  Shared by the tree kernel
// (lut.hip) and the softmax row block (blocks.hip).
//
// A slot's AES block is spread over a lane quad, one state column per lane
// (AesLds::encrypt_quad_n), one block for both parties when their blobs
// share the keystream; the keystream counters are those of the per-round
// evaluation (slot j = the row's offset in that round's output + pair
// index).  Level 0 of a row (its
// inputs) and the odd levels live in two LDS buffers per wave, [party]
// [max_row] and [party][ceil(max_row / 2)]; a level never outgrows the buffer
// it is written to.  Every wave of a workgroup runs the same number of
// rounds, so the workgroup barriers inside are uniform.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "aes_lds.hpp"
#include "suf_hip.h"
#include "sufhip_internal.hpp"

namespace sufhip {

constexpr int kTreeIntervals = 8;
constexpr size_t kTreeLutHdr = 216;

template <int kRounds>
struct TreeKeys {
  const uint8_t* key[kRounds][2];
  uint64_t mask[kRounds];
  int intervals[kRounds];
  int rounds;
  // All ones: every round's keystreams and interval searches per party,
  // even where the blobs compare equal (sufhip_set_keystream_per_party).
  uint32_t own_ks;
};

template <int kRounds>
struct TreeLds {
  uint4 rk[kRounds][2][11];
  uint64_t cuts[kRounds][2][kTreeIntervals];
  uint64_t pay[kRounds][2][2 * kTreeIntervals];
  uint64_t nonce[kRounds][2];
  uint64_t in_mask[kRounds][2];
  int party[kRounds][2];
  uint32_t diff;  // bit k: round k's two blobs differ (tree_compare)
};

// Dynamic LDS words (u64) per wave for rows of up to max_row elements.
__host__ __device__ inline size_t tree_row_words(int max_row) {
  return size_t(2) * (size_t(max_row) + size_t(max_row + 1) / 2);
}

// Staging items of one round's keys: per party the 11 round keys, 8 cut
// points, 16 payload words and the three header words (in_bits, party,
// nonce); cut and payload slots past the round's intervals stage zero.
constexpr int kTreeItemsPerParty = 11 + 3 * kTreeIntervals + 3;
constexpr int kTreeItems = 2 * kTreeItemsPerParty;  // per round

// Loads item `item` of round k: the item's offset in its blob is selected
// arithmetically and two 8-byte loads (the second at the first's address for
// 8-byte items) are always issued, so a thread's loads of several items stay
// in flight together; items past the round's intervals read the blob's
// first word and stage zero.  K may live in the kernarg segment (see
// kernarg_tree_keys), so k may be a runtime index.
template <int kRounds>
__device__ __forceinline__ uint4 tree_item_load(const TreeKeys<kRounds>& K, int k, int item) {
  const int p = item >= kTreeItemsPerParty ? 1 : 0;
  const int w = item - p * kTreeItemsPerParty;
  const uint8_t* blob = K.key[k][p];
  const int nint = K.intervals[k];
  const int c = w - 11, cp = w - 11 - kTreeIntervals, h = w - (11 + 3 * kTreeIntervals);
  const bool rk = w < 11, cut = !rk && c < kTreeIntervals;
  const bool pay = !rk && !cut && cp < 2 * kTreeIntervals;
  const bool zero = (cut && c >= nint) || (pay && cp >= 2 * nint);
  int off = rk ? 40 + 16 * w
               : (cut ? int(kTreeLutHdr) + 8 * c
                      : (pay ? int(kTreeLutHdr) + 8 * (nint + 1 + cp) : 8 * h));
  off = zero ? 0 : off;
  const uint64_t* a = reinterpret_cast<const uint64_t*>(blob + off);
  uint64_t lo = a[0], hi = a[rk ? 1 : 0];
  lo = zero ? 0 : lo;
  hi = rk ? hi : 0;
  return make_uint4(uint32_t(lo), uint32_t(lo >> 32), uint32_t(hi), uint32_t(hi >> 32));
}

template <int kRounds>
__device__ __forceinline__ void tree_item_store(TreeLds<kRounds>& L, int k, int item, uint4 v) {
  const int p = item >= kTreeItemsPerParty ? 1 : 0;
  const int w = item - p * kTreeItemsPerParty;
  const uint64_t x = uint64_t(v.x) | uint64_t(v.y) << 32;
  if (w < 11) {
    L.rk[k][p][w] = v;
  } else if (w < 11 + kTreeIntervals) {
    L.cuts[k][p][w - 11] = x;
  } else if (w < 11 + 3 * kTreeIntervals) {
    L.pay[k][p][w - 11 - kTreeIntervals] = x;
  } else {
    const int h = w - (11 + 3 * kTreeIntervals);
    if (h == 0) {
      const int bits = int(x & 0xffff);
      L.in_mask[k][p] = bits <= 0 ? 0 : (bits >= 64 ? ~uint64_t(0) : (uint64_t(1) << bits) - 1);
    } else if (h == 1) {
      L.party[k][p] = int(x & 0xff);
    } else {
      L.nonce[k][p] = x;
    }
  }
}

// A kernel's by-value TreeKeys read in place in the kernarg segment: a
// runtime index into the by-value copy would make the compiler copy the
// whole argument block to private scratch memory, while indexing the
// segment is a plain load.  `field` is the keys' byte offset in the
// kernel's (single, by-value) argument.
template <int kRounds>
__device__ __forceinline__ const TreeKeys<kRounds>* kernarg_tree_keys(size_t field) {
  const uint8_t* base = (const uint8_t*)__builtin_amdgcn_kernarg_segment_ptr();
  return reinterpret_cast<const TreeKeys<kRounds>*>(base + field);
}

// The staging items of every round as one flat list (round k's item j is
// k * kTreeItems + j) over the workgroup: thread t takes items t + m *
// blockDim in passes of kPer, each pass's loads issued before its stores.
// load/store split one pass so that a caller can put other loads in flight
// in between (one pass covers all items when rounds * kTreeItems <= kPer *
// blockDim).
template <int kRounds, int kPer>
struct TreeStager {
  uint4 v[kPer];
  int f[kPer];
  __device__ __forceinline__ void load(const TreeKeys<kRounds>* K, int f0) {
    const int n = K->rounds * kTreeItems;
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int g = f0 + u * int(blockDim.x);
      f[u] = g < n ? g : -1;
      const int gc = g < n ? g : 0;
      v[u] = n > 0 ? tree_item_load(*K, gc / kTreeItems, gc % kTreeItems) : make_uint4(0, 0, 0, 0);
    }
  }
  __device__ __forceinline__ void store(TreeLds<kRounds>& L) const {
#pragma unroll
    for (int u = 0; u < kPer; ++u)
      if (f[u] >= 0) tree_item_store(L, f[u] / kTreeItems, f[u] % kTreeItems, v[u]);
  }
};

// Cooperative staging of every round's keys (all threads); K in the kernarg
// segment (kernarg_tree_keys).  The caller syncs.
template <int kRounds>
__device__ __forceinline__ void tree_stage(const TreeKeys<kRounds>* K, TreeLds<kRounds>& L) {
  if (threadIdx.x == 0) L.diff = K->own_ks;
  const int n = K->rounds * kTreeItems;
  for (int f0 = threadIdx.x; f0 < n; f0 += 2 * blockDim.x) {
    TreeStager<kRounds, 2> s;
    s.load(K, f0);
    s.store(L);
  }
}

// Loads row r's slot offset of every round (round_off[k * rows + r]) into
// j0[k], one round per lane; call before the barrier that precedes tree_row.
template <int kRounds>
__device__ __forceinline__ void tree_row_offsets(const TreeKeys<kRounds>& K,
                                                 const int32_t* round_off, int rows, int r,
                                                 int len, uint32_t* j0) {
  const int lane = threadIdx.x & 63;
  if (len > 1 && lane < K.rounds) j0[lane] = uint32_t(round_off[size_t(lane) * rows + r]);
}

// Between the staging barrier and the next one (every thread): one staged
// word pair per lane, a difference sets round k's bit of L.diff.  After
// that barrier, bit k of ~L.diff says that round k's two blobs carry the
// same AES key, nonce, input mask and cut points (SUF's dealer derives one
// key per gate, cuda/pfss_backend_gpu.cu:508-515), so that one keystream
// block serves both parties of a slot.  tree_stage starts L.diff at
// TreeKeys::own_ks (zero unless every keystream is per party).
template <int kRounds>
__device__ __forceinline__ void tree_compare(const TreeKeys<kRounds>& K, TreeLds<kRounds>& L) {
  constexpr int kPer = 11 + kTreeIntervals + 1;  // round key words, cuts, header
  for (int t = threadIdx.x; t < K.rounds * kPer; t += blockDim.x) {
    const int k = t / kPer, w = t % kPer;
    bool differ;
    if (w < 11) {
      const uint4 a = L.rk[k][0][w], b = L.rk[k][1][w];
      differ = ((a.x ^ b.x) | (a.y ^ b.y) | (a.z ^ b.z) | (a.w ^ b.w)) != 0;
    } else if (w < 11 + kTreeIntervals) {
      const int c = w - 11;
      differ = c < K.intervals[k] && L.cuts[k][0][c] != L.cuts[k][1][c];
    } else {
      differ = L.nonce[k][0] != L.nonce[k][1] || L.in_mask[k][0] != L.in_mask[k][1];
    }
    if (differ) atomicOr(&L.diff, 1u << k);
  }
}

// Interval of xhat in round k's cut points of party p (upper bound minus one).
template <int kRounds>
__device__ __forceinline__ int tree_interval(const TreeKeys<kRounds>& K,
                                             const TreeLds<kRounds>& L, int k, int p,
                                             uint64_t xhat) {
  const uint64_t m = L.in_mask[k][p];
  const uint64_t xm = xhat & m;
  int lo = 0, hi = K.intervals[k];
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if ((L.cuts[k][p][mid] & m) <= xm)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo - 1 < 0 ? 0 : lo - 1;
}

// One chunk of a level: pair slots t0 .. t0 + nb - 1 (nb <= 64), each AES
// block spread over a lane quad (AesLds::encrypt_quad_n).  Quad m = lane / 4
// encrypts slots t0 + m + 16u for u < U (U = ceil(nb / 16)), so a level of
// at most 16 pairs costs one block's quad latency instead of a lane's whole
// block.  Every lane of the quad computes the slot's x^ and interval (the
// same LDS reads, broadcast); afterwards lane q of quad m gathers block q's
// four columns (DPP quad broadcasts) and writes slot t0 + m + 16q.  All 64
// lanes run it (the DPP reads need whole quads); slots past nb compute on a
// clamped slot and write nothing.
template <int U, int kRounds, class Aes>
__device__ __forceinline__ void tree_chunk(const TreeKeys<kRounds>& K, const TreeLds<kRounds>& L,
                                           const Aes& aes, int k, const uint64_t* src, int sw,
                                           uint64_t* dst, int dw, uint32_t j0, int t0, int nb,
                                           bool one_ks) {
  const int lane = threadIdx.x & 63, q = lane & 3, m = lane >> 2;
  uint64_t xh[U], xb[U][2];
  int iv[U][2];
  uint32_t blk[2][U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int t = t0 + (m + 16 * u < nb ? m + 16 * u : 0);
    const uint64_t xa0 = src[2 * t], xb0 = src[2 * t + 1];
    const uint64_t xa1 = src[sw + 2 * t], xb1 = src[sw + 2 * t + 1];
    xh[u] = (xa0 - xb0) + (xa1 - xb1) + K.mask[k];
    xb[u][0] = xb0;
    xb[u][1] = xb1;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      iv[u][p] = (p == 1 && one_ks) ? iv[u][0] : tree_interval(K, L, k, p, xh[u]);
      const uint64_t ctr =
          L.nonce[k][p] ^ (uint64_t(j0 + uint32_t(t)) << 32) ^ (uint64_t(iv[u][p]) * 2);
      blk[p][u] = q == 0 ? uint32_t(ctr) : (q == 1 ? uint32_t(ctr >> 32) : 0u);
    }
  }
  {
    const uint32_t* rk0 = reinterpret_cast<const uint32_t*>(L.rk[k][0]) + q;
    const uint32_t* rk1 = reinterpret_cast<const uint32_t*>(L.rk[k][1]) + q;
    const uint32_t* rks[U];
#pragma unroll
    for (int u = 0; u < U; ++u) rks[u] = rk0;
    if (one_ks) {
      aes.template encrypt_quad_n<U>(blk[0], rks);
#pragma unroll
      for (int u = 0; u < U; ++u) blk[1][u] = blk[0][u];
    } else if constexpr (U <= 2) {
      // Both parties' blocks in one lockstep group: one quad-AES latency.
      uint32_t b2[2 * U];
      const uint32_t* k2[2 * U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        b2[u] = blk[0][u];
        b2[U + u] = blk[1][u];
        k2[u] = rk0;
        k2[U + u] = rk1;
      }
      aes.template encrypt_quad_n<2 * U>(b2, k2);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        blk[0][u] = b2[u];
        blk[1][u] = b2[U + u];
      }
    } else {
      aes.template encrypt_quad_n<U>(blk[0], rks);
#pragma unroll
      for (int u = 0; u < U; ++u) rks[u] = rk1;
      aes.template encrypt_quad_n<U>(blk[1], rks);
    }
  }
  // Lane q takes block q: column c of it is lane c's word of blk[.][q].
  uint32_t w[2][4];
  uint64_t x = 0, b[2] = {0, 0};
  int ivq[2] = {0, 0};
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int c = 0; c < 4; ++c) w[p][c] = 0;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t c0 = quad_bcast<0>(blk[0][u]), c1 = quad_bcast<1>(blk[0][u]);
    const uint32_t c2 = quad_bcast<2>(blk[0][u]), c3 = quad_bcast<3>(blk[0][u]);
    uint32_t d0 = c0, d1 = c1, d2 = c2, d3 = c3;
    if (!one_ks) {
      d0 = quad_bcast<0>(blk[1][u]);
      d1 = quad_bcast<1>(blk[1][u]);
      d2 = quad_bcast<2>(blk[1][u]);
      d3 = quad_bcast<3>(blk[1][u]);
    }
    if (q == u) {
      w[0][0] = c0;
      w[0][1] = c1;
      w[0][2] = c2;
      w[0][3] = c3;
      w[1][0] = d0;
      w[1][1] = d1;
      w[1][2] = d2;
      w[1][3] = d3;
      x = xh[u];
      b[0] = xb[u][0];
      b[1] = xb[u][1];
      ivq[0] = iv[u][0];
      ivq[1] = iv[u][1];
    }
  }
  const int slot = m + 16 * q;
  if (q < U && slot < nb) {
    uint64_t o[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const uint64_t k0 = uint64_t(w[p][0]) | uint64_t(w[p][1]) << 32;
      const uint64_t k1 = uint64_t(w[p][2]) | uint64_t(w[p][3]) << 32;
      const bool p0 = L.party[k][p] == 0;
      const uint64_t q0 = p0 ? k0 : L.pay[k][p][2 * ivq[p]] - k0;
      const uint64_t q1 = p0 ? k1 : L.pay[k][p][2 * ivq[p] + 1] - k1;
      o[p] = b[p] + q0 + q1 * x;
    }
    dst[t0 + slot] = o[0];
    dst[dw + t0 + slot] = o[1];
  }
}

// Runs every round over this wave's row of `len` elements whose level 0 is
// in even[0..len) (party 0) and even[mr..mr+len) (party 1); j0[k] is the
// row's first slot in round k (tree_row_offsets, written before a barrier);
// bit k of `shared` is clear in L.diff (tree_compare).  Returns the level count; the row's max is
// at index 0 of the final level's buffer (even if the count is even, odd
// otherwise; party stride mr or ceil(mr / 2)).  Slot t of a level is pair
// (2t, 2t + 1) of the level below; an odd level's last element passes
// through as its last slot.  A wave touches only its own row buffers, so
// the levels synchronise the wave alone (LDS operations of one wave complete
// in order; the fence keeps the compiler from moving a level's reads above
// the previous level's writes) and a row stops when its length reaches one.
template <int kRounds, class Aes>
__device__ __forceinline__ int tree_row(const TreeKeys<kRounds>& K, const TreeLds<kRounds>& L,
                                        const Aes& aes, uint64_t* even,
                                        uint64_t* odd, int mr, int len, const uint32_t* j0s,
                                        uint32_t shared) {
  const int lane = threadIdx.x & 63, half = (mr + 1) / 2;
  int level = 0;
  for (int k = 0; k < K.rounds && len > 1; ++k) {
    {
      const uint64_t* src = (level & 1) ? odd : even;
      const int sw = (level & 1) ? half : mr;  // party stride of src
      uint64_t* dst = (level & 1) ? even : odd;
      const int dw = (level & 1) ? mr : half;
      const int pairs = len >> 1;
      const uint32_t j0 = j0s[k];
      const bool one_ks = (shared >> k) & 1u;
      for (int t0 = 0; t0 < pairs; t0 += 64) {
        const int nb = pairs - t0 < 64 ? pairs - t0 : 64;
        if (nb > 48)
          tree_chunk<4>(K, L, aes, k, src, sw, dst, dw, j0, t0, nb, one_ks);
        else if (nb > 32)
          tree_chunk<3>(K, L, aes, k, src, sw, dst, dw, j0, t0, nb, one_ks);
        else if (nb > 16)
          tree_chunk<2>(K, L, aes, k, src, sw, dst, dw, j0, t0, nb, one_ks);
        else
          tree_chunk<1>(K, L, aes, k, src, sw, dst, dw, j0, t0, nb, one_ks);
      }
      if ((len & 1) && lane == 0) {
        dst[pairs] = src[2 * pairs];
        dst[dw + pairs] = src[sw + 2 * pairs];
      }
      len = (len + 1) >> 1;
      ++level;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  return level;
}

// Host: validates the rounds' keys for rows of up to max_row elements.
template <int kRounds>
inline int make_tree_keys(const sufhip_relu_round_key* keys, int rounds, int max_row,
                          const char* what, TreeKeys<kRounds>* out) {
  auto fail = [&](const char* msg) {
    set_error(std::string(what) + ": " + msg);
    return SUFHIP_ERR_INVALID;
  };
  if (rounds < 0 || rounds > kRounds) return fail("too many rounds");
  if (max_row < 1 || (max_row > 1 && rounds < 1) || (1LL << rounds) < max_row)
    return fail("too few rounds for max_row");
  if (rounds > 0 && !keys) return fail("null round keys");
  TreeKeys<kRounds> K{};
  K.rounds = rounds;
  for (int k = 0; k < rounds; ++k) {
    const sufhip_relu_round_key& rk = keys[k];
    if (rk.intervals < 1 || rk.intervals > kTreeIntervals ||
        rk.key_bytes != sufhip_interval_lut_key_bytes(rk.intervals, 2))
      return fail("a round's LUT geometry is invalid");
    if (!rk.key[0] || !rk.key[1] || (reinterpret_cast<uintptr_t>(rk.key[0]) & 7) != 0 ||
        (reinterpret_cast<uintptr_t>(rk.key[1]) & 7) != 0)
      return fail("round keys must be non-null and 8-byte aligned");
    K.key[k][0] = rk.key[0];
    K.key[k][1] = rk.key[1];
    K.mask[k] = rk.mask;
    K.intervals[k] = rk.intervals;
  }
  K.own_ks = keystream_per_party() ? ~0u : 0u;
  *out = K;
  return SUFHIP_OK;
}

}  // namespace sufhip
