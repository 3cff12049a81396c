// Device side of the whole elementwise gate chains (CubicPolyTask, RecipTask,
// RsqrtTask for both parties), shared by the chain kernel (chains.hip) and
// the row-block kernels that run a chain inside a larger launch (blocks.hip).
//
// Per element i, for both parties: the coefficient LUT at the masked open of
// x (interval LUT, pfss_kernels.cu:545-719: binary search over the cut
// points, AES-CTR keystream at nonce ^ (i << 32) ^ (interval * W + w)), then
// every Beaver product (each d / e open summed in registers) and every
// truncation gate (table lookup at the product's masked open).
//
//   CUBIC  CubicPolyTask (include/runtime/phase_tasks.hpp:2718-3066):
//          m = c3 x + c2 << f; y = tr(m x); y2 = tr((y + c1 << f) x);
//          out = tr(y2 + c0 << f)                (trunc_2f + c0 as two tr_f)
//   RECIP  RecipTask, one NR step (phase_tasks.hpp:3140-3653):
//          y = tr(c1 x) + c0; xy = tr(y x); out = tr(y (2 << f - xy))
//   RSQRT  RsqrtTask, one NR step (phase_tasks.hpp:1383-1700):
//          y = tr(c1 x) + c0; y2 = tr(y y); h = tr'(x y2);
//          out = tr(y (3 << (f - 1) - h))        (tr' truncates by f + 1)
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "aes_lds.hpp"
#include "digit_planes.hpp"
#include "operand_device.hpp"
#include "suf_hip.h"
#include "sufhip_internal.hpp"
#include "trunc_device.hpp"

namespace sufhip {

constexpr size_t kChainLutHdr = 216;
constexpr int kChainMaxIntervals = 64;
constexpr int kChainMaxWords = 4;

struct ChainArgs {
  sufhip_operand2 x;
  const uint8_t* lut[2];
  uint64_t lut_mask;
  int intervals;
  int f;
  sufhip_term2 a[4], b[4], c[4];
  const uint8_t* tkey[4][2];
  const uint4* ttab[4][2];
  uint64_t tmask[4];
  int tf[4];
  uint64_t* out[2];
  sufhip_x_planes xp;
  size_t n;
  // plain: every product's a, b and c is an array of at least n rows with
  // no index, multiplier, shift or negation, all with one stride (1, or 3
  // for interleaved triples): pa/pb/pc point at their offsets and row i of
  // a term is p[i * pstride].  plain_x: x is one such term of stride 1.  The
  // kernels then read the triple shares (plain_loader) and x[p][i] straight
  // from these pointers, which keeps the general terms' fields out of the
  // scalar registers.
  bool plain, plain_x;
  int pstride;
  const uint64_t* px[2];
  const uint64_t* pa[4][2];
  const uint64_t* pb[4][2];
  const uint64_t* pc[4][2];
  // Nonzero: each party's keystream and interval search from its own blob,
  // even where the blobs compare equal (sufhip_set_keystream_per_party).
  uint32_t own_ks;
};

struct Two {
  uint64_t v[2];
};

// Both parties' LUT material staged in LDS.  (The truncation key headers
// are read with uniform loads, which land in scalar registers.)
struct ChainLds {
  uint4 rk[2][11];
  uint64_t cuts[2][kChainMaxIntervals];
  uint64_t pay[2][kChainMaxIntervals * kChainMaxWords];
  uint64_t hdr[2][3];  // header words 0-2: in_bits (low 16 bits), party (byte 8), nonce
  uint32_t diff;  // nonzero: the two blobs' keystreams differ (chain_compare)
};

// Sources of an element's triple shares for product k, both parties:
// ChainPre holds them all, loaded before the chain starts (in LDS, for a
// chain run by a lone lane, so that no product waits for its loads);
// chain_loader loads each product's shares when it is reached (for the
// element-parallel kernel, where other waves hide the latency and registers
// set the occupancy).
template <int kProds>
struct ChainPreN {
  uint64_t a[kProds][2], b[kProds][2], c[kProds][2];
  __device__ __forceinline__ void get(int k, uint64_t* a3, uint64_t* b3, uint64_t* c3) const {
    for (int p = 0; p < 2; ++p) {
      a3[p] = a[k][p];
      b3[p] = b[k][p];
      c3[p] = c[k][p];
    }
  }
  // Word w of 6 * kProds: (product, a | b | c, party).
  __device__ __forceinline__ uint64_t& word(int w) {
    const int k = w / 6, q = (w / 2) % 3, p = w & 1;
    return (q == 0 ? a : (q == 1 ? b : c))[k][p];
  }
};
using ChainPre = ChainPreN<4>;

// The triple word w (see ChainPreN::word) of element i.
__device__ __forceinline__ uint64_t chain_triple_word(const ChainArgs& A, int w, size_t i) {
  const int k = w / 6, q = (w / 2) % 3, p = w & 1;
  return term_at(q == 0 ? A.a[k] : (q == 1 ? A.b[k] : A.c[k]), p, i);
}

// All products' triple shares of element i in registers.
template <int kProds>
__device__ __forceinline__ ChainPreN<kProds> chain_prefetch(const ChainArgs& A, size_t i) {
  ChainPreN<kProds> P;
#pragma unroll
  for (int k = 0; k < kProds; ++k)
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      P.a[k][p] = term_at(A.a[k], p, i);
      P.b[k][p] = term_at(A.b[k], p, i);
      P.c[k][p] = term_at(A.c[k], p, i);
    }
  return P;
}

template <int kKind>
struct chain_loader {
  const ChainArgs* A;
  size_t i;
  __device__ __forceinline__ void get(int k, uint64_t* a3, uint64_t* b3, uint64_t* c3) const {
    for (int p = 0; p < 2; ++p) {
      a3[p] = term_at(A->a[k], p, i);
      b3[p] = term_at(A->b[k], p, i);
      c3[p] = term_at(A->c[k], p, i);
    }
  }
};

// Triple shares of product k from the plain pointers (ChainArgs::plain).
template <int kKind>
struct plain_loader {
  const ChainArgs* A;
  size_t i;
  __device__ __forceinline__ void get(int k, uint64_t* a3, uint64_t* b3, uint64_t* c3) const {
    const size_t j = i * size_t(A->pstride);
    for (int p = 0; p < 2; ++p) {
      a3[p] = A->pa[k][p][j];
      b3[p] = A->pb[k][p][j];
      c3[p] = A->pc[k][p][j];
    }
  }
};

// x's shares of element i for a plain chain.
__device__ __forceinline__ uint64_t plain_x(const ChainArgs& A, int p, size_t i) {
  return A.px[p][i] + (p == 0 ? A.x.party0_const : 0);
}

template <int kKind>
constexpr int chain_products() {
  return kKind == SUFHIP_CHAIN_RSQRT ? 4 : 3;
}

// Per-party LUT header fields: input mask, keystream nonce, party; and
// whether both parties' blobs carry the same AES key, nonce, input mask and
// cut points.  SUF's dealer derives one key per gate (seed_from_id,
// cuda/pfss_backend_gpu.cu:508-515): party 0's share is the keystream and
// party 1's the payload row minus it, so with both parties in one process
// one keystream block serves both.
struct ChainKeyInfo {
  uint64_t m[2], nonce[2];
  int party[2];
  bool same_ks;
};

__device__ __forceinline__ uint64_t chain_mask_bits(int bits) {
  return bits <= 0 ? 0 : (bits >= 64 ? ~uint64_t(0) : (uint64_t(1) << bits) - 1);
}

// Staging items of a chain's LUT material, both parties: per party the 11
// round keys, the cut points, the payload words and three header words.
// Item i is one 16-byte or 8-byte global load (chain_item_load) and one LDS
// store (chain_item_store), so a caller can issue the loads of several
// items, of several chains, before any store.
__device__ __forceinline__ int chain_items(const ChainArgs& A, int W) {
  return 2 * (11 + A.intervals + A.intervals * W + 3);
}

// Address of item i's first word and whether it is a 16-byte round key
// (branch-free, like tree_item_load: a caller issues the loads of several
// items, of several chains, before any is used).
__device__ __forceinline__ const uint64_t* chain_item_addr(const ChainArgs& A, int W, int i,
                                                          bool* rk16) {
  const int nint = A.intervals, per = 11 + nint + nint * W + 3;
  const int p = i >= per ? 1 : 0;
  const int w = i - p * per;
  const uint8_t* k = p ? A.lut[1] : A.lut[0];
  const bool rk = w < 11, cut = !rk && w < 11 + nint, pay = !rk && !cut && w < 11 + nint + nint * W;
  const int off = rk ? 40 + 16 * w
                     : (cut ? int(kChainLutHdr) + 8 * (w - 11)
                            : (pay ? int(kChainLutHdr) + 8 * (nint + 1 + (w - 11 - nint))
                                   : 8 * (w - (11 + nint + nint * W))));
  *rk16 = rk;
  return reinterpret_cast<const uint64_t*>(k + off);
}

// Two 8-byte loads, always issued (the second at the first's address for an
// 8-byte item).
__device__ __forceinline__ uint4 chain_item_fetch(const uint64_t* a, bool rk16) {
  const uint64_t lo = a[0];
  uint64_t hi = a[rk16 ? 1 : 0];
  hi = rk16 ? hi : 0;
  return make_uint4(uint32_t(lo), uint32_t(lo >> 32), uint32_t(hi), uint32_t(hi >> 32));
}

__device__ __forceinline__ uint4 chain_item_load(const ChainArgs& A, int W, int i) {
  bool rk16;
  const uint64_t* a = chain_item_addr(A, W, i, &rk16);
  return chain_item_fetch(a, rk16);
}

__device__ __forceinline__ void chain_item_store(const ChainArgs& A, int W, ChainLds& L, int i,
                                                 uint4 v) {
  const int nint = A.intervals, per = 11 + nint + nint * W + 3;
  const int p = i >= per ? 1 : 0;
  const int w = i - p * per;
  const uint64_t x = uint64_t(v.x) | uint64_t(v.y) << 32;
  if (w < 11)
    L.rk[p][w] = v;
  else if (w < 11 + nint)
    L.cuts[p][w - 11] = x;
  else if (w < 11 + nint + nint * W)
    L.pay[p][w - 11 - nint] = x;
  else
    L.hdr[p][w - (11 + nint + nint * W)] = x;
}

// A chain's items over a workgroup of kThreads threads in one pass of kPer
// items per thread (thread t takes items t + u * kThreads), loads issued
// before stores; items beyond kPer * kThreads go item by item in store().
template <int kThreads, int kPer>
struct ChainStager {
  uint4 v[kPer];
  int n;
  __device__ __forceinline__ void load(const ChainArgs& A, int W) {
    n = chain_items(A, W);
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int c = int(threadIdx.x) + u * kThreads;
      v[u] = chain_item_load(A, W, c < n ? c : 0);
    }
  }
  __device__ __forceinline__ void store(const ChainArgs& A, int W, ChainLds& L) const {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int c = int(threadIdx.x) + u * kThreads;
      if (c < n) chain_item_store(A, W, L, c, v[u]);
    }
    for (int c = int(threadIdx.x) + kPer * kThreads; c < n; c += kThreads)
      chain_item_store(A, W, L, c, chain_item_load(A, W, c));
    if (threadIdx.x == 0) L.diff = A.own_ks;
  }
};

// Cooperative staging (every thread of the workgroup); the caller syncs.
// Thread t takes items t + m * blockDim, two at a time with both loads
// issued before the stores.
__device__ __forceinline__ void chain_stage(const ChainArgs& A, int W, ChainLds& L) {
  if (threadIdx.x == 0) L.diff = A.own_ks;
  const int n = chain_items(A, W);
  for (int i = threadIdx.x; i < n; i += 2 * blockDim.x) {
    const int i2 = i + blockDim.x;
    const uint4 v = chain_item_load(A, W, i);
    uint4 v2 = make_uint4(0, 0, 0, 0);
    if (i2 < n) v2 = chain_item_load(A, W, i2);
    chain_item_store(A, W, L, i, v);
    if (i2 < n) chain_item_store(A, W, L, i2, v2);
  }
}


// Between the staging barrier and the next one (every thread): one staged
// word pair per lane (round keys, cut points, header), a difference sets
// L.diff.
__device__ __forceinline__ void chain_compare(const ChainArgs& A, ChainLds& L) {
  const int nint = A.intervals;
  for (int t = threadIdx.x; t < 12 + nint; t += blockDim.x) {
    bool differ;
    if (t < 11) {
      const uint4 a = L.rk[0][t], b = L.rk[1][t];
      differ = ((a.x ^ b.x) | (a.y ^ b.y) | (a.z ^ b.z) | (a.w ^ b.w)) != 0;
    } else if (t == 11) {  // nonce, in_bits
      differ = L.hdr[0][2] != L.hdr[1][2] || (L.hdr[0][0] & 0xffff) != (L.hdr[1][0] & 0xffff);
    } else {
      differ = L.cuts[0][t - 12] != L.cuts[1][t - 12];
    }
    if (differ) atomicOr(&L.diff, 1u);
  }
}

// After the barrier that follows chain_compare: the header fields and the
// shared-keystream test.
__device__ __forceinline__ ChainKeyInfo chain_key_info(const ChainArgs& A, const ChainLds& L) {
  ChainKeyInfo K;
  for (int p = 0; p < 2; ++p) {
    K.m[p] = chain_mask_bits(int(L.hdr[p][0] & 0xffff));
    K.party[p] = int(L.hdr[p][1] & 0xff);
    K.nonce[p] = L.hdr[p][2];
  }
  K.same_ks = L.diff == 0;
  return K;
}

// Beaver product k of the chain for both parties, opens summed in place.
template <class Src>
__device__ __forceinline__ Two chain_beaver(const Src& P, int k, Two u, Two v) {
  uint64_t a[2], b[2], c[2];
  P.get(k, a, b, c);
  const uint64_t d = (u.v[0] - a[0]) + (u.v[1] - a[1]);
  const uint64_t e = (v.v[0] - b[0]) + (v.v[1] - b[1]);
  return Two{{c[0] + d * b[0] + e * a[0] + d * e, c[1] + d * b[1] + e * a[1]}};
}

// Truncation gate j at the masked open of z, both parties.
// th: the gates' key headers staged in LDS (chain_stage_trunc_hdrs), or
// nullptr to read them from the keys.
__device__ __forceinline__ Two chain_trunc(const ChainArgs& A, int j, Two z,
                                          const TruncHdr (*th)[2]) {
  const uint64_t zh = z.v[0] + z.v[1] + A.tmask[j];
  if (th)
    return Two{{trunc_table_eval_h(th[j][0], A.ttab[j][0], A.tf[j], zh),
                trunc_table_eval_h(th[j][1], A.ttab[j][1], A.tf[j], zh)}};
  return Two{{trunc_table_eval(A.tkey[j][0], A.ttab[j][0], A.tf[j], zh),
              trunc_table_eval(A.tkey[j][1], A.ttab[j][1], A.tf[j], zh)}};
}

// The chain's truncation key headers into LDS, one (gate, party) per thread
// from thread `first` on: per use an LDS read instead of a header held in
// scalar registers for the whole launch.  load() issues the thread's eight
// key-word loads (unconditionally: other threads read gate 0's key) so that
// they share a round trip with the caller's other staging loads; store()
// writes the decoded header; the caller syncs.
template <int kProds>
struct TruncHdrStager {
  uint64_t w[8];
  int slot;
  __device__ __forceinline__ void load(const ChainArgs& A, int first) {
    const int t = int(threadIdx.x) - first;
    slot = t >= 0 && t < 2 * kProds ? t : -1;
    const uint8_t* key = A.tkey[0][0];
#pragma unroll
    for (int j = 0; j < kProds; ++j)
#pragma unroll
      for (int p = 0; p < 2; ++p)
        if (slot == 2 * j + p) key = A.tkey[j][p];
    const uint64_t* kw = reinterpret_cast<const uint64_t*>(key);
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = kw[i];
  }
  __device__ __forceinline__ void store(TruncHdr (*th)[2]) const {
    if (slot >= 0) th[slot >> 1][slot & 1] = decode_trunc_hdr(w);
  }
};

template <int kProds>
__device__ __forceinline__ void chain_stage_trunc_hdrs(const ChainArgs& A, TruncHdr (*th)[2]) {
  TruncHdrStager<kProds> s;
  s.load(A, 0);
  s.store(th);
}

// The products and truncations of a chain from its LUT coefficients cf
// (per element m and party p, W words), results in out[m].
template <int kKind, int M, class Src>
__device__ __forceinline__ void chain_finish_m(
    const ChainArgs& A, const uint64_t (&cf)[M][2][kKind == SUFHIP_CHAIN_CUBIC ? 4 : 2],
    const Two (&x)[M], const Src (&P)[M], Two (&out)[M], const TruncHdr (*th)[2]) {
  const int f = A.f;
  Two t1[M], t2[M];
  if constexpr (kKind == SUFHIP_CHAIN_CUBIC) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      Two mm = chain_beaver(P[m], 0, Two{{cf[m][0][3], cf[m][1][3]}}, x[m]);
      mm.v[0] += cf[m][0][2] << f;
      mm.v[1] += cf[m][1][2] << f;
      t1[m] = chain_trunc(A, 0, chain_beaver(P[m], 1, mm, x[m]), th);
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const Two q{{t1[m].v[0] + (cf[m][0][1] << f), t1[m].v[1] + (cf[m][1][1] << f)}};
      t2[m] = chain_trunc(A, 1, chain_beaver(P[m], 2, q, x[m]), th);
    }
#pragma unroll
    for (int m = 0; m < M; ++m)
      out[m] = chain_trunc(
          A, 2, Two{{t2[m].v[0] + (cf[m][0][0] << f), t2[m].v[1] + (cf[m][1][0] << f)}}, th);
  } else {
    Two y[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const Two t =
          chain_trunc(A, 0, chain_beaver(P[m], 0, Two{{cf[m][0][1], cf[m][1][1]}}, x[m]), th);
      y[m] = Two{{t.v[0] + cf[m][0][0], t.v[1] + cf[m][1][0]}};
    }
    if constexpr (kKind == SUFHIP_CHAIN_RECIP) {
#pragma unroll
      for (int m = 0; m < M; ++m) t1[m] = chain_trunc(A, 1, chain_beaver(P[m], 1, y[m], x[m]), th);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const Two two{{(uint64_t(2) << f) - t1[m].v[0], uint64_t(0) - t1[m].v[1]}};
        out[m] = chain_trunc(A, 2, chain_beaver(P[m], 2, y[m], two), th);
      }
    } else {
#pragma unroll
      for (int m = 0; m < M; ++m) t1[m] = chain_trunc(A, 1, chain_beaver(P[m], 1, y[m], y[m]), th);
#pragma unroll
      for (int m = 0; m < M; ++m) t2[m] = chain_trunc(A, 2, chain_beaver(P[m], 2, x[m], t1[m]), th);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const Two inner{{(uint64_t(3) << (f - 1)) - t2[m].v[0], uint64_t(0) - t2[m].v[1]}};
        out[m] = chain_trunc(A, 3, chain_beaver(P[m], 3, y[m], inner), th);
      }
    }
  }
}

// The whole chain for M elements at once (element m: index i[m], input
// shares x[m], triple shares from P[m], a ChainPreN or chain_loader), results
// in out[m].  Every step runs for all M elements before the next, so the
// LUT's AES blocks (both parties, W / 2 blocks each, per element) are
// encrypted in lockstep and the truncations' table reads of a step are in
// flight together: a lane pays one latency per step, not one per element and
// party.  kLockBoth: when party 1 needs its own keystream and each party has
// at most two blocks, both parties' blocks run as one lockstep group (for
// the latency-bound chains of the block kernels; the throughput-bound chain
// kernel keeps the smaller register footprint of one party at a time).
template <int kKind, class Aes, int M, class Src, bool kLockBoth = false>
__device__ __forceinline__ void chain_eval_m(const ChainArgs& A, const ChainLds& L,
                                             const ChainKeyInfo& K, const Aes& aes,
                                             const size_t (&i)[M], const Two (&x)[M],
                                             const Src (&P)[M], Two (&out)[M],
                                             const TruncHdr (*th)[2] = nullptr) {
  constexpr int W = kKind == SUFHIP_CHAIN_CUBIC ? 4 : 2;
  constexpr int NB = W / 2;  // AES blocks per element and party
  constexpr int NS = M * NB;  // blocks per party
  const int nint = A.intervals;
  int iv[M][2];
  uint32_t st[2][NS][4];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const uint64_t xh = x[m].v[0] + x[m].v[1] + A.lut_mask;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      if (p == 1 && K.same_ks) {
        iv[m][1] = iv[m][0];  // the same cut points and input mask
      } else {
        const uint64_t xm = xh & K.m[p];
        int lo = 0, hi = nint;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if ((L.cuts[p][mid] & K.m[p]) <= xm)
            lo = mid + 1;
          else
            hi = mid;
        }
        iv[m][p] = lo - 1 < 0 ? 0 : lo - 1;
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const uint64_t ctr =
            K.nonce[p] ^ (uint64_t(i[m]) << 32) ^ (uint64_t(iv[m][p]) * W + uint64_t(2 * b));
        st[p][m * NB + b][0] = uint32_t(ctr);
        st[p][m * NB + b][1] = uint32_t(ctr >> 32);
        st[p][m * NB + b][2] = 0;
        st[p][m * NB + b][3] = 0;
      }
    }
  }
  // Party 0's blocks, at most four in lockstep (more keep too many table
  // reads in flight for the register file); party 1's only where its
  // keystream differs (never for blobs from one dealer key, always under
  // the per-party policy).  A chain of at most two blocks per party runs
  // both parties' blocks in one lockstep group when party 1 needs its own:
  // one AES latency instead of two.
  constexpr int kLock = NS < 4 ? NS : 4;
  bool own1 = !K.same_ks;
#pragma unroll
  for (int m = 0; m < M; ++m) own1 = own1 || iv[m][0] != iv[m][1];
  bool both = false;
  if constexpr (kLockBoth && 2 * NS <= 4) {
    if (own1) {
      uint32_t sub[2 * NS][4];
      const uint4* subk[2 * NS];
#pragma unroll
      for (int u = 0; u < 2 * NS; ++u) {
        subk[u] = L.rk[u / NS];
#pragma unroll
        for (int q = 0; q < 4; ++q) sub[u][q] = st[u / NS][u % NS][q];
      }
      aes.template encrypt_n<2 * NS>(sub, subk);
#pragma unroll
      for (int u = 0; u < 2 * NS; ++u)
#pragma unroll
        for (int q = 0; q < 4; ++q) st[u / NS][u % NS][q] = sub[u][q];
      both = true;
    }
  }
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    if (both || (p == 1 && !own1)) continue;
#pragma unroll
    for (int n0 = 0; n0 < NS; n0 += kLock) {
      uint32_t sub[kLock][4];
      const uint4* subk[kLock];
#pragma unroll
      for (int u = 0; u < kLock; ++u) {
        subk[u] = L.rk[p];
#pragma unroll
        for (int q = 0; q < 4; ++q) sub[u][q] = st[p][n0 + u][q];
      }
      aes.template encrypt_n<kLock>(sub, subk);
#pragma unroll
      for (int u = 0; u < kLock; ++u)
#pragma unroll
        for (int q = 0; q < 4; ++q) st[p][n0 + u][q] = sub[u][q];
    }
  }
  uint64_t cf[M][2][W];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int n = m * NB + b;  // party p's block, or party 0's when shared
        const bool mine = p == 1 && own1;
        const uint64_t k0 = uint64_t(mine ? st[1][n][0] : st[0][n][0]) |
                            uint64_t(mine ? st[1][n][1] : st[0][n][1]) << 32;
        const uint64_t k1 = uint64_t(mine ? st[1][n][2] : st[0][n][2]) |
                            uint64_t(mine ? st[1][n][3] : st[0][n][3]) << 32;
        const uint64_t* row = L.pay[p] + size_t(iv[m][p]) * W;
        cf[m][p][2 * b] = K.party[p] == 0 ? k0 : row[2 * b] - k0;
        cf[m][p][2 * b + 1] = K.party[p] == 0 ? k1 : row[2 * b + 1] - k1;
      }
  chain_finish_m<kKind, M, Src>(A, cf, x, P, out, th);
}

// The whole chain for one element (chain_eval_m with M = 1).
template <int kKind, class Aes, class Src, bool kLockBoth = false>
__device__ __forceinline__ Two chain_eval(const ChainArgs& A, const ChainLds& L,
                                          const ChainKeyInfo& K, const Aes& aes,
                                          size_t i, Two x, const Src& P,
                                          const TruncHdr (*th)[2] = nullptr) {
  const size_t ii[1] = {i};
  const Two xx[1] = {x};
  const Src pp[1] = {P};
  Two out[1];
  chain_eval_m<kKind, Aes, 1, Src, kLockBoth>(A, L, K, aes, ii, xx, pp, out, th);
  return out[0];
}

// One element's RECIP or RSQRT chain computed by a whole wave (the per-row
// reciprocal and rsqrt of the block kernels): every lane runs the interval
// searches, products and truncations on the same (wave-uniform) i, x and
// triples, so every lane ends with the result, while the LUT keystream block
// of party p is encrypted column-parallel by lanes 4 p .. 4 p + 3
// (Aes::encrypt_quad_n, both parties' quads at once) and broadcast with
// readlane.  That is one quad-AES latency instead of a lane's two blocks.
// Party 1's block comes from its own blob; where the blobs are equal it is
// party 0's block, as in chain_eval_m.
template <int kKind, class Aes, class Src>
__device__ __forceinline__ Two chain_eval_quad(const ChainArgs& A, const ChainLds& L,
                                               const ChainKeyInfo& K, const Aes& aes, size_t i,
                                               Two x, const Src& P,
                                               const TruncHdr (*th)[2] = nullptr) {
  static_assert(kKind != SUFHIP_CHAIN_CUBIC, "chain_eval_quad: one keystream block per party");
  constexpr int W = 2;
  const int lane = threadIdx.x & 63;
  const uint64_t xh = x.v[0] + x.v[1] + A.lut_mask;
  int iv[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const uint64_t xm = xh & K.m[p];
    int lo = 0, hi = A.intervals;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if ((L.cuts[p][mid] & K.m[p]) <= xm)
        lo = mid + 1;
      else
        hi = mid;
    }
    iv[p] = lo - 1 < 0 ? 0 : lo - 1;
  }
  uint32_t ks = 0;
  if (lane < 8) {
    // Selects, not indexing: a lane-dependent index into the register
    // arrays iv and K.nonce would put them in private memory.
    const bool p1 = lane >= 4;
    const int q = lane & 3;
    const uint64_t ctr =
        (p1 ? K.nonce[1] : K.nonce[0]) ^ (uint64_t(i) << 32) ^ (uint64_t(p1 ? iv[1] : iv[0]) * W);
    uint32_t s[1] = {q == 0 ? uint32_t(ctr) : (q == 1 ? uint32_t(ctr >> 32) : 0u)};
    const uint32_t* const rk[1] = {reinterpret_cast<const uint32_t*>(L.rk[p1 ? 1 : 0]) + q};
    aes.template encrypt_quad_n<1>(s, rk);
    ks = s[0];  // column q of party p's block
  }
  uint64_t cf[1][2][W];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const uint64_t k0 = uint64_t(uint32_t(__builtin_amdgcn_readlane(int(ks), 4 * p))) |
                        uint64_t(uint32_t(__builtin_amdgcn_readlane(int(ks), 4 * p + 1))) << 32;
    const uint64_t k1 = uint64_t(uint32_t(__builtin_amdgcn_readlane(int(ks), 4 * p + 2))) |
                        uint64_t(uint32_t(__builtin_amdgcn_readlane(int(ks), 4 * p + 3))) << 32;
    const uint64_t* row = L.pay[p] + size_t(iv[p]) * W;
    cf[0][p][0] = K.party[p] == 0 ? k0 : row[0] - k0;
    cf[0][p][1] = K.party[p] == 0 ? k1 : row[1] - k1;
  }
  const Two xx[1] = {x};
  const Src pp[1] = {P};
  Two out[1];
  chain_finish_m<kKind, 1, Src>(A, cf, xx, pp, out, th);
  return out[0];
}

// Host: validates a chain's arguments for n elements and converts them.
// With own_io false the chain's input operand and outputs are the caller's
// business (a block kernel computes x and consumes the result) and are not
// checked.
inline int make_chain_args(const sufhip_chain2_args& g, bool own_io, const char* what,
                           ChainArgs* out) {
  auto fail = [&](const char* msg) {
    set_error(std::string(what) + ": " + msg);
    return SUFHIP_ERR_INVALID;
  };
  if (g.kind != SUFHIP_CHAIN_CUBIC && g.kind != SUFHIP_CHAIN_RECIP &&
      g.kind != SUFHIP_CHAIN_RSQRT)
    return fail("unknown kind");
  const int W = g.kind == SUFHIP_CHAIN_CUBIC ? 4 : 2;
  const int prods = g.kind == SUFHIP_CHAIN_RSQRT ? 4 : 3;
  if (g.frac_bits < 1 || g.frac_bits > kTruncTableBits - 1) return fail("frac_bits in [1, 13]");
  if (g.intervals < 1 || g.intervals > kChainMaxIntervals) return fail("intervals in [1, 64]");
  if (g.lut_key_bytes != sufhip_interval_lut_key_bytes(g.intervals, W))
    return fail("LUT key_bytes does not match (intervals, words)");
  if (g.n >= (size_t(1) << 40)) return fail("n too large");
  if (!g.lut[0] || !g.lut[1]) return fail("null LUT key");
  if ((reinterpret_cast<uintptr_t>(g.lut[0]) & 7) != 0 ||
      (reinterpret_cast<uintptr_t>(g.lut[1]) & 7) != 0)
    return fail("LUT keys must be 8-byte aligned");
  if (own_io) {
    if ((!g.out[0] || !g.out[1]) && !g.out_planes.planes) return fail("null output");
    if ((g.out[0] == nullptr) != (g.out[1] == nullptr)) return fail("one output share missing");
    if (!x_planes_ok(g.out_planes, g.n))
      return fail("out_planes: cols and n / cols multiples of 32, 16-byte aligned");
    if (int rc = check_operand(g.x, g.n, what)) return rc;
  }
  ChainArgs A{};
  A.x = g.x;
  A.lut[0] = g.lut[0];
  A.lut[1] = g.lut[1];
  A.lut_mask = g.lut_mask;
  A.intervals = g.intervals;
  A.f = g.frac_bits;
  A.n = g.n;
  A.out[0] = g.out[0];
  A.out[1] = g.out[1];
  A.xp = own_io ? g.out_planes : sufhip_x_planes{nullptr, 0};
  for (int k = 0; k < prods; ++k) {
    if (!g.a[k].p[0] || !g.b[k].p[0] || !g.c[k].p[0]) return fail("a product's triple is missing");
    if (int rc = check_term(g.a[k], g.n, false, what)) return rc;
    if (int rc = check_term(g.b[k], g.n, false, what)) return rc;
    if (int rc = check_term(g.c[k], g.n, false, what)) return rc;
    A.a[k] = g.a[k];
    A.b[k] = g.b[k];
    A.c[k] = g.c[k];
    const int want_f = (g.kind == SUFHIP_CHAIN_RSQRT && k == 2) ? g.frac_bits + 1 : g.frac_bits;
    if (g.trunc[k].frac_bits != want_f) return fail("truncation gate of the wrong width");
    sufhip_trunc_epilogue t = g.trunc[k];
    if (t.add[0] || t.add[1]) return fail("a chain's truncations take no addend");
    uint64_t dummy = 0;
    t.y[0] = t.y[1] = &dummy;  // outputs are the chain's own
    TruncEpi e;
    if (int rc = make_epi(&t, g.n, what, &e)) return rc;
    A.tkey[k][0] = e.key[0];
    A.tkey[k][1] = e.key[1];
    A.ttab[k][0] = e.table[0];
    A.ttab[k][1] = e.table[1];
    A.tmask[k] = g.trunc_mask[k];
    A.tf[k] = e.f;
  }
  auto plain = [&](const sufhip_term2& t, size_t stride) {
    return t.p[0] && t.p[1] && !t.index && t.stride == stride && t.shift == 0 && !t.negate &&
           (t.mul == 0 || t.mul == 1) && t.len >= g.n;
  };
  A.plain_x = plain(g.x.t[0], 1) && !g.x.t[1].p[0] && !g.x.t[1].p[1];
  if (A.plain_x) {
    A.px[0] = g.x.t[0].p[0];
    A.px[1] = g.x.t[0].p[1];
  }
  const size_t st = g.a[0].stride;
  A.plain = st == 1 || st == 3;
  for (int k = 0; k < prods; ++k)
    A.plain = A.plain && plain(g.a[k], st) && plain(g.b[k], st) && plain(g.c[k], st);
  if (A.plain) {
    A.pstride = int(st);
    for (int k = 0; k < prods; ++k)
      for (int p = 0; p < 2; ++p) {
        A.pa[k][p] = g.a[k].p[p] + g.a[k].off;
        A.pb[k][p] = g.b[k].p[p] + g.b[k].off;
        A.pc[k][p] = g.c[k].p[p] + g.c[k].off;
      }
  }
  A.own_ks = keystream_per_party() ? 1u : 0u;
  *out = A;
  return SUFHIP_OK;
}

}  // namespace sufhip
