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
  size_t n;
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
};

// Sources of an element's triple shares for product k, both parties:
// ChainPre holds them all, loaded before the chain starts (in LDS, for a
// chain run by a lone lane, so that no product waits for its loads);
// chain_loader loads each product's shares when it is reached (for the
// element-parallel kernel, where other waves hide the latency and registers
// set the occupancy).
struct ChainPre {
  uint64_t a[4][2], b[4][2], c[4][2];
  __device__ __forceinline__ void get(int k, uint64_t* a3, uint64_t* b3, uint64_t* c3) const {
    for (int p = 0; p < 2; ++p) {
      a3[p] = a[k][p];
      b3[p] = b[k][p];
      c3[p] = c[k][p];
    }
  }
};

template <int kKind>
struct chain_loader {
  const ChainArgs& A;
  size_t i;
  __device__ __forceinline__ void get(int k, uint64_t* a3, uint64_t* b3, uint64_t* c3) const {
    for (int p = 0; p < 2; ++p) {
      a3[p] = term_at(A.a[k], p, i);
      b3[p] = term_at(A.b[k], p, i);
      c3[p] = term_at(A.c[k], p, i);
    }
  }
};

template <int kKind>
constexpr int chain_products() {
  return kKind == SUFHIP_CHAIN_RSQRT ? 4 : 3;
}

// Per-party LUT header fields: input mask, keystream nonce, party.
struct ChainKeyInfo {
  uint64_t m[2], nonce[2];
  int party[2];
};

__device__ __forceinline__ uint64_t chain_mask_bits(int bits) {
  return bits <= 0 ? 0 : (bits >= 64 ? ~uint64_t(0) : (uint64_t(1) << bits) - 1);
}

// Cooperative staging (every thread of the workgroup); the caller syncs.
__device__ __forceinline__ void chain_stage(const ChainArgs& A, int W, ChainLds& L) {
  const int nint = A.intervals;
  for (int p = 0; p < 2; ++p) {
    const uint8_t* k = A.lut[p];
    const uint32_t* rkg = reinterpret_cast<const uint32_t*>(k + 40);
    for (int i = threadIdx.x; i < 11; i += blockDim.x)
      L.rk[p][i] = make_uint4(rkg[4 * i], rkg[4 * i + 1], rkg[4 * i + 2], rkg[4 * i + 3]);
    const uint64_t* cg = reinterpret_cast<const uint64_t*>(k + kChainLutHdr);
    const uint64_t* pg = cg + (nint + 1);
    for (int i = threadIdx.x; i < nint; i += blockDim.x) L.cuts[p][i] = cg[i];
    for (int i = threadIdx.x; i < nint * W; i += blockDim.x) L.pay[p][i] = pg[i];
  }
}


__device__ __forceinline__ ChainKeyInfo chain_key_info(const ChainArgs& A) {
  ChainKeyInfo K;
  for (int p = 0; p < 2; ++p) {
    K.m[p] = chain_mask_bits(*reinterpret_cast<const uint16_t*>(A.lut[p]));
    K.party[p] = A.lut[p][8];
    K.nonce[p] = *reinterpret_cast<const uint64_t*>(A.lut[p] + 16);
  }
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
__device__ __forceinline__ Two chain_trunc(const ChainArgs& A, int j, Two z) {
  const uint64_t zh = z.v[0] + z.v[1] + A.tmask[j];
  return Two{{trunc_table_eval(A.tkey[j][0], A.ttab[j][0], A.tf[j], zh),
              trunc_table_eval(A.tkey[j][1], A.ttab[j][1], A.tf[j], zh)}};
}

// The whole chain for element i with input shares x, its triple shares
// from P (ChainPre or chain_loader).
template <int kKind, int kCopies, class Src>
__device__ __forceinline__ Two chain_eval(const ChainArgs& A, const ChainLds& L,
                                          const ChainKeyInfo& K, const AesLds<kCopies>& aes,
                                          size_t i, Two x, const Src& P) {
  constexpr int W = kKind == SUFHIP_CHAIN_CUBIC ? 4 : 2;
  const int nint = A.intervals, f = A.f;
  const uint64_t xh = x.v[0] + x.v[1] + A.lut_mask;
  uint64_t cf[2][W];
  for (int p = 0; p < 2; ++p) {
    const uint64_t xm = xh & K.m[p];
    int lo = 0, hi = nint;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if ((L.cuts[p][mid] & K.m[p]) <= xm)
        lo = mid + 1;
      else
        hi = mid;
    }
    int iv = lo - 1;
    if (iv < 0) iv = 0;
#pragma unroll
    for (int w = 0; w < W; w += 2) {
      const uint64_t ctr = K.nonce[p] ^ (uint64_t(i) << 32) ^ (uint64_t(iv) * W + uint64_t(w));
      uint32_t s0 = uint32_t(ctr), s1 = uint32_t(ctr >> 32), s2 = 0, s3 = 0;
      aes.encrypt(s0, s1, s2, s3, L.rk[p]);
      const uint64_t k0 = uint64_t(s0) | uint64_t(s1) << 32;
      const uint64_t k1 = uint64_t(s2) | uint64_t(s3) << 32;
      const uint64_t* row = L.pay[p] + size_t(iv) * W;
      cf[p][w] = K.party[p] == 0 ? k0 : row[w] - k0;
      cf[p][w + 1] = K.party[p] == 0 ? k1 : row[w + 1] - k1;
    }
  }
  if constexpr (kKind == SUFHIP_CHAIN_CUBIC) {
    Two mm = chain_beaver(P, 0, Two{{cf[0][3], cf[1][3]}}, x);
    mm.v[0] += cf[0][2] << f;
    mm.v[1] += cf[1][2] << f;
    const Two y = chain_trunc(A, 0, chain_beaver(P, 1, mm, x));
    const Two q{{y.v[0] + (cf[0][1] << f), y.v[1] + (cf[1][1] << f)}};
    const Two y2 = chain_trunc(A, 1, chain_beaver(P, 2, q, x));
    return chain_trunc(A, 2, Two{{y2.v[0] + (cf[0][0] << f), y2.v[1] + (cf[1][0] << f)}});
  } else {
    const Two t = chain_trunc(A, 0, chain_beaver(P, 0, Two{{cf[0][1], cf[1][1]}}, x));
    const Two y{{t.v[0] + cf[0][0], t.v[1] + cf[1][0]}};
    if constexpr (kKind == SUFHIP_CHAIN_RECIP) {
      const Two xy = chain_trunc(A, 1, chain_beaver(P, 1, y, x));
      const Two two{{(uint64_t(2) << f) - xy.v[0], uint64_t(0) - xy.v[1]}};
      return chain_trunc(A, 2, chain_beaver(P, 2, y, two));
    } else {
      const Two y2 = chain_trunc(A, 1, chain_beaver(P, 1, y, y));
      const Two h = chain_trunc(A, 2, chain_beaver(P, 2, x, y2));
      const Two inner{{(uint64_t(3) << (f - 1)) - h.v[0], uint64_t(0) - h.v[1]}};
      return chain_trunc(A, 3, chain_beaver(P, 3, y, inner));
    }
  }
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
    if (!g.out[0] || !g.out[1]) return fail("null output");
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
  *out = A;
  return SUFHIP_OK;
}

}  // namespace sufhip
