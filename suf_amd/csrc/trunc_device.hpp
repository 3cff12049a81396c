// Device-side pieces of the truncation gate shared by the gate's own kernels
// (trunc_gate.hip) and the two-party kernels whose masked open feeds a
// truncation (twoparty.hip, matmul_public.hip): the key header, the
// postproc formulas (trunc_postproc_kernel, cuda/cuda_primitives.cu:179-252;
// include/gates/postproc_hooks.hpp:172-373) and the GapARS evaluation from a
// prepared full-domain carry table.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "suf_hip.h"
#include "sufhip_internal.hpp"

namespace sufhip {

constexpr uint32_t kTruncTag = 0x31475453u;  // "STG1"
constexpr int kTruncHdrBytes = 64;
// Carry keys up to this many bits are prepared as full-domain tables (one
// read per element at evaluation).
constexpr int kTruncTableBits = 14;

struct TruncHdr {
  uint32_t tag, kind, f, party, flags;
  uint64_t r_hi, base, cw, sw, m;
  uint32_t ckb, ukb;
};

// Header word 0: tag | kind << 32 | f << 40 | party << 48 | flags << 56.
// decode_trunc_hdr takes the key's first 8 words (word 1 is unused).
__device__ __forceinline__ TruncHdr decode_trunc_hdr(const uint64_t (&w)[8]) {
  const uint64_t h0 = w[0];
  TruncHdr h;
  h.tag = uint32_t(h0);
  h.kind = uint32_t(h0 >> 32) & 0xffu;
  h.f = uint32_t(h0 >> 40) & 0xffu;
  h.party = uint32_t(h0 >> 48) & 1u;
  h.flags = uint32_t(h0 >> 56);
  h.r_hi = w[2];
  h.base = w[3];
  h.cw = w[4];
  h.sw = w[5];
  h.m = w[6];
  h.ckb = uint32_t(w[7]);
  h.ukb = uint32_t(w[7] >> 32);
  return h;
}

__device__ __forceinline__ TruncHdr read_trunc_hdr(const uint8_t* key) {
  const uint64_t* w = reinterpret_cast<const uint64_t*>(key);
  const uint64_t h0 = w[0];
  TruncHdr h;
  h.tag = uint32_t(h0);
  h.kind = uint32_t(h0 >> 32) & 0xffu;
  h.f = uint32_t(h0 >> 40) & 0xffu;
  h.party = uint32_t(h0 >> 48) & 1u;
  h.flags = uint32_t(h0 >> 56);
  h.r_hi = w[2];
  h.base = w[3];
  h.cw = w[4];
  h.sw = w[5];
  h.m = w[6];
  h.ckb = uint32_t(w[7]);
  h.ukb = uint32_t(w[7] >> 32);
  return h;
}

template <int kKind>
__device__ __forceinline__ uint64_t trunc_postproc(const TruncHdr& h, int f, uint64_t x,
                                                   uint64_t carry, uint64_t wrap, uint64_t sign) {
  if constexpr (kKind == SUFHIP_TRUNC_GAPARS) {
    const uint64_t hb = x + (uint64_t(1) << 62);
    uint64_t y = h.base + (h.party == 0 ? hb >> f : 0) - h.r_hi - carry;
    if ((hb >> 63) == 0) y += h.m;
    if (h.party == 0) y -= uint64_t(1) << (62 - f);
    return y;
  } else {
    uint64_t y = h.base + (h.party == 0 ? x >> f : 0) - h.r_hi - carry +
                 wrap * (uint64_t(1) << (64 - f));
    if constexpr (kKind == SUFHIP_TRUNC_ARS) y += sign * (~uint64_t(0) << (64 - f));
    return y;
  }
}

// carry share = NOT(RotXor(a, 0, w)) = [p0] - w + a.
__device__ __forceinline__ uint64_t trunc_carry_from(const TruncHdr& h, uint64_t a) {
  return (h.party == 0 ? 1 : 0) - h.cw + a;
}

// One party's GapARS output at the public xhat from the key's header and its
// prepared full-domain table (node v's value word holds the carry DCF's
// share at v).  A key that is not a GapARS key for f bits yields 0; the table
// read stays inside its 2^f nodes either way.
__device__ __forceinline__ uint64_t trunc_table_eval_h(const TruncHdr& h, const uint4* table,
                                                       int f, uint64_t xhat) {
  if (h.tag != kTruncTag || h.kind != SUFHIP_TRUNC_GAPARS || int(h.f) != f) return 0;
  uint64_t carry = 0;
  if (h.flags & 1) {
    const uint4 q = table[2 * (xhat & ((uint64_t(1) << f) - 1)) + 1];
    carry = trunc_carry_from(h, uint64_t(q.x) | uint64_t(q.y) << 32);
  }
  return trunc_postproc<SUFHIP_TRUNC_GAPARS>(h, f, xhat, carry, 0, 0);
}

__device__ __forceinline__ uint64_t trunc_table_eval(const uint8_t* key, const uint4* table,
                                                     int f, uint64_t xhat) {
  return trunc_table_eval_h(read_trunc_hdr(key), table, f, xhat);
}

// A truncation gate folded into the launch that produces its masked open.
struct TruncEpi {
  const uint8_t* key[2];
  const uint4* table[2];
  uint64_t* y[2];
  const uint64_t* add[2];  // optional addend of the outputs (a residual)
  int f;
  int on;
};

// trunc_table_eval_h in two halves, so that a caller can issue several
// elements' table reads before it uses any: the table's value word at xhat
// (0 where the gate reads none), then the output from that word.
__device__ __forceinline__ bool trunc_table_key_ok(const TruncHdr& h, int f) {
  return h.tag == kTruncTag && h.kind == SUFHIP_TRUNC_GAPARS && int(h.f) == f;
}
__device__ __forceinline__ uint64_t trunc_table_word(const TruncHdr& h, const uint4* table, int f,
                                                     uint64_t xhat) {
  if (!trunc_table_key_ok(h, f) || !(h.flags & 1)) return 0;
  const uint4 q = table[2 * (xhat & ((uint64_t(1) << f) - 1)) + 1];
  return uint64_t(q.x) | uint64_t(q.y) << 32;
}
__device__ __forceinline__ uint64_t trunc_table_out(const TruncHdr& h, int f, uint64_t xhat,
                                                    uint64_t word) {
  if (!trunc_table_key_ok(h, f)) return 0;
  const uint64_t carry = (h.flags & 1) ? trunc_carry_from(h, word) : 0;
  return trunc_postproc<SUFHIP_TRUNC_GAPARS>(h, f, xhat, carry, 0, 0);
}

// The two parties' key headers of an epilogue, read once before the
// caller's element loop.  Read inside it, each header load would follow the
// previous element's output stores, which may alias the keys as far as the
// compiler knows, so every element would wait for two fresh header loads.
struct EpiHdrs {
  TruncHdr h[2];
};
__device__ __forceinline__ EpiHdrs epi_hdrs(const TruncEpi& e) {
  EpiHdrs r{};
  if (e.on) {
    r.h[0] = read_trunc_hdr(e.key[0]);
    r.h[1] = read_trunc_hdr(e.key[1]);
  }
  return r;
}

// Writes the open values v[t] of elements i[t], t < N: the gate's two
// output shares (plus the addend) when the epilogue is on, else the opens
// themselves (if requested).  Every table and addend read is issued before
// the first output store.
template <int N>
__device__ __forceinline__ void put_open_n(const TruncEpi& e, const EpiHdrs& eh, uint64_t* hat,
                                           const size_t (&i)[N], const uint64_t (&v)[N]) {
  if (e.on) {
    uint64_t w[N][2], ad[N][2];
#pragma unroll
    for (int t = 0; t < N; ++t) {
      w[t][0] = trunc_table_word(eh.h[0], e.table[0], e.f, v[t]);
      w[t][1] = trunc_table_word(eh.h[1], e.table[1], e.f, v[t]);
      ad[t][0] = e.add[0] ? e.add[0][i[t]] : 0;
      ad[t][1] = e.add[0] ? e.add[1][i[t]] : 0;
    }
#pragma unroll
    for (int t = 0; t < N; ++t) {
      e.y[0][i[t]] = trunc_table_out(eh.h[0], e.f, v[t], w[t][0]) + ad[t][0];
      e.y[1][i[t]] = trunc_table_out(eh.h[1], e.f, v[t], w[t][1]) + ad[t][1];
    }
  } else if (hat) {
#pragma unroll
    for (int t = 0; t < N; ++t) hat[i[t]] = v[t];
  }
}

__device__ __forceinline__ void put_open(const TruncEpi& e, const EpiHdrs& eh, uint64_t* hat,
                                         size_t i, uint64_t v) {
  const size_t ii[1] = {i};
  const uint64_t vv[1] = {v};
  put_open_n<1>(e, eh, hat, ii, vv);
}

// Validates an epilogue for n elements and converts it (NULL -> off).
inline int make_epi(const sufhip_trunc_epilogue* t, size_t n, const char* what, TruncEpi* out) {
  *out = TruncEpi{{nullptr, nullptr}, {nullptr, nullptr}, {nullptr, nullptr}, {nullptr, nullptr},
                  0, 0};
  if (!t) return SUFHIP_OK;
  if ((t->add[0] == nullptr) != (t->add[1] == nullptr)) {
    set_error(std::string(what) + ": truncation epilogue addend needs both parties or neither");
    return SUFHIP_ERR_INVALID;
  }
  const bool ok = t->frac_bits >= 1 && t->frac_bits <= kTruncTableBits && t->key[0] &&
                  t->key[1] && t->table[0] && t->table[1] && t->y[0] && t->y[1] &&
                  (reinterpret_cast<uintptr_t>(t->key[0]) & 7) == 0 &&
                  (reinterpret_cast<uintptr_t>(t->key[1]) & 7) == 0 &&
                  (reinterpret_cast<uintptr_t>(t->table[0]) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(t->table[1]) & 15) == 0;
  if (!ok) {
    set_error(std::string(what) + ": truncation epilogue needs frac_bits in [1, 14], both keys, "
              "tables and outputs, aligned");
    return SUFHIP_ERR_INVALID;
  }
  if (t->work_bytes < sufhip_trunc_work_bytes(t->frac_bits, n > 0 ? n : 1)) {
    set_error(std::string(what) + ": truncation epilogue table smaller than its work bytes");
    return SUFHIP_ERR_INVALID;
  }
  *out = TruncEpi{{t->key[0], t->key[1]},
                  {static_cast<const uint4*>(t->table[0]), static_cast<const uint4*>(t->table[1])},
                  {t->y[0], t->y[1]},
                  {t->add[0], t->add[1]},
                  t->frac_bits,
                  1};
  return SUFHIP_OK;
}

}  // namespace sufhip
