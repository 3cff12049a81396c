// myl7/fss v0.7.1 DCF (lambda = 16, AES-128-MMO PRG) on CDNA4: batched key
// generation and evaluation over SUF's myl7 adapter key blobs.
//
// Evaluation (third_party/myl7_fss/src/dcf.c:146-193) walks the tree from
// bit in_bits-1 down to bit 0.  At each level the reference expands the seed
// into four blocks (sl, vl, sr, vr) with four AES calls, then keeps only the
// side selected by the input bit.  Here each lane computes just the two
// blocks on that side -- AES_{K_{2b}} for the next seed and AES_{K_{2b+1}}
// for the value block, b = x_i -- which halves the AES work without changing
// any output byte.  When only share byte 0 bit 0 is needed (the
// eval_dcf_many_u64 contract, include/proto/myl7_fss_backend.hpp:88-99), the
// value block is reduced to its first byte: bit 0 of a sum or XOR depends
// only on bit 0 of the terms, and bit 0 of -v equals bit 0 of v, so this
// holds for both output groups.
//
// One element per lane; each lane streams its own key front to back
// (33 bytes per level), so successive levels hit the same cache lines.
#include <hip/hip_runtime.h>

#include <cstring>

#include "aes_lds.hpp"
#include "sufhip_internal.hpp"

namespace sufhip {
namespace {

// One workgroup per CU: the two replicated AES tables take 128 KB of the
// CU's 160 KB LDS.  Kernels loop over the batch in grid strides.
#ifndef SUFHIP_DCF_BLOCK
#define SUFHIP_DCF_BLOCK 512
#endif
constexpr int kDcfBlock = SUFHIP_DCF_BLOCK;

struct Prg4 {
  uint32_t rk[4][44];  // K_0..K_3: DCF uses PRG output blocks 0..3
};

struct DcfEvalArgs {
  Prg4 prg;
  const uint8_t* keys;
  const uint64_t* xs;
  void* out;
  size_t key_bytes;
  size_t n;
  int broadcast;
  int in_bits;
  int chunks;     // chunks to evaluate (1 for the bit modes)
  int out_bytes;  // bytes per element (OUT_BYTES)
};

struct U128 {
  uint64_t lo, hi;
};

__device__ __forceinline__ U128 mk(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
  return U128{uint64_t(w0) | uint64_t(w1) << 32, uint64_t(w2) | uint64_t(w3) << 32};
}

constexpr uint64_t kMsbClear = 0x7fffffffffffffffull;

template <int kGroup>
__device__ __forceinline__ U128 gadd(U128 a, U128 b) {
  if constexpr (kGroup == SUFHIP_GROUP_XOR) {
    return U128{a.lo ^ b.lo, a.hi ^ b.hi};
  } else {
    uint64_t lo = a.lo + b.lo;
    uint64_t hi = a.hi + b.hi + (lo < a.lo ? 1 : 0);
    return U128{lo, hi & kMsbClear};
  }
}

template <int kGroup>
__device__ __forceinline__ U128 gneg(U128 a) {
  if constexpr (kGroup == SUFHIP_GROUP_XOR) {
    return a;
  } else {
    uint64_t lo = 0 - a.lo;
    uint64_t hi = ~a.hi + (lo == 0 ? 1 : 0);
    return U128{lo, hi & kMsbClear};
  }
}

// Per-level correction word fields needed by the bit modes:
// s_cw (16 bytes), v_cw byte 0, and the t byte (tl << 1 | tr).
struct CwBit {
  uint32_t s[4];
  uint32_t v0;
  uint32_t tb;
};

__device__ __forceinline__ CwBit load_cw_bit(const uint8_t* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t* q = reinterpret_cast<const uint32_t*>(a & ~uintptr_t(3));
  const uint32_t sh = uint32_t(a & 3);
  // Bytes [0, 17) and byte 32 of the record; words 0..4 and 8 of the aligned
  // window always lie inside the record (it is 33 bytes, sh <= 3).
  uint32_t r0 = q[0], r1 = q[1], r2 = q[2], r3 = q[3], r4 = q[4], r8 = q[8];
  CwBit c;
  c.s[0] = __builtin_amdgcn_alignbyte(r1, r0, sh);
  c.s[1] = __builtin_amdgcn_alignbyte(r2, r1, sh);
  c.s[2] = __builtin_amdgcn_alignbyte(r3, r2, sh);
  c.s[3] = __builtin_amdgcn_alignbyte(r4, r3, sh);
  c.v0 = (r4 >> (8 * sh)) & 0xffu;
  c.tb = (r8 >> (8 * sh)) & 0xffu;
  return c;
}

struct CwFull {
  uint32_t s[4];
  uint32_t v[4];
  uint32_t tb;
};

__device__ __forceinline__ CwFull load_cw_full(const uint8_t* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t* q = reinterpret_cast<const uint32_t*>(a & ~uintptr_t(3));
  const uint32_t sh = uint32_t(a & 3);
  uint32_t r[9];
#pragma unroll
  for (int j = 0; j < 9; ++j) r[j] = q[j];
  CwFull c;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    c.s[j] = __builtin_amdgcn_alignbyte(r[j + 1], r[j], sh);
    c.v[j] = __builtin_amdgcn_alignbyte(r[j + 5], r[j + 4], sh);
  }
  c.tb = (r[8] >> (8 * sh)) & 0xffu;
  return c;
}

// Reads 16 bytes at p; the word after them is read only if it belongs to the
// same key (`more` = bytes remaining in the key after p + 16 > 0).
__device__ __forceinline__ void load16(const uint8_t* p, bool more, uint32_t (&w)[4]) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t* q = reinterpret_cast<const uint32_t*>(a & ~uintptr_t(3));
  const uint32_t sh = uint32_t(a & 3);
  uint32_t r0 = q[0], r1 = q[1], r2 = q[2], r3 = q[3];
  uint32_t r4 = (sh != 0 && more) ? q[4] : 0u;
  w[0] = __builtin_amdgcn_alignbyte(r1, r0, sh);
  w[1] = __builtin_amdgcn_alignbyte(r2, r1, sh);
  w[2] = __builtin_amdgcn_alignbyte(r3, r2, sh);
  w[3] = __builtin_amdgcn_alignbyte(r4, r3, sh);
}

// Bit-mode walk of one chunk: returns share byte 0 & 1.
__device__ __forceinline__ uint32_t walk_bit(const AesLds2& aes, const uint4* rkl,
                                             const uint8_t* chunk, int in_bits, uint64_t x,
                                             uint32_t party) {
  uint32_t seed[4];
  load16(chunk, true, seed);
  uint32_t s0 = seed[0], s1 = seed[1], s2 = seed[2], s3 = seed[3] & 0x7fffffffu;
  uint32_t t = party;
  uint32_t v = 0;
  const uint8_t* cw = chunk + 16;
  for (int i = 0; i < in_bits; ++i, cw += 33) {
    const uint32_t xi = uint32_t(x >> (in_bits - 1 - i)) & 1u;
    const CwBit c = load_cw_bit(cw);
    uint32_t a0 = s0, a1 = s1, a2 = s2, a3 = s3;
const uint4* ks = rkl + 22 * xi;  // K_{2 x_i}: next seed
    const uint4* kv = ks + 11;         // K_{2 x_i + 1}: value block
    aes.encrypt(a0, a1, a2, a3, ks);
    const uint32_t vb = (aes.encrypt_byte0(s0, s1, s2, s3, kv) ^ s0) & 1u;
    a0 ^= s0;
    a1 ^= s1;
    a2 ^= s2;
    a3 ^= s3;
    uint32_t tn = a3 >> 31;
    a3 &= 0x7fffffffu;
    const uint32_t tmask = 0u - t;
    a0 ^= c.s[0] & tmask;
    a1 ^= c.s[1] & tmask;
    a2 ^= c.s[2] & tmask;
    a3 ^= c.s[3] & tmask;
    tn ^= ((xi ? c.tb : (c.tb >> 1)) & 1u) & t;
    v ^= vb ^ (c.v0 & t & 1u);
    s0 = a0;
    s1 = a1;
    s2 = a2;
    s3 = a3;
    t = tn;
  }
  uint32_t np1[4];
  load16(cw, false, np1);
  return (v ^ s0 ^ (np1[0] & t)) & 1u;
}

// Full-block walk of one chunk (any group): returns the 16-byte share.
template <int kGroup>
__device__ __forceinline__ U128 walk_full(const AesLds2& aes, const uint4* rkl,
                                          const uint8_t* chunk, int in_bits, uint64_t x,
                                          uint32_t party, bool more_after) {
  uint32_t seed[4];
  load16(chunk, true, seed);
  uint32_t s0 = seed[0], s1 = seed[1], s2 = seed[2], s3 = seed[3] & 0x7fffffffu;
  uint32_t t = party;
  U128 v{0, 0};
  const uint8_t* cw = chunk + 16;
  for (int i = 0; i < in_bits; ++i, cw += 33) {
    const uint32_t xi = uint32_t(x >> (in_bits - 1 - i)) & 1u;
    const CwFull c = load_cw_full(cw);
    const uint4* ks = rkl + 22 * xi;
    const uint4* kv = ks + 11;
    uint32_t a0 = s0, a1 = s1, a2 = s2, a3 = s3;
    uint32_t b0 = s0, b1 = s1, b2 = s2, b3 = s3;
    aes.encrypt(a0, a1, a2, a3, ks);
    aes.encrypt(b0, b1, b2, b3, kv);
    a0 ^= s0;
    a1 ^= s1;
    a2 ^= s2;
    a3 ^= s3;
    U128 vd = mk(b0 ^ s0, b1 ^ s1, b2 ^ s2, (b3 ^ s3) & 0x7fffffffu);
    uint32_t tn = a3 >> 31;
    a3 &= 0x7fffffffu;
    if (t) {
      a0 ^= c.s[0];
      a1 ^= c.s[1];
      a2 ^= c.s[2];
      a3 ^= c.s[3];
      tn ^= (xi ? c.tb : (c.tb >> 1)) & 1u;
      vd = gadd<kGroup>(vd, mk(c.v[0], c.v[1], c.v[2], c.v[3]));
    }
    if (party) vd = gneg<kGroup>(vd);
    v = gadd<kGroup>(v, vd);
    s0 = a0;
    s1 = a1;
    s2 = a2;
    s3 = a3;
    t = tn;
  }
  uint32_t np1[4];
  load16(cw, more_after, np1);
  U128 s = mk(s0, s1, s2, s3);
  if (t) s = gadd<kGroup>(s, mk(np1[0], np1[1], np1[2], np1[3]));
  if (party) s = gneg<kGroup>(s);
  return gadd<kGroup>(v, s);
}

// Stages the replicated tables and the K_0..K_3 round keys in LDS.
#define SUFHIP_DCF_LDS_SETUP(PRG)                                  \
  __shared__ uint32_t tabs[2 * AesLds2::kWordsPerTable];           \
  __shared__ uint4 rkl[4 * 11];                                    \
  fill_ttable2(tabs, kTDev.v);                                     \
  fill_round_keys(rkl, (PRG).rk, 4);                               \
  __syncthreads();                                                 \
  const uint32_t lane4 = (threadIdx.x & 63u) * 4u;                 \
  const AesLds2 aes{tabs, lane4, lane4 | 0x10000u}

template <int kMode>
__global__ void __launch_bounds__(kDcfBlock) dcf_eval_bit_kernel(DcfEvalArgs a) {
  SUFHIP_DCF_LDS_SETUP(a.prg);
  const size_t stride = size_t(gridDim.x) * kDcfBlock;
  for (size_t base = size_t(blockIdx.x) * kDcfBlock; base < a.n; base += stride) {
    const size_t e = base + threadIdx.x;
    uint32_t bit = 0;
    if (e < a.n) {
      const uint8_t* key = a.broadcast ? a.keys : a.keys + e * a.key_bytes;
      const uint32_t party = key[2] & 1u;
      uint64_t x = a.xs[e];
      if (a.in_bits < 64) x &= (uint64_t(1) << a.in_bits) - 1;
      bit = walk_bit(aes, rkl, key + 8, a.in_bits, x, party);
    }
    if constexpr (kMode == SUFHIP_DCF_OUT_BIT) {
      if (e < a.n) static_cast<uint8_t*>(a.out)[e] = uint8_t(bit);
    } else {
      // Waves cover 64 consecutive elements starting at a multiple of 64.
      const uint64_t word = __ballot(bit != 0);
      if ((threadIdx.x & 63) == 0 && e < a.n) static_cast<uint64_t*>(a.out)[e >> 6] = word;
    }
  }
}

template <int kGroup>
__global__ void __launch_bounds__(kDcfBlock) dcf_eval_bytes_kernel(DcfEvalArgs a) {
  SUFHIP_DCF_LDS_SETUP(a.prg);
  const size_t stride = size_t(gridDim.x) * kDcfBlock;
  const size_t chunk_bytes = 32 + 33 * size_t(a.in_bits);
  for (size_t e = size_t(blockIdx.x) * kDcfBlock + threadIdx.x; e < a.n; e += stride) {
    const uint8_t* key = a.broadcast ? a.keys : a.keys + e * a.key_bytes;
    const uint32_t party = key[2] & 1u;
    uint64_t x = a.xs[e];
    if (a.in_bits < 64) x &= (uint64_t(1) << a.in_bits) - 1;
    uint8_t* out = static_cast<uint8_t*>(a.out) + e * size_t(a.out_bytes);
    for (int c = 0; c < a.chunks; ++c) {
      const bool more = (c + 1) * chunk_bytes + 8 < a.key_bytes;
      U128 r = walk_full<kGroup>(aes, rkl, key + 8 + c * chunk_bytes, a.in_bits, x, party, more);
      const int base = 16 * c;
      const int take = a.out_bytes - base < 16 ? a.out_bytes - base : 16;
      for (int b = 0; b < take; ++b) {
        const uint64_t word = b < 8 ? r.lo : r.hi;
        out[base + b] = uint8_t(word >> (8 * (b & 7)));
      }
    }
  }
}

// ---------------------------------------------------------------- keygen --

// Sequential little-endian byte writer: stores aligned dwords where it can
// and single bytes at unaligned edges, so lanes writing neighbouring keys
// never touch each other's bytes.
struct ByteWriter {
  uint8_t* p;
  uint64_t acc;
  int n;
  __device__ __forceinline__ void drain() {
    while (n > 0) {
      if ((reinterpret_cast<uintptr_t>(p) & 3) == 0) {
        if (n < 4) break;
        *reinterpret_cast<uint32_t*>(p) = uint32_t(acc);
        p += 4;
        acc >>= 32;
        n -= 4;
      } else {
        *p = uint8_t(acc);
        ++p;
        acc >>= 8;
        --n;
      }
    }
  }
  __device__ __forceinline__ void put8(uint32_t b) {
    acc |= uint64_t(b & 0xffu) << (8 * n);
    ++n;
    drain();
  }
  __device__ __forceinline__ void put32(uint32_t w) {
    acc |= uint64_t(w) << (8 * n);
    n += 4;
    drain();
  }
  __device__ __forceinline__ void flush() {
    while (n > 0) {
      *p = uint8_t(acc);
      ++p;
      acc >>= 8;
      --n;
    }
  }
};

struct DcfGenArgs {
  Prg4 prg;
  const uint64_t* alpha;
  const uint8_t* payload;
  const uint8_t* seeds;
  uint8_t* keys0;
  uint8_t* keys1;
  size_t key_bytes;
  size_t n;
  int payload_bcast;
  int payload_len;
  int in_bits;
  int chunks;
};

__device__ __forceinline__ void prg4(const AesLds2& aes, const uint4* rkl, const U128& s,
                                     U128 (&o)[4]) {
  const uint32_t w0 = uint32_t(s.lo), w1 = uint32_t(s.lo >> 32), w2 = uint32_t(s.hi),
                 w3 = uint32_t(s.hi >> 32);
  // One block at a time keeps the dealer kernel inside the register budget.
#pragma unroll 1
  for (int j = 0; j < 4; ++j) {
    uint32_t a0 = w0, a1 = w1, a2 = w2, a3 = w3;
    aes.encrypt(a0, a1, a2, a3, rkl + 11 * j);
    o[j] = mk(a0 ^ w0, a1 ^ w1, a2 ^ w2, a3 ^ w3);
  }
}

__device__ __forceinline__ void put128(ByteWriter& w, U128 v) {
  w.put32(uint32_t(v.lo));
  w.put32(uint32_t(v.lo >> 32));
  w.put32(uint32_t(v.hi));
  w.put32(uint32_t(v.hi >> 32));
}

template <int kGroup>
__device__ __forceinline__ void gen_one(const AesLds2& aes, const uint4* rkl, const DcfGenArgs& a,
                                        size_t e) {
  const int nb = a.in_bits;
  uint64_t alpha = a.alpha[e];
  if (nb < 64) alpha &= (uint64_t(1) << nb) - 1;
  const uint8_t* pay = a.payload_bcast ? a.payload : a.payload + e * size_t(a.payload_len);
  ByteWriter w0{a.keys0 + e * a.key_bytes, 0, 0};
  ByteWriter w1{a.keys1 + e * a.key_bytes, 0, 0};
  const uint32_t plen = uint32_t(a.payload_len);
  w0.put32(uint32_t(nb) | uint32_t(a.chunks) << 8 | 0u << 16);
  w1.put32(uint32_t(nb) | uint32_t(a.chunks) << 8 | 1u << 16);
  w0.put32(plen);
  w1.put32(plen);
  for (int c = 0; c < a.chunks; ++c) {
    uint8_t beta_b[16];
    for (int b = 0; b < 16; ++b) {
      const int idx = 16 * c + b;
      beta_b[b] = idx < a.payload_len ? pay[idx] : 0;
    }
    U128 beta{0, 0};
    for (int b = 0; b < 8; ++b) beta.lo |= uint64_t(beta_b[b]) << (8 * b);
    for (int b = 0; b < 8; ++b) beta.hi |= uint64_t(beta_b[8 + b]) << (8 * b);
    beta.hi &= kMsbClear;
    const uint8_t* sp = a.seeds + (e * size_t(a.chunks) + c) * 32;
    uint32_t sw[8];
    for (int j = 0; j < 8; ++j) {
      sw[j] = uint32_t(sp[4 * j]) | uint32_t(sp[4 * j + 1]) << 8 | uint32_t(sp[4 * j + 2]) << 16 |
              uint32_t(sp[4 * j + 3]) << 24;
    }
    for (int j = 0; j < 4; ++j) w0.put32(sw[j]);
    for (int j = 0; j < 4; ++j) w1.put32(sw[4 + j]);
    U128 s0 = mk(sw[0], sw[1], sw[2], sw[3]);
    U128 s1 = mk(sw[4], sw[5], sw[6], sw[7]);
    s0.hi &= kMsbClear;
    s1.hi &= kMsbClear;
    uint32_t t0 = 0, t1 = 1;
    U128 v{0, 0};
    for (int i = 0; i < nb; ++i) {
      U128 e0[4], e1[4];
      prg4(aes, rkl, s0, e0);
      prg4(aes, rkl, s1, e1);
      const uint32_t t0l = uint32_t(e0[0].hi >> 63), t0r = uint32_t(e0[2].hi >> 63);
      const uint32_t t1l = uint32_t(e1[0].hi >> 63), t1r = uint32_t(e1[2].hi >> 63);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        e0[j].hi &= kMsbClear;
        e1[j].hi &= kMsbClear;
      }
      const uint32_t ai = uint32_t(alpha >> (nb - 1 - i)) & 1u;
      // lose = side alpha does not take, keep = side it takes
      const U128 s0_lose = ai ? e0[0] : e0[2], s1_lose = ai ? e1[0] : e1[2];
      const U128 v0_lose = ai ? e0[1] : e0[3], v1_lose = ai ? e1[1] : e1[3];
      const U128 s0_keep = ai ? e0[2] : e0[0], s1_keep = ai ? e1[2] : e1[0];
      const U128 v0_keep = ai ? e0[3] : e0[1], v1_keep = ai ? e1[3] : e1[1];
      const U128 s_cw{s0_lose.lo ^ s1_lose.lo, s0_lose.hi ^ s1_lose.hi};
      U128 v_cw = gadd<kGroup>(v1_lose, gneg<kGroup>(v0_lose));
      v_cw = gadd<kGroup>(v_cw, gneg<kGroup>(v));
      if (t1) v_cw = gneg<kGroup>(v_cw);
      if (ai) v_cw = gadd<kGroup>(v_cw, t1 ? gneg<kGroup>(beta) : beta);
      v = gadd<kGroup>(v, gneg<kGroup>(v1_keep));
      v = gadd<kGroup>(v, v0_keep);
      v = gadd<kGroup>(v, t1 ? gneg<kGroup>(v_cw) : v_cw);
      const uint32_t tl_cw = t0l ^ t1l ^ ai ^ 1u;
      const uint32_t tr_cw = t0r ^ t1r ^ ai;
      put128(w0, s_cw);
      put128(w1, s_cw);
      put128(w0, v_cw);
      put128(w1, v_cw);
      w0.put8(tl_cw << 1 | tr_cw);
      w1.put8(tl_cw << 1 | tr_cw);
      const uint32_t t0k = ai ? t0r : t0l, t1k = ai ? t1r : t1l, tcwk = ai ? tr_cw : tl_cw;
      s0 = t0 ? U128{s0_keep.lo ^ s_cw.lo, s0_keep.hi ^ s_cw.hi} : s0_keep;
      s1 = t1 ? U128{s1_keep.lo ^ s_cw.lo, s1_keep.hi ^ s_cw.hi} : s1_keep;
      t0 = t0 ? (t0k ^ tcwk) : t0k;
      t1 = t1 ? (t1k ^ tcwk) : t1k;
    }
    U128 last = gadd<kGroup>(s1, gneg<kGroup>(s0));
    last = gadd<kGroup>(last, gneg<kGroup>(v));
    if (t1) last = gneg<kGroup>(last);
    put128(w0, last);
    put128(w1, last);
  }
  w0.flush();
  w1.flush();
}

// myl7 dcf_gen (third_party/myl7_fss/src/dcf.c:42-142) for kLtAlpha, one key
// pair per lane, written in the adapter layout (myl7_fss_backend.hpp:156-210).
template <int kGroup>
__global__ void __launch_bounds__(kDcfBlock) dcf_gen_kernel(DcfGenArgs a) {
  SUFHIP_DCF_LDS_SETUP(a.prg);
  const size_t stride = size_t(gridDim.x) * kDcfBlock;
  for (size_t e = size_t(blockIdx.x) * kDcfBlock + threadIdx.x; e < a.n; e += stride)
    gen_one<kGroup>(aes, rkl, a, e);
}

// K_0..K_3 expanded and laid out for AesLds2 (rounds 1..9 rotated).
void fill_prg4(const uint8_t* state, Prg4* p) {
  for (int j = 0; j < 4; ++j) {
    uint32_t rk[44];
    aes128_expand_words(state + 16 * j, rk);
    aes2_key_layout(rk, p->rk[j]);
  }
}

// Grid for the grid-stride DCF kernels: one workgroup per CU (LDS-limited),
// never more workgroups than the batch needs.
int dcf_grid(size_t n, unsigned int* grid) {
  int dev = 0, cus = 0;
  SUFHIP_CHECK(hipGetDevice(&dev), "hipGetDevice");
  SUFHIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev),
               "hipDeviceGetAttribute(CU count)");
  const size_t need = (n + kDcfBlock - 1) / kDcfBlock;
  *grid = static_cast<unsigned int>(need < size_t(cus) ? need : size_t(cus));
  return SUFHIP_OK;
}

constexpr size_t kMaxElems = size_t(1) << 38;

}  // namespace
}  // namespace sufhip

using namespace sufhip;

extern "C" {

size_t sufhip_dcf_key_bytes(int in_bits, int payload_len) {
  if (in_bits <= 0 || in_bits > 64 || payload_len <= 0) return 0;
  const size_t chunks = (size_t(payload_len) + 15) / 16;
  if (chunks > 255) return 0;
  return 8 + chunks * (32 + 33 * size_t(in_bits));
}

int sufhip_dcf_gen(int group, int in_bits, const uint8_t* prg_state, const uint64_t* d_alpha,
                   const uint8_t* d_payload, int payload_len, int payload_broadcast,
                   const uint8_t* d_seeds, size_t n, uint8_t* d_keys0, uint8_t* d_keys1,
                   void* stream) {
  SUFHIP_REQUIRE(group == SUFHIP_GROUP_XOR || group == SUFHIP_GROUP_ADD,
                 "sufhip_dcf_gen: unknown group");
  SUFHIP_REQUIRE(in_bits >= 1 && in_bits <= 64, "sufhip_dcf_gen: in_bits out of range");
  SUFHIP_REQUIRE(payload_len >= 1 && payload_len <= 255 * 16,
                 "sufhip_dcf_gen: payload_len out of range");
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(n < kMaxElems, "sufhip_dcf_gen: n too large");
  SUFHIP_REQUIRE(prg_state && d_alpha && d_payload && d_seeds && d_keys0 && d_keys1,
                 "sufhip_dcf_gen: null pointer");
  DcfGenArgs a{};
  fill_prg4(prg_state, &a.prg);
  a.alpha = d_alpha;
  a.payload = d_payload;
  a.seeds = d_seeds;
  a.keys0 = d_keys0;
  a.keys1 = d_keys1;
  a.key_bytes = sufhip_dcf_key_bytes(in_bits, payload_len);
  a.n = n;
  a.payload_bcast = payload_broadcast ? 1 : 0;
  a.payload_len = payload_len;
  a.in_bits = in_bits;
  a.chunks = (payload_len + 15) / 16;
  unsigned int g = 0;
  if (int rc = dcf_grid(n, &g)) return rc;
  if (group == SUFHIP_GROUP_XOR)
    hipLaunchKernelGGL((dcf_gen_kernel<SUFHIP_GROUP_XOR>), dim3(g), dim3(kDcfBlock), 0,
                       as_stream(stream), a);
  else
    hipLaunchKernelGGL((dcf_gen_kernel<SUFHIP_GROUP_ADD>), dim3(g), dim3(kDcfBlock), 0,
                       as_stream(stream), a);
  return check_launch("dcf_gen_kernel");
}

int sufhip_dcf_eval(int group, int in_bits, int payload_len, const uint8_t* prg_state,
                    const uint8_t* d_keys, size_t key_bytes, int key_broadcast,
                    const uint64_t* d_xs, size_t n, int out_mode, int out_bytes, void* d_out,
                    void* stream) {
  SUFHIP_REQUIRE(group == SUFHIP_GROUP_XOR || group == SUFHIP_GROUP_ADD,
                 "sufhip_dcf_eval: unknown group");
  SUFHIP_REQUIRE(in_bits >= 1 && in_bits <= 64, "sufhip_dcf_eval: in_bits out of range");
  SUFHIP_REQUIRE(payload_len >= 1 && payload_len <= 255 * 16,
                 "sufhip_dcf_eval: payload_len out of range");
  SUFHIP_REQUIRE(key_bytes == sufhip_dcf_key_bytes(in_bits, payload_len),
                 "sufhip_dcf_eval: key_bytes does not match (in_bits, payload_len)");
  SUFHIP_REQUIRE(out_mode == SUFHIP_DCF_OUT_BIT || out_mode == SUFHIP_DCF_OUT_BYTES ||
                     out_mode == SUFHIP_DCF_OUT_PACKED,
                 "sufhip_dcf_eval: unknown out_mode");
  if (out_mode == SUFHIP_DCF_OUT_BYTES)
    SUFHIP_REQUIRE(out_bytes >= 1 && out_bytes <= payload_len,
                   "sufhip_dcf_eval: out_bytes must be in [1, payload_len]");
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(n < kMaxElems, "sufhip_dcf_eval: n too large");
  SUFHIP_REQUIRE(prg_state && d_keys && d_xs && d_out, "sufhip_dcf_eval: null pointer");
  DcfEvalArgs a{};
  fill_prg4(prg_state, &a.prg);
  a.keys = d_keys;
  a.xs = d_xs;
  a.out = d_out;
  a.key_bytes = key_bytes;
  a.n = n;
  a.broadcast = key_broadcast ? 1 : 0;
  a.in_bits = in_bits;
  a.chunks = 1;
  a.out_bytes = out_mode == SUFHIP_DCF_OUT_BYTES ? out_bytes : 1;
  unsigned int g = 0;
  if (int rc = dcf_grid(n, &g)) return rc;
  const dim3 grid(g), block(kDcfBlock);
  hipStream_t s = as_stream(stream);
  if (out_mode == SUFHIP_DCF_OUT_BIT) {
    hipLaunchKernelGGL((dcf_eval_bit_kernel<SUFHIP_DCF_OUT_BIT>), grid, block, 0, s, a);
  } else if (out_mode == SUFHIP_DCF_OUT_PACKED) {
    SUFHIP_REQUIRE((reinterpret_cast<uintptr_t>(d_out) & 7) == 0,
                   "sufhip_dcf_eval: packed output must be 8-byte aligned");
    hipLaunchKernelGGL((dcf_eval_bit_kernel<SUFHIP_DCF_OUT_PACKED>), grid, block, 0, s, a);
  } else {
    a.chunks = (out_bytes + 15) / 16;
    if (group == SUFHIP_GROUP_XOR)
      hipLaunchKernelGGL((dcf_eval_bytes_kernel<SUFHIP_GROUP_XOR>), grid, block, 0, s, a);
    else
      hipLaunchKernelGGL((dcf_eval_bytes_kernel<SUFHIP_GROUP_ADD>), grid, block, 0, s, a);
  }
  return check_launch("dcf_eval kernel");
}

}  // extern "C"
