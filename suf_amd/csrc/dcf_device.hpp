// Device building blocks of the myl7/fss v0.7.1 DCF shared by the batch
// kernels (dcf.hip) and the truncation gate (trunc_gate.hip): AES tables,
// correction-word loaders, the tree walks and the per-lane key writer.
#pragma once

#include <hip/hip_runtime.h>

#include "aes_lds.hpp"
#include "sufhip_internal.hpp"

namespace sufhip {
namespace {


// One workgroup per CU: the four replicated AES tables take 128 KB of the
// CU's 160 KB LDS.  Kernels loop over the batch in grid strides.
#ifndef SUFHIP_DCF_BLOCK
#define SUFHIP_DCF_BLOCK 512
#endif
constexpr int kDcfBlock = SUFHIP_DCF_BLOCK;

// AES tables for every DCF kernel: four rotated T tables, 32 copies each.
using DcfAes = AesLds4;

struct Prg4 {
  uint32_t rk[4][44];  // K_0..K_3: DCF uses PRG output blocks 0..3
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

struct CwFull {
  uint32_t s[4];
  uint32_t v[4];
  uint32_t tb;
};


// Reads 16 bytes at p.  When p + 16 is the end of the key (`more` false) and
// p is not 4-byte aligned, the last sh bytes come from byte loads so that no
// word past the key is touched.
__device__ __forceinline__ void load16_bytes(const uint8_t* p, bool more, uint32_t (&w)[4]) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t* q = reinterpret_cast<const uint32_t*>(a & ~uintptr_t(3));
  const uint32_t sh = uint32_t(a & 3);
  uint32_t r0 = q[0], r1 = q[1], r2 = q[2], r3 = q[3];
  uint32_t r4 = 0;
  if (sh != 0) {
    if (more) {
      r4 = q[4];
    } else {
      const uint8_t* tail = reinterpret_cast<const uint8_t*>(q + 4);
      for (uint32_t k = 0; k < sh; ++k) r4 |= uint32_t(tail[k]) << (8 * k);
    }
  }
  w[0] = __builtin_amdgcn_alignbyte(r1, r0, sh);
  w[1] = __builtin_amdgcn_alignbyte(r2, r1, sh);
  w[2] = __builtin_amdgcn_alignbyte(r3, r2, sh);
  w[3] = __builtin_amdgcn_alignbyte(r4, r3, sh);
}

// ---------------------------------------------------------------------------
// Bit-mode walk (share byte 0 & 1) with the round keys in scalar registers.
//
// At level i every lane needs K_{2 x_i} (next seed) and K_{2 x_i + 1} (value
// block), x_i being its own input bit.  With m = -x_i (all ones or zero) they
// are K_0 ^ (m & (K_0 ^ K_2)) and K_1 ^ (m & (K_1 ^ K_3)): the four uniform
// words of each pair come from the kernel argument through the scalar unit,
// and the per-lane choice is one 3-input bit operation per key word.  Reading
// the chosen keys from LDS instead costs 20 ds_read_b128 per level (about 4
// LDS clocks each) on the pipe that bounds the walk, and 80 VGPRs.
//
// DcfKeySel row r: K_0[r], (K_0 ^ K_2)[r], K_1[r], (K_1 ^ K_3)[r].
struct DcfKeySel {
  uint32_t w[11][16];
};

void fill_key_sel(const Prg4& p, DcfKeySel* k) {
  for (int r = 0; r < 11; ++r)
    for (int j = 0; j < 4; ++j) {
      k->w[r][j] = p.rk[0][4 * r + j];
      k->w[r][4 + j] = p.rk[0][4 * r + j] ^ p.rk[2][4 * r + j];
      k->w[r][8 + j] = p.rk[1][4 * r + j];
      k->w[r][12 + j] = p.rk[1][4 * r + j] ^ p.rk[3][4 * r + j];
    }
}

// A DcfKeySel inside the kernel's by-value argument, addressed through the
// constant (kernel-argument) address space so that its loads are scalar.
typedef const __attribute__((address_space(4))) uint32_t* KeySelPtr;

__device__ __forceinline__ KeySelPtr kernarg_key_sel(size_t field) {
  return (KeySelPtr)((const __attribute__((address_space(4))) uint8_t*)
                         __builtin_amdgcn_kernarg_segment_ptr() + field);
}

#define SUFHIP_BITOP3(a, b, c, f) __builtin_amdgcn_bitop3_b32((a), (b), (c), (f))
// x ^ (m & d) as one v_bitop3 (truth table over src0 = 0xf0, src1 = 0xcc,
// src2 = 0xaa).
__device__ __forceinline__ uint32_t xor_and(uint32_t x, uint32_t m, uint32_t d) {
  return SUFHIP_BITOP3(x, m, d, 0x78);
}

__device__ __forceinline__ uint32_t lds_word(const uint32_t* lds, uint32_t byte_addr) {
  return *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(lds) + byte_addr);
}

// One middle round of the seed block A and of columns [0, kB) of the value
// block B, in three groups: every table address, then every table read with
// the round's key loads, then the combines.  The scheduling barriers keep the
// compiler from interleaving reads with their uses (each read's latency
// would then be paid in turn).
template <int kB>
__device__ __forceinline__ void key_sel_round(const AesLds4& aes, KeySelPtr q, uint32_t m,
                                              uint32_t (&A)[4], uint32_t (&B)[4]) {
  constexpr int kN = 16 + 4 * kB;
  uint32_t ad[kN];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ad[4 * c + j] = __builtin_amdgcn_perm(A[(c + j) & 3], aes.base[j], AesLds4::sel(j));
      if (c < kB)
        ad[16 + 4 * c + j] = __builtin_amdgcn_perm(B[(c + j) & 3], aes.base[j], AesLds4::sel(j));
    }
  __builtin_amdgcn_sched_barrier(0);
  uint32_t tv[kN];
#pragma unroll
  for (int n = 0; n < kN; ++n) tv[n] = lds_word(aes.lds, ad[n]);
  uint32_t kq[16];
#pragma unroll
  for (int n = 0; n < 8; ++n) kq[n] = q[n];
#pragma unroll
  for (int c = 0; c < kB; ++c) {
    kq[8 + c] = q[8 + c];
    kq[12 + c] = q[12 + c];
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int c = 0; c < 4; ++c)
    A[c] = xor_and(SUFHIP_BITOP3(SUFHIP_BITOP3(tv[4 * c], tv[4 * c + 1], tv[4 * c + 2], 0x96),
                                 tv[4 * c + 3], kq[c], 0x96),
                   m, kq[4 + c]);
#pragma unroll
  for (int c = 0; c < kB; ++c)
    B[c] = xor_and(SUFHIP_BITOP3(SUFHIP_BITOP3(tv[16 + 4 * c], tv[17 + 4 * c], tv[18 + 4 * c], 0x96),
                                 tv[19 + 4 * c], kq[8 + c], 0x96),
                   m, kq[12 + c]);
}

// The aligned words of a 33-byte correction-word record that hold s_cw,
// byte 0 of v_cw and the t byte (words 0..4 and 8), read with global loads:
// a flat load also counts on the LDS wait counter, so every LDS wait of the
// level would wait for it too.
struct CwRaw {
  uint32_t r[6];
  uint32_t sh;
};

typedef const __attribute__((address_space(1))) uint32_t* GlobalWords;

__device__ __forceinline__ CwRaw load_cw_raw(const uint8_t* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  GlobalWords q = (GlobalWords)(a & ~uintptr_t(3));
  CwRaw c;
  c.r[0] = q[0];
  c.r[1] = q[1];
  c.r[2] = q[2];
  c.r[3] = q[3];
  c.r[4] = q[4];
  c.r[5] = q[8];
  c.sh = uint32_t(a & 3);
  return c;
}

__device__ __forceinline__ CwBit decode_cw(const CwRaw& w) {
  CwBit c;
  c.s[0] = __builtin_amdgcn_alignbyte(w.r[1], w.r[0], w.sh);
  c.s[1] = __builtin_amdgcn_alignbyte(w.r[2], w.r[1], w.sh);
  c.s[2] = __builtin_amdgcn_alignbyte(w.r[3], w.r[2], w.sh);
  c.s[3] = __builtin_amdgcn_alignbyte(w.r[4], w.r[3], w.sh);
  c.v0 = (w.r[4] >> (8 * w.sh)) & 0xffu;
  c.tb = (w.r[5] >> (8 * w.sh)) & 0xffu;
  return c;
}

// Bit-mode walk of one chunk: returns share byte 0 & 1.  The seed block is
// AES_{K_{2 x_i}}(s) ^ s in full; of the value block only byte 0 is formed
// (round 9 column 0, then one final S-box byte).
__device__ __forceinline__ uint32_t walk_bit(const AesLds4& aes, KeySelPtr keys,
                                             const uint8_t* chunk, int in_bits, uint64_t x,
                                             uint32_t party) {
  uint32_t seed[4];
  load16_bytes(chunk, true, seed);
  uint32_t s[4] = {seed[0], seed[1], seed[2], seed[3] & 0x7fffffffu};
  uint32_t t = party;
  uint32_t v = 0;
  const uint8_t* cw = chunk + 16;
  for (int i = 0; i < in_bits; ++i, cw += 33) {
    const uint32_t xi = uint32_t(x >> (in_bits - 1 - i)) & 1u;
    const uint32_t m = 0u - xi;
    const CwRaw cr = load_cw_raw(cw);
    // An opaque copy of the key pointer per level: the compiler would
    // otherwise hoist all 176 key words out of the level loop into scalar
    // registers it does not have.
    KeySelPtr k = keys;
    asm volatile("" : "+s"(k));
    uint32_t A[4], B[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      A[j] = xor_and(s[j], m, k[4 + j]) ^ k[j];
      B[j] = xor_and(s[j], m, k[12 + j]) ^ k[8 + j];
    }
#pragma unroll
    for (int r = 1; r < 9; ++r) key_sel_round<4>(aes, k + 16 * r, m, A, B);
    key_sel_round<1>(aes, k + 16 * 9, m, A, B);
    // Final round of the seed block: S(x) is byte 0 of T3[x], bytes 1 and 2
    // of T0[x] and byte 3 of T1[x]; byte 0 of the value block from T3.
    uint32_t ad[17];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      ad[4 * c + 0] = __builtin_amdgcn_perm(A[c], aes.base[3], AesLds4::sel(0));
      ad[4 * c + 1] = __builtin_amdgcn_perm(A[(c + 1) & 3], aes.base[0], AesLds4::sel(1));
      ad[4 * c + 2] = __builtin_amdgcn_perm(A[(c + 2) & 3], aes.base[0], AesLds4::sel(2));
      ad[4 * c + 3] = __builtin_amdgcn_perm(A[(c + 3) & 3], aes.base[1], AesLds4::sel(3));
    }
    ad[16] = __builtin_amdgcn_perm(B[0], aes.base[3], AesLds4::sel(0));
    __builtin_amdgcn_sched_barrier(0);
    uint32_t tv[17];
#pragma unroll
    for (int n = 0; n < 17; ++n) tv[n] = lds_word(aes.lds, ad[n]);
    const KeySelPtr q = k + 160;
    uint32_t kq[10];
#pragma unroll
    for (int n = 0; n < 8; ++n) kq[n] = q[n];
    kq[8] = q[8];
    kq[9] = q[12];
    __builtin_amdgcn_sched_barrier(0);
    uint32_t o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t lo = __builtin_amdgcn_perm(tv[4 * c + 1], tv[4 * c], 0x0c0c0500u);
      const uint32_t hi = __builtin_amdgcn_perm(tv[4 * c + 3], tv[4 * c + 2], 0x07020c0cu);
      // ((lo | hi) ^ s) ^ K_sel: the Matyas-Meyer-Oseas output of the seed block.
      o[c] = xor_and(SUFHIP_BITOP3(lo, hi, s[c], 0x56) ^ kq[c], m, kq[4 + c]);
    }
    const uint32_t vb = xor_and(tv[16] ^ s[0] ^ kq[8], m, kq[9]) & 1u;
    const CwBit c = decode_cw(cr);
    uint32_t tn = o[3] >> 31;
    o[3] &= 0x7fffffffu;
    const uint32_t tmask = 0u - t;
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = o[j] ^ (c.s[j] & tmask);
    tn ^= ((xi ? c.tb : (c.tb >> 1)) & 1u) & t;
    v ^= vb ^ (c.v0 & t & 1u);
    t = tn;
  }
  uint32_t np1[4];
  load16_bytes(cw, false, np1);
  return (v ^ s[0] ^ (np1[0] & t)) & 1u;
}

// The aligned words 0..8 around a 33-byte correction-word record (s_cw,
// v_cw, the t byte), read with global loads at the start of a level and
// decoded after its AES (as CwRaw for the bit walk).
struct CwRawFull {
  uint32_t r[9];
  uint32_t sh;
};

__device__ __forceinline__ CwRawFull load_cw_raw_full(const uint8_t* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  GlobalWords q = (GlobalWords)(a & ~uintptr_t(3));
  CwRawFull c;
#pragma unroll
  for (int j = 0; j < 9; ++j) c.r[j] = q[j];
  c.sh = uint32_t(a & 3);
  return c;
}

__device__ __forceinline__ CwFull decode_cw_full(const CwRawFull& w) {
  CwFull c;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    c.s[j] = __builtin_amdgcn_alignbyte(w.r[j + 1], w.r[j], w.sh);
    c.v[j] = __builtin_amdgcn_alignbyte(w.r[j + 5], w.r[j + 4], w.sh);
  }
  c.tb = (w.r[8] >> (8 * w.sh)) & 0xffu;
  return c;
}

// Full-block walk of one chunk (any group): returns the 16-byte share.  The
// same scheme as walk_bit -- round keys chosen per lane from scalar
// registers, grouped rounds -- with both blocks computed in full.
template <int kGroup>
__device__ __forceinline__ U128 walk_full(const AesLds4& aes, KeySelPtr keys, const uint8_t* chunk,
                                          int in_bits, uint64_t x, uint32_t party,
                                          bool more_after) {
  uint32_t seed[4];
  load16_bytes(chunk, true, seed);
  uint32_t s[4] = {seed[0], seed[1], seed[2], seed[3] & 0x7fffffffu};
  uint32_t t = party;
  U128 v{0, 0};
  const uint8_t* cw = chunk + 16;
  for (int i = 0; i < in_bits; ++i, cw += 33) {
    const uint32_t xi = uint32_t(x >> (in_bits - 1 - i)) & 1u;
    const uint32_t m = 0u - xi;
    const CwRawFull cr = load_cw_raw_full(cw);
    KeySelPtr k = keys;
    asm volatile("" : "+s"(k));
    uint32_t A[4], B[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      A[j] = xor_and(s[j], m, k[4 + j]) ^ k[j];
      B[j] = xor_and(s[j], m, k[12 + j]) ^ k[8 + j];
    }
#pragma unroll
    for (int r = 1; r < 10; ++r) key_sel_round<4>(aes, k + 16 * r, m, A, B);
    // Final round of both blocks: S(x) is byte 0 of T3[x], bytes 1 and 2 of
    // T0[x] and byte 3 of T1[x].
    uint32_t ad[32];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      ad[4 * c + 0] = __builtin_amdgcn_perm(A[c], aes.base[3], AesLds4::sel(0));
      ad[4 * c + 1] = __builtin_amdgcn_perm(A[(c + 1) & 3], aes.base[0], AesLds4::sel(1));
      ad[4 * c + 2] = __builtin_amdgcn_perm(A[(c + 2) & 3], aes.base[0], AesLds4::sel(2));
      ad[4 * c + 3] = __builtin_amdgcn_perm(A[(c + 3) & 3], aes.base[1], AesLds4::sel(3));
      ad[16 + 4 * c + 0] = __builtin_amdgcn_perm(B[c], aes.base[3], AesLds4::sel(0));
      ad[16 + 4 * c + 1] = __builtin_amdgcn_perm(B[(c + 1) & 3], aes.base[0], AesLds4::sel(1));
      ad[16 + 4 * c + 2] = __builtin_amdgcn_perm(B[(c + 2) & 3], aes.base[0], AesLds4::sel(2));
      ad[16 + 4 * c + 3] = __builtin_amdgcn_perm(B[(c + 3) & 3], aes.base[1], AesLds4::sel(3));
    }
    __builtin_amdgcn_sched_barrier(0);
    uint32_t tv[32];
#pragma unroll
    for (int n = 0; n < 32; ++n) tv[n] = lds_word(aes.lds, ad[n]);
    const KeySelPtr q = k + 160;
    uint32_t kq[16];
#pragma unroll
    for (int n = 0; n < 16; ++n) kq[n] = q[n];
    __builtin_amdgcn_sched_barrier(0);
    uint32_t o[4], ob[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t lo = __builtin_amdgcn_perm(tv[4 * c + 1], tv[4 * c], 0x0c0c0500u);
      const uint32_t hi = __builtin_amdgcn_perm(tv[4 * c + 3], tv[4 * c + 2], 0x07020c0cu);
      o[c] = xor_and(SUFHIP_BITOP3(lo, hi, s[c], 0x56) ^ kq[c], m, kq[4 + c]);
      const uint32_t lb = __builtin_amdgcn_perm(tv[16 + 4 * c + 1], tv[16 + 4 * c], 0x0c0c0500u);
      const uint32_t hb = __builtin_amdgcn_perm(tv[16 + 4 * c + 3], tv[16 + 4 * c + 2], 0x07020c0cu);
      ob[c] = xor_and(SUFHIP_BITOP3(lb, hb, s[c], 0x56) ^ kq[8 + c], m, kq[12 + c]);
    }
    const CwFull c = decode_cw_full(cr);
    U128 vd = mk(ob[0], ob[1], ob[2], ob[3] & 0x7fffffffu);
    uint32_t tn = o[3] >> 31;
    o[3] &= 0x7fffffffu;
    if (t) {
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] ^= c.s[j];
      tn ^= (xi ? c.tb : (c.tb >> 1)) & 1u;
      vd = gadd<kGroup>(vd, mk(c.v[0], c.v[1], c.v[2], c.v[3]));
    }
    if (party) vd = gneg<kGroup>(vd);
    v = gadd<kGroup>(v, vd);
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = o[j];
    t = tn;
  }
  uint32_t np1[4];
  load16_bytes(cw, more_after, np1);
  U128 sv = mk(s[0], s[1], s[2], s[3]);
  if (t) sv = gadd<kGroup>(sv, mk(np1[0], np1[1], np1[2], np1[3]));
  if (party) sv = gneg<kGroup>(sv);
  return gadd<kGroup>(v, sv);
}

// Additive-group walk that keeps only the low 64 bits of the 16-byte
// value: + mod 2^127 and negation never carry from bit 63 upward into the
// low word, so the low 8 bytes of the share are exact.  Used for DCF keys
// with an 8-byte payload (SUF's AddU64 predicates).
struct Add64State {
  uint32_t s0, s1, s2, s3;  // seed, MSB cleared
  uint32_t t;
  uint64_t v;  // accumulated value, low 64 bits
};

// Correction word fields for the low-64 walk: s_cw, v_cw bytes 0..7, t byte.
struct CwAdd64 {
  uint32_t s[4];
  uint64_t v;
  uint32_t tb;
};

__device__ __forceinline__ CwAdd64 load_cw_add64(const uint8_t* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t* q = reinterpret_cast<const uint32_t*>(a & ~uintptr_t(3));
  const uint32_t sh = uint32_t(a & 3);
  // Words 0..6 and 8 of the aligned window: bytes [0, 24) and byte 32 of
  // the 33-byte record (word 8 may reach into the next record or cw_np1,
  // both inside the key).
  const uint32_t r0 = q[0], r1 = q[1], r2 = q[2], r3 = q[3], r4 = q[4], r5 = q[5], r6 = q[6],
                 r8 = q[8];
  CwAdd64 c;
  c.s[0] = __builtin_amdgcn_alignbyte(r1, r0, sh);
  c.s[1] = __builtin_amdgcn_alignbyte(r2, r1, sh);
  c.s[2] = __builtin_amdgcn_alignbyte(r3, r2, sh);
  c.s[3] = __builtin_amdgcn_alignbyte(r4, r3, sh);
  c.v = uint64_t(__builtin_amdgcn_alignbyte(r5, r4, sh)) |
        uint64_t(__builtin_amdgcn_alignbyte(r6, r5, sh)) << 32;
  c.tb = (r8 >> (8 * sh)) & 0xffu;
  return c;
}

// State at the root of one chunk (chunk = key + 8: seed, CWs, cw_np1).
__device__ __forceinline__ Add64State add64_root(const uint8_t* chunk, uint32_t party) {
  uint32_t seed[4];
  load16_bytes(chunk, true, seed);
  return Add64State{seed[0], seed[1], seed[2], seed[3] & 0x7fffffffu, party, 0};
}

// Levels [from, to) of an in_bits-level walk at x (only bits in_bits-1-i used).
__device__ __forceinline__ void add64_walk(const DcfAes& aes, const uint4* rkl,
                                           const uint8_t* chunk, int in_bits, int from, int to,
                                           uint64_t x, uint32_t party, Add64State& st) {
  const uint8_t* cw = chunk + 16 + 33 * from;
  for (int i = from; i < to; ++i, cw += 33) {
    const uint32_t xi = uint32_t(x >> (in_bits - 1 - i)) & 1u;
    const CwAdd64 c = load_cw_add64(cw);
    const uint4* ks = rkl + 22 * xi;
    const uint4* kv = ks + 11;
    uint32_t a0 = st.s0, a1 = st.s1, a2 = st.s2, a3 = st.s3;
    uint32_t b0, b1;
    aes.encrypt(a0, a1, a2, a3, ks);
    aes.encrypt_lo2(st.s0, st.s1, st.s2, st.s3, kv, b0, b1);
    uint64_t vd = uint64_t(b0 ^ st.s0) | uint64_t(b1 ^ st.s1) << 32;
    a0 ^= st.s0;
    a1 ^= st.s1;
    a2 ^= st.s2;
    a3 ^= st.s3;
    uint32_t tn = a3 >> 31;
    a3 &= 0x7fffffffu;
    if (st.t) {
      a0 ^= c.s[0];
      a1 ^= c.s[1];
      a2 ^= c.s[2];
      a3 ^= c.s[3];
      tn ^= (xi ? c.tb : (c.tb >> 1)) & 1u;
      vd += c.v;
    }
    st.v += party ? 0 - vd : vd;
    st.s0 = a0;
    st.s1 = a1;
    st.s2 = a2;
    st.s3 = a3;
    st.t = tn;
  }
}

// Share after the last level: v + (-1)^party (s + t * cw_np1), low 64 bits.
__device__ __forceinline__ uint64_t add64_finish(const uint8_t* chunk, int in_bits,
                                                 uint32_t party, const Add64State& st) {
  uint32_t np1[4];
  load16_bytes(chunk + 16 + 33 * in_bits, false, np1);
  uint64_t s = uint64_t(st.s0) | uint64_t(st.s1) << 32;
  if (st.t) s += uint64_t(np1[0]) | uint64_t(np1[1]) << 32;
  return st.v + (party ? 0 - s : s);
}

// Stages the replicated tables in LDS (the bit-mode walk's setup).
#define SUFHIP_DCF_TABLE_SETUP()                                   \
  __shared__ __align__(16) uint32_t tabs[DcfAes::kWords];          \
  __shared__ uint32_t tstage[256];                                 \
  DcfAes::fill(tabs, tstage, kTDev.v);                             \
  __syncthreads();                                                 \
  const DcfAes aes = DcfAes::make(tabs)

// Stages the replicated tables and the K_0..K_3 round keys in LDS.
#define SUFHIP_DCF_LDS_SETUP(PRG)                                  \
  __shared__ __align__(16) uint32_t tabs[DcfAes::kWords];          \
  __shared__ uint32_t tstage[256];                                 \
  __shared__ uint4 rkl[4 * 11];                                    \
  DcfAes::fill(tabs, tstage, kTDev.v);                             \
  fill_round_keys(rkl, (PRG).rk, 4);                               \
  __syncthreads();                                                 \
  const DcfAes aes = DcfAes::make(tabs)

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

__device__ __forceinline__ void prg4(const DcfAes& aes, const uint4* rkl, const U128& s,
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

// One DCF key pair for f(x) = beta * 1[x < alpha] (myl7 dcf_gen,
// third_party/myl7_fss/src/dcf.c:42-142), written in the adapter layout
// (include/proto/myl7_fss_backend.hpp:156-210).  seeds: [chunks][32]
// (party-0 seed, party-1 seed).
template <int kGroup>
__device__ __forceinline__ void gen_key(const DcfAes& aes, const uint4* rkl, int nb, int chunks,
                                        int payload_len, uint64_t alpha, const uint8_t* pay,
                                        const uint8_t* seeds, uint8_t* out0, uint8_t* out1) {
  if (nb < 64) alpha &= (uint64_t(1) << nb) - 1;
  ByteWriter w0{out0, 0, 0};
  ByteWriter w1{out1, 0, 0};
  const uint32_t plen = uint32_t(payload_len);
  w0.put32(uint32_t(nb) | uint32_t(chunks) << 8 | 0u << 16);
  w1.put32(uint32_t(nb) | uint32_t(chunks) << 8 | 1u << 16);
  w0.put32(plen);
  w1.put32(plen);
  for (int c = 0; c < chunks; ++c) {
    uint8_t beta_b[16];
    for (int b = 0; b < 16; ++b) {
      const int idx = 16 * c + b;
      beta_b[b] = idx < payload_len ? pay[idx] : 0;
    }
    U128 beta{0, 0};
    for (int b = 0; b < 8; ++b) beta.lo |= uint64_t(beta_b[b]) << (8 * b);
    for (int b = 0; b < 8; ++b) beta.hi |= uint64_t(beta_b[8 + b]) << (8 * b);
    beta.hi &= kMsbClear;
    const uint8_t* sp = seeds + size_t(c) * 32;
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

// K_0..K_3 expanded (FIPS-197 word order).
void fill_prg4(const uint8_t* state, Prg4* p) {
  for (int j = 0; j < 4; ++j) {
    aes128_expand_words(state + 16 * j, p->rk[j]);
  }
}

// Grid for the grid-stride DCF kernels: one workgroup per CU (LDS-limited),
// never more workgroups than the batch needs.
int dcf_grid(size_t n, unsigned int* grid, int block = kDcfBlock) {
  int dev = 0, cus = 0;
  SUFHIP_CHECK(hipGetDevice(&dev), "hipGetDevice");
  SUFHIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev),
               "hipDeviceGetAttribute(CU count)");
  const size_t need = (n + size_t(block) - 1) / size_t(block);
  *grid = static_cast<unsigned int>(need < size_t(cus) ? need : size_t(cus));
  return SUFHIP_OK;
}

}  // namespace
}  // namespace sufhip
