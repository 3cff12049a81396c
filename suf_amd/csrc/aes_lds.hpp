// AES-128 encryption for CDNA4 with the round table resident in LDS.
//
// State words are little-endian 32-bit columns (word c = bytes 4c..4c+3 of
// the block), so blocks, keys and round keys load straight from memory.  One
// 1 KB table T(x) = {2s, s, s, 3s} (s = SubBytes(x), bytes in row order) is
// enough: the other three columns of the classic four-table form are byte
// rotations of it, and the final round's S-box bytes are read out of T.
//
// Bank conflicts: a wave's 64 lookups per step use data-dependent indices.
// The table is replicated kCopies times in LDS, copy c holding entry e at
// word e * kCopies + c, and lane l always reads copy l % kCopies, so lanes
// with distinct (l % kCopies) never share a bank whatever the indices are.
// The S-box itself is derived at compile time from its FIPS-197 definition
// (inverse in GF(2^8) then the affine map with 0x63).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sufhip {

struct SboxTable {
  uint8_t v[256];
};

constexpr uint8_t gf_mul_c(uint8_t a, uint8_t b) {
  uint8_t r = 0;
  for (int i = 0; i < 8; ++i) {
    if (b & 1) r = static_cast<uint8_t>(r ^ a);
    a = static_cast<uint8_t>((a << 1) ^ ((a & 0x80) ? 0x1b : 0));
    b = static_cast<uint8_t>(b >> 1);
  }
  return r;
}

constexpr SboxTable make_sbox() {
  SboxTable t{};
  for (int x = 0; x < 256; ++x) {
    uint8_t inv = 0;
    if (x != 0) {
      // x^254 = x^-1
      uint8_t r = 1, base = static_cast<uint8_t>(x);
      int e = 254;
      while (e) {
        if (e & 1) r = gf_mul_c(r, base);
        base = gf_mul_c(base, base);
        e >>= 1;
      }
      inv = r;
    }
    uint8_t s = 0x63;
    for (int i = 0; i < 8; ++i) {
      int bit = ((inv >> i) ^ (inv >> ((i + 4) & 7)) ^ (inv >> ((i + 5) & 7)) ^
                 (inv >> ((i + 6) & 7)) ^ (inv >> ((i + 7) & 7))) & 1;
      s = static_cast<uint8_t>(s ^ (bit << i));
    }
    t.v[x] = s;
  }
  return t;
}

struct TTable {
  uint32_t v[256];
};

constexpr TTable make_ttable() {
  TTable t{};
  SboxTable s = make_sbox();
  for (int x = 0; x < 256; ++x) {
    uint32_t v = s.v[x];
    uint32_t v2 = gf_mul_c(static_cast<uint8_t>(v), 2);
    uint32_t v3 = v2 ^ v;
    t.v[x] = v2 | (v << 8) | (v << 16) | (v3 << 24);
  }
  return t;
}

inline constexpr SboxTable kSboxHost = make_sbox();
inline constexpr TTable kTHost = make_ttable();

// Per-translation-unit device copy of T (no relocatable device code).
static __device__ const TTable kTDev = make_ttable();

// Round keys of one AES-128 key as 44 little-endian words (kernel argument).
struct RoundKeys {
  uint32_t w[44];
};

// The myl7 PRG keys K_0..K_7 (prg_init, third_party/myl7_fss/src/prg/
// aes128_mmo.c:16-31 with kBlocks = 8), expanded; passed by value.
constexpr int kPrgMaxBlocks = 8;
struct PrgKeys {
  uint32_t rk[kPrgMaxBlocks][44];
};

// Host-side key expansion (FIPS-197 5.2) producing 44 little-endian words.
inline void aes128_expand_words(const uint8_t key[16], uint32_t rk[44]) {
  uint8_t b[176];
  for (int i = 0; i < 16; ++i) b[i] = key[i];
  uint8_t rcon = 1;
  for (int w = 4; w < 44; ++w) {
    uint8_t t0 = b[4 * (w - 1)], t1 = b[4 * (w - 1) + 1], t2 = b[4 * (w - 1) + 2],
            t3 = b[4 * (w - 1) + 3];
    if (w % 4 == 0) {
      uint8_t r0 = t0;
      t0 = static_cast<uint8_t>(kSboxHost.v[t1] ^ rcon);
      t1 = kSboxHost.v[t2];
      t2 = kSboxHost.v[t3];
      t3 = kSboxHost.v[r0];
      rcon = gf_mul_c(rcon, 2);
    }
    b[4 * w] = static_cast<uint8_t>(b[4 * (w - 4)] ^ t0);
    b[4 * w + 1] = static_cast<uint8_t>(b[4 * (w - 4) + 1] ^ t1);
    b[4 * w + 2] = static_cast<uint8_t>(b[4 * (w - 4) + 2] ^ t2);
    b[4 * w + 3] = static_cast<uint8_t>(b[4 * (w - 4) + 3] ^ t3);
  }
  for (int w = 0; w < 44; ++w)
    rk[w] = uint32_t(b[4 * w]) | uint32_t(b[4 * w + 1]) << 8 | uint32_t(b[4 * w + 2]) << 16 |
            uint32_t(b[4 * w + 3]) << 24;
}

inline void expand_prg_keys(const uint8_t* state, int blocks, PrgKeys* k) {
  for (int j = 0; j < kPrgMaxBlocks; ++j)
    for (int w = 0; w < 44; ++w) k->rk[j][w] = 0;
  for (int j = 0; j < blocks && j < kPrgMaxBlocks; ++j) aes128_expand_words(state + 16 * j, k->rk[j]);
}

__device__ __forceinline__ uint32_t rotl32(uint32_t x, int r) {
  return __builtin_amdgcn_alignbit(x, x, 32 - r);
}

// Value of lane (q + k) % 4 of this lane's quad (q = lane & 3; DPP quad
// permute, every lane of the quad active).
template <int k>
__device__ __forceinline__ uint32_t quad_rot(uint32_t v) {
  constexpr int ctrl = ((0 + k) & 3) | ((1 + k) & 3) << 2 | ((2 + k) & 3) << 4 | ((3 + k) & 3) << 6;
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), ctrl, 0xf, 0xf, false));
}

// Value of lane c of this lane's quad, in every lane of the quad.
template <int c>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
  constexpr int ctrl = c | c << 2 | c << 4 | c << 6;
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), ctrl, 0xf, 0xf, false));
}

// LDS-resident T table, kCopies-way replicated.  `lane_word` is this lane's
// copy index (lane % kCopies).
template <int kCopies>
struct AesLds {
  static constexpr int kWords = 256 * kCopies;
  const uint32_t* tab;  // LDS
  uint32_t lane_word;

  __device__ __forceinline__ uint32_t T(uint32_t byte) const {
    return tab[byte * kCopies + lane_word];
  }
  __device__ __forceinline__ uint32_t b0(uint32_t w) const { return T(w & 0xffu); }
  __device__ __forceinline__ uint32_t b1(uint32_t w) const { return T((w >> 8) & 0xffu); }
  __device__ __forceinline__ uint32_t b2(uint32_t w) const { return T((w >> 16) & 0xffu); }
  __device__ __forceinline__ uint32_t b3(uint32_t w) const { return T(w >> 24); }

  // One full middle round: SubBytes, ShiftRows, MixColumns, AddRoundKey.
  __device__ __forceinline__ void round(uint32_t& s0, uint32_t& s1, uint32_t& s2, uint32_t& s3,
                                        uint32_t k0, uint32_t k1, uint32_t k2,
                                        uint32_t k3) const {
    uint32_t t0 = b0(s0) ^ rotl32(b1(s1), 8) ^ rotl32(b2(s2), 16) ^ rotl32(b3(s3), 24) ^ k0;
    uint32_t t1 = b0(s1) ^ rotl32(b1(s2), 8) ^ rotl32(b2(s3), 16) ^ rotl32(b3(s0), 24) ^ k1;
    uint32_t t2 = b0(s2) ^ rotl32(b1(s3), 8) ^ rotl32(b2(s0), 16) ^ rotl32(b3(s1), 24) ^ k2;
    uint32_t t3 = b0(s3) ^ rotl32(b1(s0), 8) ^ rotl32(b2(s1), 16) ^ rotl32(b3(s2), 24) ^ k3;
    s0 = t0;
    s1 = t1;
    s2 = t2;
    s3 = t3;
  }

  // Final-round column c from state words (a = s_c, b = s_{c+1}, ...).
  __device__ __forceinline__ uint32_t last_col(uint32_t a, uint32_t b, uint32_t c,
                                               uint32_t d) const {
    return ((b0(a) >> 8) & 0xffu) | (b1(b) & 0xff00u) | (b2(c) & 0xff0000u) |
           ((b3(d) << 8) & 0xff000000u);
  }

  // Full AES-128 encryption of (s0..s3); rk points at the 11 round keys
  // (uint4 per round, usually in LDS).  The nine middle rounds stay a loop:
  // the kernels that use this table inline it at many sites, and unrolled
  // copies (~5 KB each) overflow the instruction cache of a latency-bound
  // kernel, while the loop costs three scalar instructions per round.
  __device__ __forceinline__ void encrypt(uint32_t& s0, uint32_t& s1, uint32_t& s2, uint32_t& s3,
                                          const uint4* rk) const {
    uint4 k = rk[0];
    s0 ^= k.x;
    s1 ^= k.y;
    s2 ^= k.z;
    s3 ^= k.w;
#pragma unroll 1
    for (int r = 1; r < 10; ++r) {
      k = rk[r];
      round(s0, s1, s2, s3, k.x, k.y, k.z, k.w);
    }
    k = rk[10];
    uint32_t o0 = last_col(s0, s1, s2, s3) ^ k.x;
    uint32_t o1 = last_col(s1, s2, s3, s0) ^ k.y;
    uint32_t o2 = last_col(s2, s3, s0, s1) ^ k.z;
    uint32_t o3 = last_col(s3, s0, s1, s2) ^ k.w;
    s0 = o0;
    s1 = o1;
    s2 = o2;
    s3 = o3;
  }

  // encrypt() with all rounds unrolled, for round keys held in registers (a
  // per-element key read from HBM): a runtime round index into a register
  // array would put the keys in private scratch memory.
  __device__ __forceinline__ void encrypt_unrolled(uint32_t& s0, uint32_t& s1, uint32_t& s2,
                                                   uint32_t& s3, const uint4 (&rk)[11]) const {
    s0 ^= rk[0].x;
    s1 ^= rk[0].y;
    s2 ^= rk[0].z;
    s3 ^= rk[0].w;
#pragma unroll
    for (int r = 1; r < 10; ++r) round(s0, s1, s2, s3, rk[r].x, rk[r].y, rk[r].z, rk[r].w);
    const uint32_t o0 = last_col(s0, s1, s2, s3) ^ rk[10].x;
    const uint32_t o1 = last_col(s1, s2, s3, s0) ^ rk[10].y;
    const uint32_t o2 = last_col(s2, s3, s0, s1) ^ rk[10].z;
    const uint32_t o3 = last_col(s3, s0, s1, s2) ^ rk[10].w;
    s0 = o0;
    s1 = o1;
    s2 = o2;
    s3 = o3;
  }

  // N independent encryptions in lockstep (state n under round keys rk[n]):
  // each round issues the table reads of all N states before any of them is
  // used, so a lane pays about one block's latency for N blocks.  For the
  // latency-bound kernels, where a lane encrypts several blocks whose inputs
  // are all known.
  template <int N>
  __device__ __forceinline__ void encrypt_n(uint32_t (&st)[N][4], const uint4* const (&rk)[N]) const {
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const uint4 k = rk[n][0];
      st[n][0] ^= k.x;
      st[n][1] ^= k.y;
      st[n][2] ^= k.z;
      st[n][3] ^= k.w;
    }
#pragma unroll 1
    for (int r = 1; r < 10; ++r) {
      // All 16 N table reads (and the round keys) are issued before any is
      // used: left to itself the scheduler interleaves reads and uses in
      // runs of a few, and the round then pays the LDS latency several
      // times over.
      const uint32_t* p[N][16];
#pragma unroll
      for (int n = 0; n < N; ++n)
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            p[n][4 * c + j] = tab + (((st[n][(c + j) & 3] >> (8 * j)) & 0xffu) * kCopies + lane_word);
      __builtin_amdgcn_sched_barrier(0);
      uint32_t v[N][16];
      uint4 k[N];
#pragma unroll
      for (int n = 0; n < N; ++n) {
        k[n] = rk[n][r];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[n][i] = *p[n][i];
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int n = 0; n < N; ++n) {
        const uint32_t kk[4] = {k[n].x, k[n].y, k[n].z, k[n].w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
          st[n][c] = v[n][4 * c] ^ rotl32(v[n][4 * c + 1], 8) ^ rotl32(v[n][4 * c + 2], 16) ^
                     rotl32(v[n][4 * c + 3], 24) ^ kk[c];
      }
    }
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const uint4 k = rk[n][10];
      const uint32_t o0 = last_col(st[n][0], st[n][1], st[n][2], st[n][3]) ^ k.x;
      const uint32_t o1 = last_col(st[n][1], st[n][2], st[n][3], st[n][0]) ^ k.y;
      const uint32_t o2 = last_col(st[n][2], st[n][3], st[n][0], st[n][1]) ^ k.z;
      const uint32_t o3 = last_col(st[n][3], st[n][0], st[n][1], st[n][2]) ^ k.w;
      st[n][0] = o0;
      st[n][1] = o1;
      st[n][2] = o2;
      st[n][3] = o3;
    }
  }

  // Column-parallel encryption over a quad of lanes (lanes 4m..4m+3, all
  // active), N independent blocks in lockstep: lane q = lane & 3 holds
  // column q of block n in s[n] and reads column q of its round key r at
  // rkq[n][4 r].  Byte k of a lane's column feeds output column q - k
  // through T rotated by 8k; the lane takes the three terms of its own
  // output column that other columns produce from lanes q + 1, q + 2 and
  // q + 3.  Per round and block a lane issues 4 table reads and about 16
  // VALU operations instead of 16 and 60: the same lane-work as encrypt(),
  // a quarter of its dependent issue time per block.
  template <int N>
  __device__ __forceinline__ void encrypt_quad_n(uint32_t (&s)[N],
                                                 const uint32_t* const (&rkq)[N]) const {
#pragma unroll
    for (int n = 0; n < N; ++n) s[n] ^= rkq[n][0];
#pragma unroll 1
    for (int r = 1; r < 10; ++r) {
      // The round's table reads are all issued before any is used.
      const uint32_t* p[N][4];
#pragma unroll
      for (int n = 0; n < N; ++n)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          p[n][j] = tab + (((s[n] >> (8 * j)) & 0xffu) * kCopies + lane_word);
      __builtin_amdgcn_sched_barrier(0);
      uint32_t a[N][4], k[N];
#pragma unroll
      for (int n = 0; n < N; ++n) {
        k[n] = rkq[n][4 * r];
#pragma unroll
        for (int j = 0; j < 4; ++j) a[n][j] = *p[n][j];
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int n = 0; n < N; ++n)
        s[n] = a[n][0] ^ quad_rot<1>(rotl32(a[n][1], 8)) ^ quad_rot<2>(rotl32(a[n][2], 16)) ^
               quad_rot<3>(rotl32(a[n][3], 24)) ^ k[n];
    }
    // Final round: S(x) is byte 1 of T(x) (also byte 2).
    uint32_t u[N][4];
#pragma unroll
    for (int n = 0; n < N; ++n) {
      u[n][0] = (b0(s[n]) >> 8) & 0xffu;
      u[n][1] = b1(s[n]) & 0xff00u;
      u[n][2] = b2(s[n]) & 0xff0000u;
      u[n][3] = (b3(s[n]) << 8) & 0xff000000u;
    }
#pragma unroll
    for (int n = 0; n < N; ++n)
      s[n] = (u[n][0] | quad_rot<1>(u[n][1]) | quad_rot<2>(u[n][2]) | quad_rot<3>(u[n][3])) ^
             rkq[n][40];
  }

  // Only byte 0 of the ciphertext: rounds 1-8 in full, column 0 of round 9,
  // one S-box lookup in round 10.
  __device__ __forceinline__ uint32_t encrypt_byte0(uint32_t s0, uint32_t s1, uint32_t s2,
                                                    uint32_t s3, const uint4* rk) const {
    uint4 k = rk[0];
    s0 ^= k.x;
    s1 ^= k.y;
    s2 ^= k.z;
    s3 ^= k.w;
#pragma unroll
    for (int r = 1; r < 9; ++r) {
      k = rk[r];
      round(s0, s1, s2, s3, k.x, k.y, k.z, k.w);
    }
    const uint32_t k9 = reinterpret_cast<const uint32_t*>(rk)[36];
    const uint32_t k10 = reinterpret_cast<const uint32_t*>(rk)[40];
    uint32_t c0 = b0(s0) ^ rotl32(b1(s1), 8) ^ rotl32(b2(s2), 16) ^ rotl32(b3(s3), 24) ^ k9;
    return ((b0(c0) >> 8) ^ k10) & 0xffu;
  }
};

// Copies `nkeys` expanded keys (44 words each) from a kernel argument into
// LDS as uint4 rounds.  Must be followed by __syncthreads().
__device__ __forceinline__ void fill_round_keys(uint4* lds, const uint32_t (*rk)[44], int nkeys) {
  for (int i = threadIdx.x; i < nkeys * 11; i += blockDim.x) {
    const uint32_t* k = rk[i / 11] + 4 * (i % 11);
    lds[i] = make_uint4(k[0], k[1], k[2], k[3]);
  }
}

// ---------------------------------------------------------------------------
// Four-table variant: T0..T3 = rotl(8j)(T), each replicated 32 ways.  LDS
// banks serve a wave64 read as two 32-lane halves, so lane l reading copy
// l % 32 is conflict-free.  Two tables share each 64 KB half:
//   byte address = (j >> 1) * 65536 + e * 256 + (j & 1) * 128 + c * 4,
// so a lookup is still one v_perm_b32 from the state word and a per-lane
// base, and a column is T0[a] ^ T1[b] ^ T2[c] ^ T3[d] ^ k -- two 3-input
// XORs, no rotates, round keys in plain FIPS-197 order.
struct AesLds4 {
  static constexpr int kCopies = 32;
  static constexpr int kWords = 4 * 256 * kCopies;  // 128 KB
  const uint32_t* lds;
  uint32_t base[4];  // per-lane address byte 0 / byte 2 for T0..T3

  __device__ __forceinline__ static AesLds4 make(const uint32_t* lds) {
    const uint32_t c4 = (threadIdx.x & 31u) * 4u;
    return AesLds4{lds, {c4, c4 | 128u, c4 | 0x10000u, c4 | 0x10080u}};
  }
  __device__ __forceinline__ static uint32_t sel(int k) {
    // byte0 <- src1 byte0, byte1 <- src0 byte k, byte2 <- src1 byte2, byte3 <- 0
    return 0x0c020000u | uint32_t(4 + k) << 8;
  }
  template <int j, int k>
  __device__ __forceinline__ uint32_t t(uint32_t w) const {
    const uint32_t addr = __builtin_amdgcn_perm(w, base[j], sel(k));
    return *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(lds) + addr);
  }
  __device__ __forceinline__ static uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
  }
  __device__ __forceinline__ uint32_t col(uint32_t a, uint32_t b, uint32_t c, uint32_t d,
                                          uint32_t k) const {
    return xor3(xor3(t<0, 0>(a), t<1, 1>(b), t<2, 2>(c)), t<3, 3>(d), k);
  }
  __device__ __forceinline__ void round(uint32_t& s0, uint32_t& s1, uint32_t& s2, uint32_t& s3,
                                        const uint4 k) const {
    const uint32_t n0 = col(s0, s1, s2, s3, k.x);
    const uint32_t n1 = col(s1, s2, s3, s0, k.y);
    const uint32_t n2 = col(s2, s3, s0, s1, k.z);
    const uint32_t n3 = col(s3, s0, s1, s2, k.w);
    s0 = n0;
    s1 = n1;
    s2 = n2;
    s3 = n3;
  }
  // Final round: S(x) is byte 0 of T3[x], byte 1 of T0[x], byte 2 of T0[x]
  // and byte 3 of T1[x].
  __device__ __forceinline__ uint32_t last_col(uint32_t a, uint32_t b, uint32_t c, uint32_t d,
                                               uint32_t k) const {
    const uint32_t lo = __builtin_amdgcn_perm(t<0, 1>(b), t<3, 0>(a), 0x0c0c0500u);  // bytes 0,1
    const uint32_t hi = __builtin_amdgcn_perm(t<1, 3>(d), t<0, 2>(c), 0x07020c0cu);  // bytes 2,3
    return (lo | hi) ^ k;
  }
  __device__ __forceinline__ void encrypt(uint32_t& s0, uint32_t& s1, uint32_t& s2, uint32_t& s3,
                                          const uint4* rk) const {
    uint4 k = rk[0];
    s0 ^= k.x;
    s1 ^= k.y;
    s2 ^= k.z;
    s3 ^= k.w;
#pragma unroll
    for (int r = 1; r < 10; ++r) round(s0, s1, s2, s3, rk[r]);
    k = rk[10];
    const uint32_t o0 = last_col(s0, s1, s2, s3, k.x);
    const uint32_t o1 = last_col(s1, s2, s3, s0, k.y);
    const uint32_t o2 = last_col(s2, s3, s0, s1, k.z);
    const uint32_t o3 = last_col(s3, s0, s1, s2, k.w);
    s0 = o0;
    s1 = o1;
    s2 = o2;
    s3 = o3;
  }
  __device__ __forceinline__ uint32_t encrypt_byte0(uint32_t s0, uint32_t s1, uint32_t s2,
                                                    uint32_t s3, const uint4* rk) const {
    uint4 k = rk[0];
    s0 ^= k.x;
    s1 ^= k.y;
    s2 ^= k.z;
    s3 ^= k.w;
#pragma unroll
    for (int r = 1; r < 9; ++r) round(s0, s1, s2, s3, rk[r]);
    const uint32_t c0 = col(s0, s1, s2, s3, rk[9].x);
    return (t<3, 0>(c0) ^ rk[10].x) & 0xffu;
  }
  // N independent blocks in lockstep (AesLds2::encrypt_n's contract): each
  // round computes every table address, then issues every table read and
  // round key, then combines (two 3-input XORs per column), with scheduling
  // barriers between the three groups.
  template <int N>
  __device__ __forceinline__ void encrypt_n(uint32_t (&st)[N][4], const uint4* const (&rk)[N]) const {
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const uint4 k = rk[n][0];
      st[n][0] ^= k.x;
      st[n][1] ^= k.y;
      st[n][2] ^= k.z;
      st[n][3] ^= k.w;
    }
#pragma unroll 1
    for (int r = 1; r < 10; ++r) {
      uint32_t addr[N][16];
#pragma unroll
      for (int n = 0; n < N; ++n)
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            addr[n][4 * c + j] = __builtin_amdgcn_perm(st[n][(c + j) & 3], base[j], sel(j));
      __builtin_amdgcn_sched_barrier(0);
      uint32_t v[N][16];
      uint4 k[N];
#pragma unroll
      for (int n = 0; n < N; ++n) {
        k[n] = rk[n][r];
#pragma unroll
        for (int i = 0; i < 16; ++i)
          v[n][i] = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(lds) +
                                                       addr[n][i]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int n = 0; n < N; ++n) {
        const uint32_t kk[4] = {k[n].x, k[n].y, k[n].z, k[n].w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
          st[n][c] = xor3(xor3(v[n][4 * c], v[n][4 * c + 1], v[n][4 * c + 2]), v[n][4 * c + 3],
                          kk[c]);
      }
    }
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const uint4 k = rk[n][10];
      const uint32_t o0 = last_col(st[n][0], st[n][1], st[n][2], st[n][3], k.x);
      const uint32_t o1 = last_col(st[n][1], st[n][2], st[n][3], st[n][0], k.y);
      const uint32_t o2 = last_col(st[n][2], st[n][3], st[n][0], st[n][1], k.z);
      const uint32_t o3 = last_col(st[n][3], st[n][0], st[n][1], st[n][2], k.w);
      st[n][0] = o0;
      st[n][1] = o1;
      st[n][2] = o2;
      st[n][3] = o3;
    }
  }
  // Staging split into loads and stores (AesLds2::Filler's contract), so a
  // kernel can issue its other staging loads between them: each of kThreads
  // threads loads the T words of its slots, then stores them rotated into
  // the four tables, four copies per 16-byte store.
  template <int kThreads>
  struct Filler {
    static constexpr int kSlots = kWords / 4;
    static constexpr int kPer = (kSlots + kThreads - 1) / kThreads;
    uint32_t v[kPer];
    __device__ __forceinline__ static int entry(int q) { return ((4 * q) >> 6) & 255; }
    __device__ __forceinline__ void load(const uint32_t* tsrc) {
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int q = int(threadIdx.x) + u * kThreads;
        v[u] = tsrc[entry(q < kSlots ? q : kSlots - 1)];
      }
    }
    __device__ __forceinline__ void store(uint32_t* lds) const {
      uint4* dst = reinterpret_cast<uint4*>(lds);
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int q = int(threadIdx.x) + u * kThreads;
        const int i = 4 * q;
        const int j = 2 * (i >> 14) + ((i >> 5) & 1);
        const uint32_t w = rotl32(v[u], 8 * j);
        if (q < kSlots) dst[q] = make_uint4(w, w, w, w);
      }
    }
  };
  // Column-parallel AES-128 over a quad of lanes (lanes 4m..4m+3, all
  // active): lane q = lane & 3 holds column q of the state and reads column
  // q of round key r at rkq[4 r].  A lane looks up the four bytes of its own
  // column -- byte k feeds output column q - k through T_k -- and takes the
  // other three terms of its column from lanes q + 1, q + 2 and q + 3 (DPP
  // quad permutes).  Per round a lane issues 4 table reads and about 8 VALU
  // operations instead of 16 and 24: a quarter of encrypt()'s dependent
  // issue time for one block, at 4 lanes per block.  encrypt_quad_n runs
  // N independent blocks in lockstep (their table reads issued together).
  template <int N>
  __device__ __forceinline__ void encrypt_quad_n(uint32_t (&s)[N],
                                                 const uint32_t* const (&rkq)[N]) const {
#pragma unroll
    for (int n = 0; n < N; ++n) s[n] ^= rkq[n][0];
#pragma unroll
    for (int r = 1; r < 10; ++r) {
      uint32_t a[N][4];
#pragma unroll
      for (int n = 0; n < N; ++n) {
        a[n][0] = t<0, 0>(s[n]);
        a[n][1] = t<1, 1>(s[n]);
        a[n][2] = t<2, 2>(s[n]);
        a[n][3] = t<3, 3>(s[n]);
      }
#pragma unroll
      for (int n = 0; n < N; ++n)
        s[n] = a[n][0] ^ quad_rot<1>(a[n][1]) ^ quad_rot<2>(a[n][2]) ^ quad_rot<3>(a[n][3]) ^
               rkq[n][4 * r];
    }
    // Final round: S(x) is byte 0 of T3[x], bytes 1 and 2 of T0[x] and
    // byte 3 of T1[x].
    uint32_t u[N][4];
#pragma unroll
    for (int n = 0; n < N; ++n) {
      u[n][0] = t<3, 0>(s[n]);
      u[n][1] = t<0, 1>(s[n]);
      u[n][2] = t<0, 2>(s[n]);
      u[n][3] = t<1, 3>(s[n]);
    }
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const uint32_t lo = (u[n][0] & 0xffu) | (quad_rot<1>(u[n][1]) & 0xff00u);
      const uint32_t hi = (quad_rot<2>(u[n][2]) & 0xff0000u) | (quad_rot<3>(u[n][3]) & 0xff000000u);
      s[n] = (lo | hi) ^ rkq[n][40];
    }
  }
  __device__ __forceinline__ uint32_t encrypt_quad(uint32_t pt, const uint32_t* rkq) const {
    uint32_t s[1] = {pt};
    const uint32_t* const k[1] = {rkq};
    encrypt_quad_n<1>(s, k);
    return s[0];
  }
  // Ciphertext words 0 and 1 only (the final round skips columns 2 and 3).
  __device__ __forceinline__ void encrypt_lo2(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t s3,
                                              const uint4* rk, uint32_t& o0,
                                              uint32_t& o1) const {
    uint4 k = rk[0];
    s0 ^= k.x;
    s1 ^= k.y;
    s2 ^= k.z;
    s3 ^= k.w;
#pragma unroll
    for (int r = 1; r < 10; ++r) round(s0, s1, s2, s3, rk[r]);
    k = rk[10];
    o0 = last_col(s0, s1, s2, s3, k.x);
    o1 = last_col(s1, s2, s3, s0, k.y);
  }
  // Cooperative fill; follow with __syncthreads().  T is first staged in
  // LDS (`stage`, 256 words) so that the replication loop reads LDS, not
  // global memory: the fill then costs a few microseconds even for kernels
  // with little other work.
  __device__ __forceinline__ static void fill(uint32_t* lds, uint32_t* stage,
                                              const uint32_t* tsrc) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x) stage[i] = tsrc[i];
    __syncthreads();
    // 16-byte stores: words 4q..4q+3 are four copies of one (table, entry).
    uint4* dst = reinterpret_cast<uint4*>(lds);
#pragma unroll 4
    for (int q = threadIdx.x; q < kWords / 4; q += blockDim.x) {
      const int i = 4 * q;
      const int half = i >> 14;  // 16384 words per 64 KB half
      const int e = (i >> 6) & 255;
      const int j = 2 * half + ((i >> 5) & 1);
      const uint32_t v = rotl32(stage[e], 8 * j);
      dst[q] = make_uint4(v, v, v, v);
    }
  }
  static void key_layout(const uint32_t rk[44], uint32_t out[44]) {
    for (int w = 0; w < 44; ++w) out[w] = rk[w];
  }
};

// Two-table variant for kernels that cannot spend AesLds4's 128 KB:
// T0 = T and T1 = rotl(8)(T), kCopies-way replicated (kCopies <= 32) in a
// 64 KB span, byte address e * 256 + j * 128 + c * 4 (the first half of
// AesLds4's layout; lane l reads copy l % kCopies).  T2 and T3 are rotl(16)
// of T0 and T1, so a column is
//   T0[a] ^ T1[b] ^ rotl16(T0[c] ^ T1[d]) ^ k:
// four single-instruction lookups (v_perm_b32 of the state word and a
// per-lane base), one rotate and three XORs -- about 32 VALU operations per
// round against 52 for the single-table form's shifted addresses and three
// rotates per column.
template <int kCopies>
struct AesLds2 {
  static_assert(kCopies >= 4 && kCopies <= 32 && (kCopies & (kCopies - 1)) == 0,
                "AesLds2: 4..32 copies, a power of two");
  static constexpr int kSpanWords = 256 * 64;  // 64 KB whatever kCopies is
  const uint32_t* lds;
  uint32_t base[2];

  __device__ __forceinline__ static AesLds2 make(const uint32_t* lds) {
    const uint32_t c4 = (threadIdx.x % kCopies) * 4u;
    return AesLds2{lds, {c4, c4 | 128u}};
  }
  template <int j, int k>
  __device__ __forceinline__ uint32_t t(uint32_t w) const {
    // byte0 <- base byte0, byte1 <- w byte k, bytes 2 and 3 <- 0
    const uint32_t addr = __builtin_amdgcn_perm(w, base[j], 0x0c0c0000u | uint32_t(4 + k) << 8);
    return *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(lds) + addr);
  }
  __device__ __forceinline__ static uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
  }
  __device__ __forceinline__ uint32_t col(uint32_t a, uint32_t b, uint32_t c, uint32_t d,
                                          uint32_t k) const {
    return xor3(t<0, 0>(a), t<1, 1>(b), k) ^ rotl32(t<0, 2>(c) ^ t<1, 3>(d), 16);
  }
  __device__ __forceinline__ void round(uint32_t& s0, uint32_t& s1, uint32_t& s2, uint32_t& s3,
                                        uint32_t k0, uint32_t k1, uint32_t k2,
                                        uint32_t k3) const {
    const uint32_t n0 = col(s0, s1, s2, s3, k0);
    const uint32_t n1 = col(s1, s2, s3, s0, k1);
    const uint32_t n2 = col(s2, s3, s0, s1, k2);
    const uint32_t n3 = col(s3, s0, s1, s2, k3);
    s0 = n0;
    s1 = n1;
    s2 = n2;
    s3 = n3;
  }
  // Final round: S(x) is byte 1 (and byte 2) of T0[x] and byte 3 of T1[x].
  __device__ __forceinline__ uint32_t last_col(uint32_t a, uint32_t b, uint32_t c, uint32_t d,
                                               uint32_t k) const {
    const uint32_t lo = __builtin_amdgcn_perm(t<0, 1>(b), t<0, 0>(a), 0x0c0c0501u);  // bytes 0,1
    const uint32_t hi = __builtin_amdgcn_perm(t<1, 3>(d), t<0, 2>(c), 0x07020c0cu);  // bytes 2,3
    return (lo | hi) ^ k;
  }
  __device__ __forceinline__ void last(uint32_t& s0, uint32_t& s1, uint32_t& s2, uint32_t& s3,
                                       const uint4 k) const {
    const uint32_t o0 = last_col(s0, s1, s2, s3, k.x);
    const uint32_t o1 = last_col(s1, s2, s3, s0, k.y);
    const uint32_t o2 = last_col(s2, s3, s0, s1, k.z);
    const uint32_t o3 = last_col(s3, s0, s1, s2, k.w);
    s0 = o0;
    s1 = o1;
    s2 = o2;
    s3 = o3;
  }
  // Same contract as AesLds::encrypt; the middle rounds stay a loop for the
  // same instruction-cache reason.
  __device__ __forceinline__ void encrypt(uint32_t& s0, uint32_t& s1, uint32_t& s2, uint32_t& s3,
                                          const uint4* rk) const {
    uint4 k = rk[0];
    s0 ^= k.x;
    s1 ^= k.y;
    s2 ^= k.z;
    s3 ^= k.w;
#pragma unroll 1
    for (int r = 1; r < 10; ++r) {
      k = rk[r];
      round(s0, s1, s2, s3, k.x, k.y, k.z, k.w);
    }
    last(s0, s1, s2, s3, rk[10]);
  }
  template <int N>
  __device__ __forceinline__ void encrypt_n(uint32_t (&st)[N][4], const uint4* const (&rk)[N]) const {
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const uint4 k = rk[n][0];
      st[n][0] ^= k.x;
      st[n][1] ^= k.y;
      st[n][2] ^= k.z;
      st[n][3] ^= k.w;
    }
#pragma unroll 1
    for (int r = 1; r < 10; ++r) {
      // All table reads of the round issued before any is used.
      uint32_t addr[N][16];
#pragma unroll
      for (int n = 0; n < N; ++n)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          addr[n][4 * c] = __builtin_amdgcn_perm(st[n][c], base[0], 0x0c0c0400u);
          addr[n][4 * c + 1] = __builtin_amdgcn_perm(st[n][(c + 1) & 3], base[1], 0x0c0c0500u);
          addr[n][4 * c + 2] = __builtin_amdgcn_perm(st[n][(c + 2) & 3], base[0], 0x0c0c0600u);
          addr[n][4 * c + 3] = __builtin_amdgcn_perm(st[n][(c + 3) & 3], base[1], 0x0c0c0700u);
        }
      __builtin_amdgcn_sched_barrier(0);
      uint32_t v[N][16];
      uint4 k[N];
#pragma unroll
      for (int n = 0; n < N; ++n) {
        k[n] = rk[n][r];
#pragma unroll
        for (int i = 0; i < 16; ++i)
          v[n][i] = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(lds) +
                                                       addr[n][i]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int n = 0; n < N; ++n) {
        const uint32_t kk[4] = {k[n].x, k[n].y, k[n].z, k[n].w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
          st[n][c] = xor3(v[n][4 * c], v[n][4 * c + 1], kk[c]) ^
                     rotl32(v[n][4 * c + 2] ^ v[n][4 * c + 3], 16);
      }
    }
#pragma unroll
    for (int n = 0; n < N; ++n) last(st[n][0], st[n][1], st[n][2], st[n][3], rk[n][10]);
  }
  // Column-parallel encryption over a lane quad (AesLds::encrypt_quad_n's
  // contract): byte k of a lane's column is looked up in T0 (k even) or T1
  // (k odd); the terms of bytes 2 and 3 arrive from lanes q + 2 and q + 3
  // and share one rotate by 16.
  template <int N>
  __device__ __forceinline__ void encrypt_quad_n(uint32_t (&s)[N],
                                                 const uint32_t* const (&rkq)[N]) const {
#pragma unroll
    for (int n = 0; n < N; ++n) s[n] ^= rkq[n][0];
#pragma unroll 1
    for (int r = 1; r < 10; ++r) {
      uint32_t addr[N][4];
#pragma unroll
      for (int n = 0; n < N; ++n) {
        addr[n][0] = __builtin_amdgcn_perm(s[n], base[0], 0x0c0c0400u);
        addr[n][1] = __builtin_amdgcn_perm(s[n], base[1], 0x0c0c0500u);
        addr[n][2] = __builtin_amdgcn_perm(s[n], base[0], 0x0c0c0600u);
        addr[n][3] = __builtin_amdgcn_perm(s[n], base[1], 0x0c0c0700u);
      }
      __builtin_amdgcn_sched_barrier(0);
      uint32_t a[N][4], k[N];
#pragma unroll
      for (int n = 0; n < N; ++n) {
        k[n] = rkq[n][4 * r];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          a[n][j] = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(lds) +
                                                       addr[n][j]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int n = 0; n < N; ++n)
        s[n] = xor3(a[n][0], quad_rot<1>(a[n][1]), k[n]) ^
               rotl32(quad_rot<2>(a[n][2]) ^ quad_rot<3>(a[n][3]), 16);
    }
    // Final round: S(x) is byte 1 (and byte 2) of T0[x] and byte 3 of T1[x].
    uint32_t u[N][4];
#pragma unroll
    for (int n = 0; n < N; ++n) {
      u[n][0] = (t<0, 0>(s[n]) >> 8) & 0xffu;
      u[n][1] = t<0, 1>(s[n]) & 0xff00u;
      u[n][2] = t<0, 2>(s[n]) & 0xff0000u;
      u[n][3] = t<1, 3>(s[n]) & 0xff000000u;
    }
#pragma unroll
    for (int n = 0; n < N; ++n)
      s[n] = (u[n][0] | quad_rot<1>(u[n][1]) | quad_rot<2>(u[n][2]) | quad_rot<3>(u[n][3])) ^
             rkq[n][40];
  }
  // Fill of the whole span by kThreads threads without a barrier: uint4
  // slot q holds entry q / 16 of table (q / 8) & 1 four times (kCopies ==
  // 32 uses every word), read straight from T in global memory.  load()
  // issues a thread's table reads, store() writes its slots, so a caller can
  // put other loads in flight between the two; follow store() with
  // __syncthreads().
  template <int kThreads>
  struct Filler {
    static_assert(kCopies == 32, "AesLds2::Filler: the 32-copy span");
    static constexpr int kSlots = kSpanWords / 4;
    static constexpr int kPer = (kSlots + kThreads - 1) / kThreads;
    uint32_t v[kPer];
    __device__ __forceinline__ void load(const uint32_t* tsrc) {
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int q = int(threadIdx.x) + u * kThreads;
        v[u] = tsrc[(q < kSlots ? q : kSlots - 1) >> 4];
      }
    }
    __device__ __forceinline__ void store(uint32_t* lds) const {
      uint4* dst = reinterpret_cast<uint4*>(lds);
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int q = int(threadIdx.x) + u * kThreads;
        const uint32_t w = rotl32(v[u], 8 * ((q >> 3) & 1));
        if (q < kSlots) dst[q] = make_uint4(w, w, w, w);
      }
    }
  };
  // Cooperative fill of the used words of the span from T in global memory
  // (staged once in LDS); contains a barrier, follow with __syncthreads().
  __device__ __forceinline__ static void fill(uint32_t* lds, const uint32_t* tsrc) {
    constexpr int kVec = kCopies / 4;  // uint4 stores per (entry, table)
    __shared__ uint32_t stage[256];
    for (int i = threadIdx.x; i < 256; i += blockDim.x) stage[i] = tsrc[i];
    __syncthreads();
    uint4* dst = reinterpret_cast<uint4*>(lds);
    for (int q = threadIdx.x; q < 256 * 2 * kVec; q += blockDim.x) {
      const int e = q / (2 * kVec), j = (q / kVec) & 1, v4 = q % kVec;
      const uint32_t v = rotl32(stage[e], 8 * j);
      dst[e * 16 + j * 8 + v4] = make_uint4(v, v, v, v);
    }
  }
};

// Cooperative fill of the replicated table from the constant T table in
// global memory (`tsrc`, 256 words): the 256 words are loaded once (one
// global round trip) into a 1 KB LDS staging copy, then replicated from LDS
// with 16-byte stores.  `lds` must be 16-byte aligned.  Contains a barrier,
// so every thread of the workgroup must call it; must be followed by
// __syncthreads() before the table is read.
template <int kCopies>
__device__ __forceinline__ void fill_ttable(uint32_t* lds, const uint32_t* tsrc) {
  static_assert(kCopies % 4 == 0, "fill_ttable: copies in groups of four");
  constexpr int kVec = kCopies / 4;
  __shared__ uint32_t stage[256];
  const int nthreads = blockDim.x;
  for (int i = threadIdx.x; i < 256; i += nthreads) stage[i] = tsrc[i];
  __syncthreads();
  uint4* dst = reinterpret_cast<uint4*>(lds);
  for (int i = threadIdx.x; i < 256 * kVec; i += nthreads) {
    const uint32_t v = stage[i / kVec];
    dst[i] = make_uint4(v, v, v, v);
  }
}

}  // namespace sufhip
