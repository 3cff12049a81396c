// Bitsliced AES-128 on the VALU: 32 blocks per lane, one 32-bit word per
// state bit (word 8 j + b holds bit b of byte j of the 32 blocks, block k in
// bit k), no tables.  Written to measure against the LDS T-table AES
// (aes_lds.hpp); the product kernels keep the T table (the measurement is in
// the DCF profile).
//
// The S-box is the field inverse followed by the FIPS-197 affine map.  The
// inverse runs in the tower field GF((2^4)^2) = GF(2^4)[z] / (z^2 + z + lam),
// GF(2^4) = GF(2)[y] / (y^4 + y + 1): for a = ah z + al,
//   a^-1 = (ah z + (ah + al)) d^-1,  d = lam ah^2 + ah al + al^2,
// with d^-1 = d^14 in GF(2^4).  The maps between the AES polynomial basis and
// the tower basis are 8 x 8 GF(2) matrices derived below at compile time
// from their definition (Y with Y^4 + Y + 1 = 0 and Z with Z^2 + Z + lam(Y)
// = 0 in the AES field; lam the smallest element making z^2 + z + lam
// irreducible), so a constant folds into XORs of slices.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sufhip {
namespace aes_bs {

// ---- compile-time field arithmetic (bytes) --------------------------------

constexpr uint32_t aes_mul(uint32_t a, uint32_t b) {
  uint32_t r = 0;
  for (int i = 0; i < 8; ++i) {
    if ((b >> i) & 1u) r ^= a;
    a <<= 1;
    if (a & 0x100u) a ^= 0x11bu;
  }
  return r;
}

constexpr uint32_t aes_pow(uint32_t a, int e) {
  uint32_t r = 1;
  for (int i = 0; i < e; ++i) r = aes_mul(r, a);
  return r;
}

constexpr uint32_t g16_mul(uint32_t a, uint32_t b) {
  uint32_t r = 0;
  for (int i = 0; i < 4; ++i)
    if ((b >> i) & 1u) r ^= a << i;
  for (int k = 6; k >= 4; --k)
    if ((r >> k) & 1u) r ^= 0x13u << (k - 4);
  return r;
}

constexpr uint32_t find_lam() {
  for (uint32_t l = 1; l < 16; ++l) {
    bool root = false;
    for (uint32_t t = 0; t < 16; ++t) root = root || ((g16_mul(t, t) ^ t) == l);
    if (!root) return l;
  }
  return 0;
}

constexpr uint32_t kLam = find_lam();

constexpr uint32_t find_y() {
  for (uint32_t y = 2; y < 256; ++y)
    if ((aes_pow(y, 4) ^ y ^ 1u) == 0) return y;
  return 0;
}

constexpr uint32_t eval_at(uint32_t poly4, uint32_t y) {
  uint32_t r = 0;
  for (int i = 0; i < 4; ++i)
    if ((poly4 >> i) & 1u) r ^= aes_pow(y, i);
  return r;
}

constexpr uint32_t find_z(uint32_t y) {
  const uint32_t l = eval_at(kLam, y);
  for (uint32_t z = 2; z < 256; ++z)
    if ((aes_mul(z, z) ^ z ^ l) == 0) return z;
  return 0;
}

// An 8 x 8 GF(2) matrix as its columns (column j: the image of bit j).
struct Mat8 {
  uint32_t col[8];
};

constexpr uint32_t apply(const Mat8& m, uint32_t v) {
  uint32_t r = 0;
  for (int j = 0; j < 8; ++j)
    if ((v >> j) & 1u) r ^= m.col[j];
  return r;
}

// Tower -> AES basis: bits 0-3 of a tower byte are al (y^i), bits 4-7 ah
// (y^i z).
constexpr Mat8 tower_to_aes() {
  const uint32_t y = find_y(), z = find_z(y);
  Mat8 m{};
  for (int i = 0; i < 4; ++i) {
    m.col[i] = aes_pow(y, i);
    m.col[4 + i] = aes_mul(aes_pow(y, i), z);
  }
  return m;
}

constexpr Mat8 invert(const Mat8& m) {
  Mat8 r{};
  for (uint32_t v = 0; v < 256; ++v) {
    const uint32_t w = apply(m, v);
    for (int j = 0; j < 8; ++j)
      if (w == (1u << j)) r.col[j] = v;
  }
  return r;
}

// FIPS-197 5.1.1: b_i ^= b_{i+4} ^ b_{i+5} ^ b_{i+6} ^ b_{i+7} (then ^ 0x63).
constexpr Mat8 affine_mat() {
  Mat8 m{};
  for (int j = 0; j < 8; ++j) {
    uint32_t c = 0;
    for (int i = 0; i < 8; ++i) {
      const bool on = i == j || (i + 4) % 8 == j || (i + 5) % 8 == j || (i + 6) % 8 == j ||
                      (i + 7) % 8 == j;
      if (on) c |= 1u << i;
    }
    m.col[j] = c;
  }
  return m;
}

constexpr Mat8 mul(const Mat8& a, const Mat8& b) {  // a after b
  Mat8 r{};
  for (int j = 0; j < 8; ++j) r.col[j] = apply(a, b.col[j]);
  return r;
}

constexpr Mat8 kIn = invert(tower_to_aes());                // AES basis -> tower
constexpr Mat8 kOut = mul(affine_mat(), tower_to_aes());    // tower -> affine(AES)

// lam * v in GF(2^4) as a 4 x 4 matrix (columns: lam y^j).
constexpr uint32_t lam_col(int j) { return g16_mul(kLam, 1u << j); }

static_assert(find_y() != 0 && kLam != 0, "tower field constants");
static_assert(apply(kIn, apply(tower_to_aes(), 0x5a)) == 0x5a, "basis maps are inverse");

// ---- slice arithmetic ------------------------------------------------------

// out = M x over 8 slices, M = kIn or kOut (a constant: each output slice an
// XOR of input slices).
template <bool kToTower>
__host__ __device__ __forceinline__ void mat8(const uint32_t (&x)[8], uint32_t (&o)[8]) {
  constexpr Mat8 m = kToTower ? kIn : kOut;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t v = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if ((m.col[j] >> i) & 1u) v ^= x[j];
    o[i] = v;
  }
}

// GF(2^4) product of 4-slice values: schoolbook, then y^4 = y + 1.
__host__ __device__ __forceinline__ void g16_mul_s(const uint32_t (&a)[4], const uint32_t (&b)[4],
                                                   uint32_t (&r)[4]) {
  uint32_t c[7];
  c[0] = a[0] & b[0];
  c[1] = (a[0] & b[1]) ^ (a[1] & b[0]);
  c[2] = (a[0] & b[2]) ^ (a[1] & b[1]) ^ (a[2] & b[0]);
  c[3] = (a[0] & b[3]) ^ (a[1] & b[2]) ^ (a[2] & b[1]) ^ (a[3] & b[0]);
  c[4] = (a[1] & b[3]) ^ (a[2] & b[2]) ^ (a[3] & b[1]);
  c[5] = (a[2] & b[3]) ^ (a[3] & b[2]);
  c[6] = a[3] & b[3];
  r[0] = c[0] ^ c[4];
  r[1] = c[1] ^ c[4] ^ c[5];
  r[2] = c[2] ^ c[5] ^ c[6];
  r[3] = c[3] ^ c[6];
}

// Square in GF(2^4): a0 + a1 y^2 + a2 (y + 1) + a3 (y^3 + y^2).
__host__ __device__ __forceinline__ void g16_sq_s(const uint32_t (&a)[4], uint32_t (&r)[4]) {
  r[0] = a[0] ^ a[2];
  r[1] = a[2];
  r[2] = a[1] ^ a[3];
  r[3] = a[3];
}

__host__ __device__ __forceinline__ void g16_inv_s(const uint32_t (&a)[4], uint32_t (&r)[4]) {
  uint32_t a2[4], a3[4], a6[4], a12[4];
  g16_sq_s(a, a2);
  g16_mul_s(a2, a, a3);
  g16_sq_s(a3, a6);
  g16_sq_s(a6, a12);
  g16_mul_s(a12, a2, r);  // a^14 = a^-1 (0 -> 0)
}

// S-box of 8 slices in place.
__host__ __device__ __forceinline__ void sbox_s(uint32_t (&x)[8]) {
  uint32_t t[8];
  mat8<true>(x, t);
  const uint32_t al[4] = {t[0], t[1], t[2], t[3]}, ah[4] = {t[4], t[5], t[6], t[7]};
  uint32_t h2[4], l2[4], hl[4], d[4], di[4], lh2[4];
  g16_sq_s(ah, h2);
  g16_sq_s(al, l2);
  g16_mul_s(ah, al, hl);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t v = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if ((lam_col(j) >> i) & 1u) v ^= h2[j];
    lh2[i] = v;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) d[i] = lh2[i] ^ hl[i] ^ l2[i];
  g16_inv_s(d, di);
  const uint32_t hs[4] = {ah[0] ^ al[0], ah[1] ^ al[1], ah[2] ^ al[2], ah[3] ^ al[3]};
  uint32_t oh[4], ol[4];
  g16_mul_s(ah, di, oh);
  g16_mul_s(hs, di, ol);
  const uint32_t inv[8] = {ol[0], ol[1], ol[2], ol[3], oh[0], oh[1], oh[2], oh[3]};
  mat8<false>(inv, x);
  // ^ 0x63: bits 0, 1, 5, 6
  x[0] = ~x[0];
  x[1] = ~x[1];
  x[5] = ~x[5];
  x[6] = ~x[6];
}

// State: s[8 j + b] = bit b of byte j (column c = bytes 4c..4c+3).
__host__ __device__ __forceinline__ void sub_bytes(uint32_t (&s)[128]) {
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    uint32_t x[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) x[b] = s[8 * j + b];
    sbox_s(x);
#pragma unroll
    for (int b = 0; b < 8; ++b) s[8 * j + b] = x[b];
  }
}

// ShiftRows then MixColumns (FIPS-197 5.1.2-5.1.3); `mix` false: the last
// round's ShiftRows alone.  Byte r of column c comes from column c + r.
template <bool kMix>
__host__ __device__ __forceinline__ void shift_mix(uint32_t (&s)[128]) {
  uint32_t t[128];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int b = 0; b < 8; ++b) t[8 * (4 * c + r) + b] = s[8 * (4 * ((c + r) & 3) + r) + b];
  if constexpr (!kMix) {
#pragma unroll
    for (int i = 0; i < 128; ++i) s[i] = t[i];
  } else {
    // out_r = a_r ^ u ^ xtime(a_r ^ a_{r+1}), u = a_0 ^ a_1 ^ a_2 ^ a_3.
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint32_t u[8];
#pragma unroll
      for (int b = 0; b < 8; ++b)
        u[b] = t[8 * (4 * c) + b] ^ t[8 * (4 * c + 1) + b] ^ t[8 * (4 * c + 2) + b] ^
               t[8 * (4 * c + 3) + b];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        uint32_t e[8];
#pragma unroll
        for (int b = 0; b < 8; ++b) e[b] = t[8 * (4 * c + r) + b] ^ t[8 * (4 * c + ((r + 1) & 3)) + b];
        // xtime: shift left, reduce by 0x1b (bits 0, 1, 3, 4).
        const uint32_t x[8] = {e[7], e[0] ^ e[7], e[1], e[2] ^ e[7], e[3] ^ e[7], e[4], e[5], e[6]};
#pragma unroll
        for (int b = 0; b < 8; ++b) s[8 * (4 * c + r) + b] = t[8 * (4 * c + r) + b] ^ u[b] ^ x[b];
      }
    }
  }
}

// AddRoundKey with round key words rk[0..3] (uniform over the 32 blocks).
__host__ __device__ __forceinline__ void add_round_key(uint32_t (&s)[128], const uint32_t* rk) {
#pragma unroll
  for (int i = 0; i < 128; ++i) s[i] ^= 0u - ((rk[i >> 5] >> (i & 31)) & 1u);
}

// 32 x 32 bit transpose: bit k of a[i] <-> bit i of a[k].
__host__ __device__ __forceinline__ void transpose32(uint32_t (&a)[32]) {
  uint32_t m = 0x0000ffffu;
#pragma unroll
  for (int j = 16; j != 0; j >>= 1, m ^= m << j) {
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      if (k & j) continue;
      const uint32_t t = ((a[k] >> j) ^ a[k | j]) & m;
      a[k] ^= t << j;
      a[k | j] ^= t;
    }
  }
}

// Full encryption of the 32 blocks in s; rk: the 44 expanded key words.
__host__ __device__ __forceinline__ void encrypt(uint32_t (&s)[128], const uint32_t* rk) {
  add_round_key(s, rk);
#pragma unroll 1
  for (int r = 1; r < 10; ++r) {
    sub_bytes(s);
    shift_mix<true>(s);
    add_round_key(s, rk + 4 * r);
  }
  sub_bytes(s);
  shift_mix<false>(s);
  add_round_key(s, rk + 40);
}

}  // namespace aes_bs
}  // namespace sufhip
