/*
 * Truncation gate: keygen and evaluation (test infrastructure only).
 *
 * Restates, for one gate instance with a scalar input mask r:
 *   - keygen  composite_gen_trunc_gate (include/gates/composite_fss.hpp:645-833)
 *             with the predicate SUFs of include/suf/trunc_suf_builders.hpp:16-75,
 *             the mask rewrites of include/suf/mask_rewrite.hpp:13-42 and the
 *             64-bit wrap query of src/compiler/suf_to_pfss.cpp:443-455;
 *   - eval    the AddU64 branch of composite_eval_batch_backend
 *             (composite_fss.hpp:1385-1638: carry = NOT(RotXor), RotXor =
 *             (b - a) + w on additive predicate shares);
 *   - postproc FaithfulTruncPostProc / FaithfulArsPostProc / GapArsPostProc
 *             (include/gates/postproc_hooks.hpp:172-373).
 *
 * Predicates after the rewrite (x^ = x + r public, r_low = r mod 2^f):
 *   carry  = NOT(RotXor(1[x^_low < r_low], 1[x^_low < 0], w = 1)) = 1[x^_low < r_low]
 *            (no query at all when r_low == 0: carry is the constant 0);
 *   wrap   = 1[x^ < r]                                   (TR, ARS)
 *   sign   = RotXor(1[x^ < r + 2^63], 1[x^ < r], w = 1[r < 2^63])   (ARS)
 * The query 1[x^_low < 0] is identically 0 (unsigned compare), so it is
 * folded to 0 instead of being keyed: the carry share is [p0] - w_p + a_p.
 *
 * Randomness comes from the caller as 19 u64 words at fixed positions (the
 * reference draws the same quantities from its std::mt19937_64 and the DCF
 * seeds from std::random_device):
 *   0 r | 1 r_in split | 2 r_out split (zero-sum) | 3 carry-w split |
 *   4 sign-w split | 5 r_hi split | 6 m split |
 *   7..10 carry DCF seeds | 11..14 wrap DCF seeds | 15..18 sign DCF seeds
 * (a DCF's four words: party-0 seed = words 0,1 LE, party-1 seed = words 2,3).
 * A split of v gives party 0 the word s and party 1 v - s.
 *
 * Blob (per party, little-endian):
 *   0 u32 tag 'STG1' | 4 u8 kind | 5 u8 frac_bits | 6 u8 party | 7 u8 flags
 *   (bit 0 carry key, bit 1 wrap key, bit 2 sign key) | 8 r_in share |
 *   16 r_hi share | 24 base share (r_out) | 32 carry-w share | 40 sign-w share |
 *   48 m share | 56 u32 carry key bytes | 60 u32 64-bit key bytes |
 *   64 carry DCF key (f bits, 8-byte payload 1, additive group), padded to 8 |
 *   wrap DCF key (64 bits) | sign DCF key (64 bits), each padded to 8.
 */
#include <string.h>

#include "oracle.h"

#define TAG 0x31475453u /* "STG1" */

static size_t pad8(size_t v) { return (v + 7) & ~(size_t)7; }

static void put64(uint8_t* p, uint64_t v) {
  for (int i = 0; i < 8; i++) p[i] = (uint8_t)(v >> (8 * i));
}
static uint64_t get64(const uint8_t* p) {
  uint64_t v = 0;
  for (int i = 0; i < 8; i++) v |= (uint64_t)p[i] << (8 * i);
  return v;
}
static uint32_t get32(const uint8_t* p) {
  return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}

size_t orc_trunc_key_bytes(int kind, int f) {
  if (kind < ORC_TRUNC_TR || kind > ORC_TRUNC_GAPARS || f < 1 || f > 62) return 0;
  size_t b = 64 + pad8(orc_myl7_key_bytes(f, 8));
  if (kind != ORC_TRUNC_GAPARS) b += pad8(orc_myl7_key_bytes(64, 8));
  if (kind == ORC_TRUNC_ARS) b += pad8(orc_myl7_key_bytes(64, 8));
  return b;
}

static void seeds_from(const uint64_t* w, uint8_t out[32]) {
  for (int j = 0; j < 4; j++) put64(out + 8 * j, w[j]);
}

int orc_trunc_gen(const orc_prg_state* p, int kind, int f, const uint64_t* rnd, uint8_t* key0,
                  uint8_t* key1) {
  size_t total = orc_trunc_key_bytes(kind, f);
  if (!total) return -1;
  memset(key0, 0, total);
  memset(key1, 0, total);
  const uint64_t r = rnd[0];
  const uint64_t r_low = r & ((1ULL << f) - 1);
  const uint64_t r_hi = r >> f;
  const uint64_t m = (kind == ORC_TRUNC_GAPARS && (r >> 63)) ? (1ULL << (64 - f)) : 0;
  const uint64_t sign_w = (r < (1ULL << 63)) ? 1 : 0; /* 1[r < r + 2^63 mod 2^64] */
  const int has_carry = r_low != 0;
  const int has_wrap = kind != ORC_TRUNC_GAPARS;
  const int has_sign = kind == ORC_TRUNC_ARS;
  const uint32_t ckb = (uint32_t)orc_myl7_key_bytes(f, 8);
  const uint32_t ukb = (uint32_t)orc_myl7_key_bytes(64, 8);
  uint8_t* keys[2] = {key0, key1};
  for (int b = 0; b < 2; b++) {
    uint8_t* k = keys[b];
    k[0] = (uint8_t)TAG;
    k[1] = (uint8_t)(TAG >> 8);
    k[2] = (uint8_t)(TAG >> 16);
    k[3] = (uint8_t)(TAG >> 24);
    k[4] = (uint8_t)kind;
    k[5] = (uint8_t)f;
    k[6] = (uint8_t)b;
    k[7] = (uint8_t)(has_carry | has_wrap << 1 | has_sign << 2);
#define SPLIT(v, s) (b == 0 ? (s) : (v) - (s))
    put64(k + 8, SPLIT(r, rnd[1]));
    put64(k + 16, SPLIT(r_hi, rnd[5]));
    put64(k + 24, SPLIT(0ULL, rnd[2]));
    put64(k + 32, has_carry ? SPLIT(1ULL, rnd[3]) : 0);
    put64(k + 40, has_sign ? SPLIT(sign_w, rnd[4]) : 0);
    put64(k + 48, kind == ORC_TRUNC_GAPARS ? SPLIT(m, rnd[6]) : 0);
#undef SPLIT
    for (int i = 0; i < 4; i++) k[56 + i] = (uint8_t)(ckb >> (8 * i));
    for (int i = 0; i < 4; i++) k[60 + i] = (uint8_t)(ukb >> (8 * i));
  }
  const uint8_t one[8] = {1, 0, 0, 0, 0, 0, 0, 0};
  uint8_t seeds[32];
  size_t off = 64;
  if (has_carry) {
    seeds_from(rnd + 7, seeds);
    if (orc_myl7_gen(p, ORC_GROUP_ADD, f, r_low, one, 8, seeds, key0 + off, key1 + off)) return -1;
  }
  off += pad8(ckb);
  if (has_wrap) {
    seeds_from(rnd + 11, seeds);
    if (orc_myl7_gen(p, ORC_GROUP_ADD, 64, r, one, 8, seeds, key0 + off, key1 + off)) return -1;
    off += pad8(ukb);
  }
  if (has_sign) {
    seeds_from(rnd + 15, seeds);
    if (orc_myl7_gen(p, ORC_GROUP_ADD, 64, r + (1ULL << 63), one, 8, seeds, key0 + off,
                     key1 + off))
      return -1;
  }
  return 0;
}

static uint64_t dcf_share(const orc_prg_state* p, int in_bits, const uint8_t* key, uint64_t x) {
  uint8_t out[8];
  orc_myl7_eval(p, ORC_GROUP_ADD, in_bits, key, x, out);
  return get64(out);
}

int orc_trunc_eval(const orc_prg_state* p, int kind, int f, const uint8_t* key,
                   const uint64_t* xhat, size_t n, uint64_t* y) {
  if (!orc_trunc_key_bytes(kind, f) || get32(key) != TAG || key[4] != kind || key[5] != f)
    return -1;
  const int party = key[6];
  const int flags = key[7];
  const uint64_t r_hi = get64(key + 16), base = get64(key + 24), cw = get64(key + 32);
  const uint64_t sw = get64(key + 40), m = get64(key + 48);
  const size_t ckb = get32(key + 56), ukb = get32(key + 60);
  const uint8_t* carry_key = key + 64;
  const uint8_t* wrap_key = carry_key + pad8(ckb);
  const uint8_t* sign_key = wrap_key + pad8(ukb);
  const uint64_t one = party == 0 ? 1 : 0;
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; i++) {
    const uint64_t x = xhat[i];
    uint64_t carry = 0, wrap = 0, sign = 0;
    if (flags & 1) {
      uint64_t a = dcf_share(p, f, carry_key, x & ((1ULL << f) - 1));
      carry = one - ((0 - a) + cw); /* NOT(RotXor(a, b = 0, w)) */
    }
    if (flags & 2) wrap = dcf_share(p, 64, wrap_key, x);
    if (flags & 4) sign = (wrap - dcf_share(p, 64, sign_key, x)) + sw;
    uint64_t v;
    if (kind == ORC_TRUNC_GAPARS) {
      const uint64_t hb = x + (1ULL << 62);
      v = base + (party == 0 ? hb >> f : 0) - r_hi - carry;
      if ((hb >> 63) == 0) v += m;
      if (party == 0) v -= 1ULL << (62 - f);
    } else {
      v = base + (party == 0 ? x >> f : 0) - r_hi - carry + wrap * (1ULL << (64 - f));
      if (kind == ORC_TRUNC_ARS) v += sign * (~0ULL << (64 - f));
    }
    y[i] = v;
  }
  return 0;
}
