/*
 * Oracle: myl7/fss v0.7.1 DCF (lambda = 16 bytes) and SUF's myl7 adapter.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Restates, byte for byte:
 *   - prg():      third_party/myl7_fss/src/prg/aes128_mmo.c:41-52
 *                 block i of the output = AES_{K_i}(seed) xor seed,
 *                 K_i = state[16 i .. 16 i + 16)   (prg_init, :16-31)
 *   - dcf_gen():  third_party/myl7_fss/src/dcf.c:42-142
 *   - dcf_eval(): third_party/myl7_fss/src/dcf.c:146-193
 *   - groups:     src/group/bytes.c:8-16 (XOR) and src/group/u128_le.c
 *                 (+ mod 2^127 on little-endian bytes)
 *   - key blob:   include/proto/myl7_fss_backend.hpp:131-256
 *                 [in_bits u8][num_chunks u8][party u8][0][payload_len u32 LE]
 *                 then per chunk [seed 16][cws in_bits*33][cw_np1 16]
 *   - batch:      myl7_fss_backend.hpp:73-100 (one byte per key: out[0] & 1)
 * Alpha and x are packed LSB-first into little-endian bytes
 * (myl7_fss_backend.hpp:33-71 with bits_msb_first = false), and the tree is
 * walked from bit in_bits-1 down to bit 0 (dcf.c:72-73, :177-178).
 */
#include "oracle.h"

#include <string.h>

typedef struct {
  uint64_t lo, hi;
} u128p;

static u128p ld(const uint8_t* b) {
  u128p v;
  memcpy(&v.lo, b, 8);
  memcpy(&v.hi, b + 8, 8);
  return v;
}
static void st(uint8_t* b, u128p v) {
  memcpy(b, &v.lo, 8);
  memcpy(b + 8, &v.hi, 8);
}
static const uint64_t MSB_CLEAR = 0x7FFFFFFFFFFFFFFFULL;

static u128p g_add(int group, u128p a, u128p b) {
  u128p r;
  if (group == ORC_GROUP_XOR) {
    r.lo = a.lo ^ b.lo;
    r.hi = a.hi ^ b.hi;
  } else {
    r.lo = a.lo + b.lo;
    r.hi = a.hi + b.hi + (r.lo < a.lo ? 1 : 0);
    r.hi &= MSB_CLEAR;
  }
  return r;
}
static u128p g_neg(int group, u128p a) {
  if (group == ORC_GROUP_XOR) return a;
  u128p r;
  r.lo = ~a.lo + 1;
  r.hi = ~a.hi + (r.lo == 0 ? 1 : 0);
  r.hi &= MSB_CLEAR;
  return r;
}
static u128p g_xor(u128p a, u128p b) {
  u128p r = {a.lo ^ b.lo, a.hi ^ b.hi};
  return r;
}
static int msb(u128p a) { return (int)(a.hi >> 63); }
static u128p clr(u128p a) {
  a.hi &= MSB_CLEAR;
  return a;
}
static int bit_le(const uint8_t* b, int i) { return (b[i >> 3] >> (i & 7)) & 1; }

void orc_prg_init(orc_prg_state* p, const uint8_t* state, int state_len) {
  (void)state_len;
  for (int i = 0; i < ORC_PRG_BLOCKS; i++) orc_aes128_expand(state + 16 * i, p->rk[i]);
}

void orc_prg(const orc_prg_state* p, uint8_t* out, int out_len, const uint8_t seed[16]) {
  if (orc_mmo_fast((const uint8_t(*)[176])p->rk, out_len / 16, seed, out)) return;
  for (int i = 0; i < out_len / 16; i++) {
    orc_aes128_encrypt(p->rk[i], seed, out + 16 * i);
    for (int j = 0; j < 16; j++) out[16 * i + j] ^= seed[j];
  }
}

/* PRG(s) -> (sl, vl, sr, vr) with t bits taken from the MSB of sl / sr
 * and the MSB of all four blocks cleared (dcf.c:23-28). */
static void expand(const orc_prg_state* p, u128p s, u128p out[4], int* tl, int* tr) {
  uint8_t sb[16], buf[64];
  st(sb, s);
  orc_prg(p, buf, 64, sb);
  for (int i = 0; i < 4; i++) out[i] = ld(buf + 16 * i);
  *tl = msb(out[0]);
  *tr = msb(out[2]);
  for (int i = 0; i < 4; i++) out[i] = clr(out[i]);
}

void orc_dcf_gen(const orc_prg_state* p, int group, int bitlen, const uint8_t* alpha_le,
                 const uint8_t beta_in[16], const uint8_t s0_in[16], const uint8_t s1_in[16],
                 uint8_t* cws, uint8_t cw_np1[16]) {
  u128p s0 = clr(ld(s0_in)), s1 = clr(ld(s1_in));
  int t0 = 0, t1 = 1;
  u128p v = {0, 0};
  u128p beta = clr(ld(beta_in));
  for (int i = 0; i < bitlen; i++) {
    u128p e0[4], e1[4];
    int t0l, t0r, t1l, t1r;
    expand(p, s0, e0, &t0l, &t0r);
    expand(p, s1, e1, &t1l, &t1r);
    int a = bit_le(alpha_le, bitlen - 1 - i);
    /* lose = the side alpha does not take; keep = the side it takes. */
    int lose = a ? 0 : 2, keep = a ? 2 : 0;
    u128p s_cw = g_xor(e0[lose], e1[lose]);
    u128p v_cw = g_add(group, e1[lose + 1], g_neg(group, e0[lose + 1]));
    v_cw = g_add(group, v_cw, g_neg(group, v));
    if (t1) v_cw = g_neg(group, v_cw);
    if (a) v_cw = g_add(group, v_cw, t1 ? g_neg(group, beta) : beta); /* kLtAlpha */
    v = g_add(group, v, g_neg(group, e1[keep + 1]));
    v = g_add(group, v, e0[keep + 1]);
    v = g_add(group, v, t1 ? g_neg(group, v_cw) : v_cw);
    int tl_cw = t0l ^ t1l ^ a ^ 1;
    int tr_cw = t0r ^ t1r ^ a;
    uint8_t* cw = cws + (size_t)i * ORC_DCF_CW_LEN;
    st(cw, s_cw);
    st(cw + 16, v_cw);
    cw[32] = (uint8_t)(tl_cw << 1 | tr_cw);
    int t0k = a ? t0r : t0l, t1k = a ? t1r : t1l, tcwk = a ? tr_cw : tl_cw;
    u128p s0n = e0[keep], s1n = e1[keep];
    if (t0) s0n = g_xor(s0n, s_cw);
    if (t1) s1n = g_xor(s1n, s_cw);
    s0 = s0n;
    s1 = s1n;
    t0 = t0 ? (t0k ^ tcwk) : t0k;
    t1 = t1 ? (t1k ^ tcwk) : t1k;
  }
  u128p last = g_add(group, s1, g_neg(group, s0));
  last = g_add(group, last, g_neg(group, v));
  if (t1) last = g_neg(group, last);
  st(cw_np1, last);
}

void orc_dcf_eval(const orc_prg_state* p, int group, int party, int bitlen, const uint8_t* x_le,
                  const uint8_t seed[16], const uint8_t* cws, const uint8_t cw_np1[16],
                  uint8_t out[16]) {
  u128p s = clr(ld(seed));
  int t = party;
  u128p v = {0, 0};
  for (int i = 0; i < bitlen; i++) {
    const uint8_t* cw = cws + (size_t)i * ORC_DCF_CW_LEN;
    u128p e[4];
    int tl, tr;
    expand(p, s, e, &tl, &tr);
    if (t) {
      u128p scw = ld(cw);
      e[0] = g_xor(e[0], scw);
      e[2] = g_xor(e[2], scw);
      tl ^= cw[32] >> 1;
      tr ^= cw[32] & 1;
    }
    int xi = bit_le(x_le, bitlen - 1 - i);
    u128p vd = xi ? e[3] : e[1];
    if (t) vd = g_add(group, vd, ld(cw + 16));
    if (party) vd = g_neg(group, vd);
    v = g_add(group, v, vd);
    s = xi ? e[2] : e[0];
    t = xi ? tr : tl;
  }
  if (t) s = g_add(group, s, ld(cw_np1));
  if (party) s = g_neg(group, s);
  v = g_add(group, v, s);
  st(out, v);
}

/* ---------------- myl7 adapter blob ---------------- */
size_t orc_myl7_key_bytes(int in_bits, int payload_len) {
  size_t chunks = (size_t)(payload_len + 15) / 16;
  return 8 + chunks * (16 + (size_t)in_bits * ORC_DCF_CW_LEN + 16);
}

static void le64(uint64_t x, uint8_t b[8]) {
  for (int i = 0; i < 8; i++) b[i] = (uint8_t)(x >> (8 * i));
}

int orc_myl7_gen(const orc_prg_state* p, int group, int in_bits, uint64_t alpha,
                 const uint8_t* payload, int payload_len, const uint8_t* seeds,
                 uint8_t* key0, uint8_t* key1) {
  if (in_bits <= 0 || in_bits > 64 || payload_len <= 0) return -1;
  int chunks = (payload_len + 15) / 16;
  if (chunks > 255) return -1;
  uint8_t alpha_le[8];
  if (in_bits < 64) alpha &= (1ULL << in_bits) - 1;
  le64(alpha, alpha_le);
  uint8_t* keys[2] = {key0, key1};
  for (int b = 0; b < 2; b++) {
    keys[b][0] = (uint8_t)in_bits;
    keys[b][1] = (uint8_t)chunks;
    keys[b][2] = (uint8_t)b;
    keys[b][3] = 0;
    for (int i = 0; i < 4; i++) keys[b][4 + i] = (uint8_t)((uint32_t)payload_len >> (8 * i));
  }
  size_t cwb = (size_t)in_bits * ORC_DCF_CW_LEN;
  size_t off = 8;
  for (int c = 0; c < chunks; c++) {
    uint8_t beta[16] = {0};
    int take = payload_len - 16 * c < 16 ? payload_len - 16 * c : 16;
    memcpy(beta, payload + 16 * c, (size_t)take);
    beta[15] &= 0x7F; /* myl7_fss_backend.hpp:180 */
    const uint8_t* s0 = seeds + 32 * c;
    const uint8_t* s1 = s0 + 16;
    orc_dcf_gen(p, group, in_bits, alpha_le, beta, s0, s1, key0 + off + 16, key0 + off + 16 + cwb);
    memcpy(key0 + off, s0, 16);
    memcpy(key1 + off, s1, 16);
    memcpy(key1 + off + 16, key0 + off + 16, cwb + 16);
    off += 16 + cwb + 16;
  }
  return 0;
}

int orc_myl7_eval(const orc_prg_state* p, int group, int in_bits, const uint8_t* key,
                  uint64_t x, uint8_t* out) {
  if (key[0] != in_bits) return -1;
  int chunks = key[1], party = key[2];
  if (party != 0 && party != 1) return -2;
  uint32_t plen = (uint32_t)key[4] | (uint32_t)key[5] << 8 | (uint32_t)key[6] << 16 |
                  (uint32_t)key[7] << 24;
  uint8_t x_le[8];
  if (in_bits < 64) x &= (1ULL << in_bits) - 1;
  le64(x, x_le);
  size_t cwb = (size_t)in_bits * ORC_DCF_CW_LEN;
  size_t off = 8, done = 0;
  for (int c = 0; c < chunks; c++) {
    uint8_t blk[16];
    orc_dcf_eval(p, group, party, in_bits, x_le, key + off, key + off + 16, key + off + 16 + cwb,
                 blk);
    size_t take = plen - done < 16 ? plen - done : 16;
    memcpy(out + done, blk, take);
    done += take;
    off += 16 + cwb + 16;
  }
  return 0;
}

int orc_myl7_eval_many_bit(const orc_prg_state* p, int group, int in_bits, size_t key_bytes,
                           const uint8_t* keys, const uint64_t* xs, size_t n,
                           uint8_t* out, int threads) {
  int bad = 0;
  (void)threads;
#pragma omp parallel for schedule(static) num_threads(orc_threads_or_default(threads)) reduction(| : bad)
  for (long i = 0; i < (long)n; i++) {
    uint8_t buf[4096];
    const uint8_t* k = keys + (size_t)i * key_bytes;
    uint32_t plen = (uint32_t)k[4] | (uint32_t)k[5] << 8 | (uint32_t)k[6] << 16 |
                    (uint32_t)k[7] << 24;
    if (plen > sizeof(buf) || orc_myl7_eval(p, group, in_bits, k, xs[i], buf) != 0) {
      bad |= 1;
      continue;
    }
    out[i] = (uint8_t)(buf[0] & 1u);
  }
  return bad ? -1 : 0;
}
