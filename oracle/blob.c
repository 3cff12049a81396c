/*
 * Oracle: packed multi-threshold compare and interval LUT with AES-CTR masks,
 * following the reference CUDA backend's key blobs and its *kernel* counter
 * convention (the host fallback uses a different one and is not normative).
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 *   packed header  cuda/pfss_backend_gpu.cu:86-94 (packed, 208 bytes)
 *     [in_bits u16][num_thr u16][party u8][flags u8][2 pad][nonce u64]
 *     [seed 16][round_keys 176] then u64 thresholds (& in_bits mask)
 *     flags bit 0 = thresholds sorted (:257-288)
 *   LUT header     cuda/pfss_backend_gpu.cu:75-84 (alignas 8, 216 bytes)
 *     [in_bits u16][out_words u16][intervals u32][party u8][3 pad][4 pad]
 *     [nonce u64][seed 16][round_keys 176] then u64 cuts[intervals+1],
 *     u64 payload[intervals][out_words] (:223-255)
 *   seed           seed_from_id, cuda/pfss_backend_gpu.cu:189-194
 *   packed eval    cuda/pfss_kernels.cu:240-330: bit j of word w is
 *                  1[x < thr_{64w+j}]; words (w, w+1) are masked with the two
 *                  halves of AES(le64(nonce ^ idx<<32 ^ w/2) || 0^64);
 *                  party 0 holds the keystream, party 1 holds word ^ keystream
 *   LUT eval       cuda/pfss_kernels.cu:545-590: iv = (upper_bound over
 *                  cuts[0..intervals) of x) - 1 clamped to [0, intervals-1];
 *                  words (w, w+1) masked by AES(le64(nonce ^ idx<<32 ^
 *                  (iv*out_words + w)) || 0); party 0 = keystream,
 *                  party 1 = row - keystream (mod 2^64)
 */
#include "oracle.h"

#include <string.h>

static uint64_t mask_bits(int bits) {
  if (bits <= 0) return 0;
  if (bits >= 64) return ~0ULL;
  return (1ULL << bits) - 1;
}
static uint16_t ld16(const uint8_t* p) { return (uint16_t)(p[0] | p[1] << 8); }
static uint32_t ld32(const uint8_t* p) {
  return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}
static uint64_t ld64(const uint8_t* p) {
  uint64_t v;
  memcpy(&v, p, 8);
  return v;
}
static void st64(uint8_t* p, uint64_t v) { memcpy(p, &v, 8); }

static void keystream(const uint8_t* rk, uint64_t ctr, uint64_t* ks0, uint64_t* ks1) {
  uint8_t blk[16] = {0}, out[16];
  st64(blk, ctr);
  orc_aes128_encrypt_fast(rk, blk, out);
  *ks0 = ld64(out);
  *ks1 = ld64(out + 8);
}

void orc_seed_from_id(uint64_t id, uint64_t tweak, uint8_t seed[16]) {
  orc_mt64 g;
  orc_mt64_seed(&g, id ^ (tweak * 0x9e3779b97f4a7c15ULL));
  for (int i = 0; i < 16; i++) seed[i] = (uint8_t)(orc_mt64_next(&g) & 0xFF);
}

size_t orc_packed_key_bytes(int num_thr) { return ORC_PACKED_HDR + 8 * (size_t)num_thr; }

void orc_packed_build_key(int party, uint64_t nonce, int in_bits, const uint64_t* thr,
                          int num_thr, const uint8_t seed[16], uint8_t* blob) {
  memset(blob, 0, ORC_PACKED_HDR);
  blob[0] = (uint8_t)in_bits;
  blob[1] = (uint8_t)(in_bits >> 8);
  blob[2] = (uint8_t)num_thr;
  blob[3] = (uint8_t)(num_thr >> 8);
  blob[4] = (uint8_t)party;
  st64(blob + 8, nonce);
  memcpy(blob + 16, seed, 16);
  orc_aes128_expand(seed, blob + 32);
  uint64_t m = mask_bits(in_bits);
  int sorted = 1;
  for (int i = 0; i < num_thr; i++) {
    uint64_t v = thr[i] & m;
    st64(blob + ORC_PACKED_HDR + 8 * (size_t)i, v);
    if (i > 0 && v < (thr[i - 1] & m)) sorted = 0;
  }
  blob[5] = (uint8_t)sorted;
}

void orc_packed_eval(const uint8_t* keys, size_t key_bytes, int broadcast,
                     const uint64_t* xs, size_t n, uint64_t* out) {
#pragma omp parallel for schedule(static)
  for (size_t idx = 0; idx < n; idx++) {
    const uint8_t* k = broadcast ? keys : keys + idx * key_bytes;
    int in_bits = ld16(k), num_thr = ld16(k + 2), party = k[4];
    uint64_t nonce = ld64(k + 8);
    const uint8_t* rk = k + 32;
    const uint8_t* thr = k + ORC_PACKED_HDR;
    int out_words = (num_thr + 63) / 64;
    uint64_t m = mask_bits(in_bits);
    uint64_t x = xs[idx] & m;
    for (int w = 0; w < out_words; w += 2) {
      uint64_t word[2] = {0, 0};
      for (int h = 0; h < 2 && w + h < out_words; h++) {
        int base = 64 * (w + h);
        for (int b = base; b < base + 64 && b < num_thr; b++)
          if (x < (ld64(thr + 8 * (size_t)b) & m)) word[h] |= 1ULL << (b - base);
      }
      uint64_t ks[2];
      keystream(rk, nonce ^ ((uint64_t)idx << 32) ^ (uint64_t)(w / 2), &ks[0], &ks[1]);
      for (int h = 0; h < 2 && w + h < out_words; h++)
        out[idx * (size_t)out_words + (size_t)(w + h)] = party == 0 ? ks[h] : (word[h] ^ ks[h]);
    }
  }
}

size_t orc_lut_key_bytes(int intervals, int out_words) {
  return ORC_LUT_HDR + 8 * (size_t)(intervals + 1) + 8 * (size_t)intervals * (size_t)out_words;
}

void orc_lut_build_key(int party, uint64_t nonce, int in_bits, int out_words,
                       const uint64_t* cuts, int intervals, const uint64_t* payload,
                       const uint8_t seed[16], uint8_t* blob) {
  memset(blob, 0, ORC_LUT_HDR);
  blob[0] = (uint8_t)in_bits;
  blob[1] = (uint8_t)(in_bits >> 8);
  blob[2] = (uint8_t)out_words;
  blob[3] = (uint8_t)(out_words >> 8);
  for (int i = 0; i < 4; i++) blob[4 + i] = (uint8_t)((uint32_t)intervals >> (8 * i));
  blob[8] = (uint8_t)party;
  st64(blob + 16, nonce);
  memcpy(blob + 24, seed, 16);
  orc_aes128_expand(seed, blob + 40);
  for (int i = 0; i <= intervals; i++) st64(blob + ORC_LUT_HDR + 8 * (size_t)i, cuts[i]);
  uint8_t* pay = blob + ORC_LUT_HDR + 8 * (size_t)(intervals + 1);
  for (size_t i = 0; i < (size_t)intervals * (size_t)out_words; i++) st64(pay + 8 * i, payload[i]);
}

void orc_lut_eval(const uint8_t* keys, size_t key_bytes, int broadcast,
                  const uint64_t* xs, size_t n, uint64_t* out) {
  orc_lut_eval_at(keys, key_bytes, broadcast, xs, n, 0, out);
}

/* Elements idx0 .. idx0 + n - 1 of a batch: the keystream counter uses the
 * element's index in the whole batch. */
void orc_lut_eval_at(const uint8_t* keys, size_t key_bytes, int broadcast,
                     const uint64_t* xs, size_t n, size_t idx0, uint64_t* out) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; i++) {
    const size_t idx = idx0 + i;
    const uint8_t* k = broadcast ? keys : keys + i * key_bytes;
    int in_bits = ld16(k), out_words = ld16(k + 2);
    int intervals = (int)ld32(k + 4), party = k[8];
    uint64_t nonce = ld64(k + 16);
    const uint8_t* rk = k + 40;
    const uint8_t* cuts = k + ORC_LUT_HDR;
    const uint8_t* pay = cuts + 8 * (size_t)(intervals + 1);
    uint64_t m = mask_bits(in_bits);
    uint64_t x = xs[i] & m;
    int iv = intervals - 1;
    if (intervals > 1) {
      int lo = 0, hi = intervals;
      while (lo < hi) {
        int mid = (lo + hi) >> 1;
        if ((ld64(cuts + 8 * (size_t)mid) & m) <= x) lo = mid + 1;
        else hi = mid;
      }
      iv = lo - 1;
      if (iv < 0) iv = 0;
      if (iv >= intervals) iv = intervals - 1;
    }
    const uint8_t* row = pay + 8 * (size_t)iv * (size_t)out_words;
    for (int w = 0; w < out_words; w += 2) {
      uint64_t ks[2];
      uint64_t ctr = nonce ^ ((uint64_t)idx << 32) ^ ((uint64_t)iv * (uint64_t)out_words + (uint64_t)w);
      keystream(rk, ctr, &ks[0], &ks[1]);
      for (int h = 0; h < 2 && w + h < out_words; h++) {
        uint64_t r = ld64(row + 8 * (size_t)(w + h));
        out[i * (size_t)out_words + (size_t)(w + h)] = party == 0 ? ks[h] : r - ks[h];
      }
    }
  }
}
