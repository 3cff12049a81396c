/*
 * Oracle: AES-128 and std::mt19937_64, written from their specifications.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * AES-128 follows FIPS-197 section 5 literally: the S-box is derived from
 * its definition (inverse in GF(2^8) followed by the affine map with 0x63),
 * the state is column-major bytes, and encryption is
 * AddRoundKey, 9 x (SubBytes, ShiftRows, MixColumns, AddRoundKey),
 * SubBytes, ShiftRows, AddRoundKey.  The reference uses the same cipher as
 * OpenSSL EVP_aes_128_ecb (third_party/myl7_fss/src/prg/aes128_mmo.c:16-52)
 * and as a T-table device function (cuda/pfss_kernels.cu:112-165) with the
 * key schedule of cuda/pfss_backend_gpu.cu:165-187.
 *
 * mt19937_64 follows the C++ standard [rand.eng.mers] parameters
 * (w=64, n=312, m=156, r=31, a=0xb5026f5aa96619e9, u=29, d=0x5555555555555555,
 * s=17, b=0x71d67fffeda60000, t=37, c=0xfff7eee000000000, l=43,
 * f=6364136223846793005); the reference seeds blob keys with it
 * (cuda/pfss_backend_gpu.cu:189-194).
 */
#include "oracle.h"

#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__x86_64__)
#include <immintrin.h>
#endif

static uint8_t g_sbox[256];
static int g_sbox_ready = 0;

static uint8_t gf_mul(uint8_t a, uint8_t b) {
  uint8_t r = 0;
  while (b) {
    if (b & 1) r ^= a;
    a = (uint8_t)((a << 1) ^ ((a & 0x80) ? 0x1b : 0));
    b >>= 1;
  }
  return r;
}

static uint8_t gf_inv(uint8_t a) {
  /* a^254 = a^-1 in GF(2^8) (0 maps to 0). */
  uint8_t r = 1, base = a;
  int e = 254;
  while (e) {
    if (e & 1) r = gf_mul(r, base);
    base = gf_mul(base, base);
    e >>= 1;
  }
  return a ? r : 0;
}

static void build_sbox(void) {
  if (g_sbox_ready) return;
  for (int x = 0; x < 256; x++) {
    uint8_t b = gf_inv((uint8_t)x);
    uint8_t s = 0x63;
    for (int i = 0; i < 8; i++) {
      int bit = ((b >> i) ^ (b >> ((i + 4) & 7)) ^ (b >> ((i + 5) & 7)) ^
                 (b >> ((i + 6) & 7)) ^ (b >> ((i + 7) & 7))) & 1;
      s ^= (uint8_t)(bit << i);
    }
    g_sbox[x] = s;
  }
  g_sbox_ready = 1;
}

/* The S-box is built before any caller's threads start. */
__attribute__((constructor)) static void init_sbox(void) { build_sbox(); }

void orc_aes128_expand(const uint8_t key[16], uint8_t rk[176]) {
  build_sbox();
  memcpy(rk, key, 16);
  uint8_t rcon = 1;
  for (int w = 4; w < 44; w++) {
    uint8_t t[4];
    memcpy(t, rk + 4 * (w - 1), 4);
    if (w % 4 == 0) {
      uint8_t r0 = t[0];
      t[0] = (uint8_t)(g_sbox[t[1]] ^ rcon);
      t[1] = g_sbox[t[2]];
      t[2] = g_sbox[t[3]];
      t[3] = g_sbox[r0];
      rcon = gf_mul(rcon, 2);
    }
    for (int i = 0; i < 4; i++) rk[4 * w + i] = (uint8_t)(rk[4 * (w - 4) + i] ^ t[i]);
  }
}

void orc_aes128_encrypt(const uint8_t rk[176], const uint8_t in[16], uint8_t out[16]) {
  build_sbox();
  uint8_t s[16];
  for (int i = 0; i < 16; i++) s[i] = (uint8_t)(in[i] ^ rk[i]);
  for (int round = 1; round <= 10; round++) {
    uint8_t u[16];
    /* SubBytes + ShiftRows: row r of column c takes column (c + r) mod 4. */
    for (int c = 0; c < 4; c++)
      for (int r = 0; r < 4; r++) u[4 * c + r] = g_sbox[s[4 * ((c + r) & 3) + r]];
    if (round < 10) {
      for (int c = 0; c < 4; c++) {
        uint8_t a0 = u[4 * c], a1 = u[4 * c + 1], a2 = u[4 * c + 2], a3 = u[4 * c + 3];
        u[4 * c + 0] = (uint8_t)(gf_mul(a0, 2) ^ gf_mul(a1, 3) ^ a2 ^ a3);
        u[4 * c + 1] = (uint8_t)(a0 ^ gf_mul(a1, 2) ^ gf_mul(a2, 3) ^ a3);
        u[4 * c + 2] = (uint8_t)(a0 ^ a1 ^ gf_mul(a2, 2) ^ gf_mul(a3, 3));
        u[4 * c + 3] = (uint8_t)(gf_mul(a0, 3) ^ a1 ^ a2 ^ gf_mul(a3, 2));
      }
    }
    for (int i = 0; i < 16; i++) s[i] = (uint8_t)(u[i] ^ rk[16 * round + i]);
  }
  memcpy(out, s, 16);
}

/* The same cipher on the x86 AES instructions (Intel's AES-NI: AESENC runs
 * SubBytes, ShiftRows, MixColumns and AddRoundKey of one middle round,
 * AESENCLAST the final round), taking the FIPS-197 key schedule above as
 * sixteen-byte round keys.  It is used when the CPU has the instructions and
 * not disabled by orc_aes_use_ni(0); tests/test_oracle_aes.py checks it
 * byte for byte against orc_aes128_encrypt. */
static int g_ni = -1; /* -1: not yet probed */

int orc_aes_ni_available(void) {
#if defined(__x86_64__)
  __builtin_cpu_init();
  return __builtin_cpu_supports("aes") ? 1 : 0;
#else
  return 0;
#endif
}

void orc_aes_use_ni(int on) { g_ni = on ? orc_aes_ni_available() : 0; }

int orc_aes_ni_active(void) {
  if (g_ni < 0) g_ni = orc_aes_ni_available();
  return g_ni;
}

#if defined(__x86_64__)
__attribute__((target("aes,sse2"))) static void ni_encrypt(const uint8_t rk[176],
                                                            const uint8_t in[16],
                                                            uint8_t out[16]) {
  __m128i s = _mm_xor_si128(_mm_loadu_si128((const __m128i*)in),
                            _mm_loadu_si128((const __m128i*)rk));
  for (int r = 1; r < 10; r++) s = _mm_aesenc_si128(s, _mm_loadu_si128((const __m128i*)(rk + 16 * r)));
  s = _mm_aesenclast_si128(s, _mm_loadu_si128((const __m128i*)(rk + 160)));
  _mm_storeu_si128((__m128i*)out, s);
}

/* MMO blocks out[i] = AES_{rk[i]}(seed) xor seed for i < nb <= 8, the blocks'
 * rounds interleaved. */
__attribute__((target("aes,sse2"))) static void ni_mmo(const uint8_t (*rk)[176], int nb,
                                                        const uint8_t seed[16], uint8_t* out) {
  const __m128i sd = _mm_loadu_si128((const __m128i*)seed);
  __m128i s[8];
  for (int i = 0; i < nb; i++) s[i] = _mm_xor_si128(sd, _mm_loadu_si128((const __m128i*)rk[i]));
  for (int r = 1; r < 10; r++)
    for (int i = 0; i < nb; i++)
      s[i] = _mm_aesenc_si128(s[i], _mm_loadu_si128((const __m128i*)(rk[i] + 16 * r)));
  for (int i = 0; i < nb; i++) {
    s[i] = _mm_aesenclast_si128(s[i], _mm_loadu_si128((const __m128i*)(rk[i] + 160)));
    _mm_storeu_si128((__m128i*)(out + 16 * i), _mm_xor_si128(s[i], sd));
  }
}
#endif

void orc_aes128_encrypt_fast(const uint8_t rk[176], const uint8_t in[16], uint8_t out[16]) {
#if defined(__x86_64__)
  if (orc_aes_ni_active()) {
    ni_encrypt(rk, in, out);
    return;
  }
#endif
  orc_aes128_encrypt(rk, in, out);
}

int orc_mmo_fast(const uint8_t (*rk)[176], int nb, const uint8_t seed[16], uint8_t* out) {
#if defined(__x86_64__)
  if (nb <= 8 && orc_aes_ni_active()) {
    ni_mmo(rk, nb, seed, out);
    return 1;
  }
#endif
  (void)rk;
  (void)nb;
  (void)seed;
  (void)out;
  return 0;
}

void orc_set_threads(int n) {
#ifdef _OPENMP
  omp_set_num_threads(n > 0 ? n : omp_get_num_procs());
#else
  (void)n;
#endif
}

int orc_threads_or_default(int n) { return n > 0 ? n : orc_get_threads(); }

int orc_get_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void orc_aes128_ctr(const uint8_t rk[176], uint64_t ctr_lo, uint64_t ctr_hi,
                    size_t blocks, uint8_t* out) {
  /* Counter layout of cuda/pfss_kernels.cu:169-184 (test_cuda_prg.cpp:28-34). */
  for (size_t i = 0; i < blocks; i++) {
    uint8_t blk[16];
    uint64_t c = ctr_lo + (uint64_t)i;
    for (int j = 0; j < 8; j++) blk[j] = (uint8_t)(c >> (8 * j));
    for (int j = 0; j < 8; j++) blk[8 + j] = (uint8_t)(ctr_hi >> (8 * j));
    orc_aes128_encrypt(rk, blk, out + 16 * i);
  }
}

/* ---------------- mt19937_64 ---------------- */
void orc_mt64_seed(orc_mt64* g, uint64_t seed) {
  g->mt[0] = seed;
  for (int i = 1; i < 312; i++)
    g->mt[i] = 6364136223846793005ULL * (g->mt[i - 1] ^ (g->mt[i - 1] >> 62)) + (uint64_t)i;
  g->idx = 312;
}

uint64_t orc_mt64_next(orc_mt64* g) {
  const uint64_t upper = 0xFFFFFFFF80000000ULL, lower = 0x7FFFFFFFULL;
  if (g->idx >= 312) {
    for (int i = 0; i < 312; i++) {
      uint64_t y = (g->mt[i] & upper) | (g->mt[(i + 1) % 312] & lower);
      uint64_t v = g->mt[(i + 156) % 312] ^ (y >> 1);
      if (y & 1) v ^= 0xB5026F5AA96619E9ULL;
      g->mt[i] = v;
    }
    g->idx = 0;
  }
  uint64_t z = g->mt[g->idx++];
  z ^= (z >> 29) & 0x5555555555555555ULL;
  z ^= (z << 17) & 0x71D67FFFEDA60000ULL;
  z ^= (z << 37) & 0xFFF7EEE000000000ULL;
  z ^= z >> 43;
  return z;
}

void orc_mt64_fill(uint64_t seed, uint64_t* out, size_t n) {
  orc_mt64 g;
  orc_mt64_seed(&g, seed);
  for (size_t i = 0; i < n; i++) out[i] = orc_mt64_next(&g);
}
