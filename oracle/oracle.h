/*
 * CPU oracle for the PFSS hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: only tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py may load it.
 * The product (suf_amd/, include/suf_hip.h) never links or calls it.
 *
 * Every function restates the reference algorithm in plain C; each
 * definition cites the reference file:line it follows (paths relative to
 * the ponyyuhan/SUF tree).  How each function is pinned:
 *   - AES-128: FIPS-197 Appendix B / C.1 vectors and OpenSSL libcrypto.
 *   - myl7 PRG + DCF gen/eval: byte-exact against the vendored myl7/fss
 *     v0.7.1 sources compiled unmodified into oracle/_ref (see
 *     oracle/build_ref.sh), against committed golden vectors made from that
 *     build, and against the closed form 1[x < alpha] by brute force.
 *   - interval LUT / packed compare: closed forms (reconstruction equals the
 *     payload row / the threshold bitmask), the FIPS-pinned AES, and
 *     std::mt19937_64 (10000th output of the default seed).
 *   - trunc / Beaver / Horner / row reductions: __int128 closed forms
 *     (x >> f, X*W mod 2^64, ...) in tests/test_oracle_*.py.
 *   - truncation gate (gates.c): two-party reconstruction equals x >> f
 *     (TR), the arithmetic shift (ARS) and the gap shift (GapARS) over
 *     random and edge-case inputs and masks; DCF keys via the pinned myl7
 *     functions above.
 */
#ifndef SUF_ORACLE_H
#define SUF_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- AES-128 (FIPS-197) ---------------- */
void orc_aes128_expand(const uint8_t key[16], uint8_t rk[176]);
void orc_aes128_encrypt(const uint8_t rk[176], const uint8_t in[16], uint8_t out[16]);
/* The same cipher on the x86 AES instructions when the CPU has them (else
 * orc_aes128_encrypt): orc_aes_use_ni(0 / 1) turns that path off / on,
 * orc_aes_ni_active() says which is in use.  orc_mmo_fast writes nb <= 8
 * MMO blocks AES_{rk[i]}(seed) ^ seed and returns 1, or returns 0 (nothing
 * written) when the AES instructions are off. */
int orc_aes_ni_available(void);
void orc_aes_use_ni(int on);
int orc_aes_ni_active(void);
void orc_aes128_encrypt_fast(const uint8_t rk[176], const uint8_t in[16], uint8_t out[16]);
int orc_mmo_fast(const uint8_t (*rk)[176], int nb, const uint8_t seed[16], uint8_t* out);
/* OpenMP threads of the per-element loops (n <= 0: all processors). */
void orc_set_threads(int n);
int orc_get_threads(void);
/* n when positive, else the current OpenMP default. */
int orc_threads_or_default(int n);
/* CTR block i = AES(le64(ctr_lo + i) || le64(ctr_hi)); out is [blocks][16]. */
void orc_aes128_ctr(const uint8_t rk[176], uint64_t ctr_lo, uint64_t ctr_hi,
                    size_t blocks, uint8_t* out);

/* ---------------- std::mt19937_64 ---------------- */
typedef struct {
  uint64_t mt[312];
  int idx;
} orc_mt64;
void orc_mt64_seed(orc_mt64* g, uint64_t seed);
uint64_t orc_mt64_next(orc_mt64* g);
void orc_mt64_fill(uint64_t seed, uint64_t* out, size_t n);

/* ---------------- myl7 PRG (AES-128 MMO, kBlocks = 8) ---------------- */
#define ORC_PRG_BLOCKS 8
typedef struct {
  uint8_t rk[ORC_PRG_BLOCKS][176];
} orc_prg_state;
void orc_prg_init(orc_prg_state* p, const uint8_t* state, int state_len);
void orc_prg(const orc_prg_state* p, uint8_t* out, int out_len, const uint8_t seed[16]);

/* ---------------- myl7 DCF (lambda = 16) ---------------- */
#define ORC_GROUP_XOR 0  /* src/group/bytes.c: XOR of 16 bytes          */
#define ORC_GROUP_ADD 1  /* src/group/u128_le.c: + mod 2^127, LE bytes  */
#define ORC_DCF_CW_LEN 33
void orc_dcf_gen(const orc_prg_state* p, int group, int bitlen, const uint8_t* alpha_le,
                 const uint8_t beta[16], const uint8_t s0[16], const uint8_t s1[16],
                 uint8_t* cws, uint8_t cw_np1[16]);
void orc_dcf_eval(const orc_prg_state* p, int group, int party, int bitlen, const uint8_t* x_le,
                  const uint8_t seed[16], const uint8_t* cws, const uint8_t cw_np1[16],
                  uint8_t out[16]);

/* myl7 adapter key blob (include/proto/myl7_fss_backend.hpp:131-213). */
size_t orc_myl7_key_bytes(int in_bits, int payload_len);
/* seeds: [num_chunks][2][16] (party-0 seed then party-1 seed per chunk). */
int orc_myl7_gen(const orc_prg_state* p, int group, int in_bits, uint64_t alpha,
                 const uint8_t* payload, int payload_len, const uint8_t* seeds,
                 uint8_t* key0, uint8_t* key1);
/* Writes payload_len bytes of the party's share. Returns 0 or <0 on a bad key. */
int orc_myl7_eval(const orc_prg_state* p, int group, int in_bits, const uint8_t* key,
                  uint64_t x, uint8_t* out);
/* eval_dcf_many_u64 (myl7_fss_backend.hpp:73-100): out[i] = share byte 0 & 1. */
int orc_myl7_eval_many_bit(const orc_prg_state* p, int group, int in_bits, size_t key_bytes,
                           const uint8_t* keys, const uint64_t* xs, size_t n,
                           uint8_t* out, int threads);

/* ---------------- reference GPU blob semantics (packed LT, interval LUT) ------- */
#define ORC_PACKED_HDR 208
#define ORC_LUT_HDR 216
void orc_seed_from_id(uint64_t id, uint64_t tweak, uint8_t seed[16]);
size_t orc_packed_key_bytes(int num_thr);
void orc_packed_build_key(int party, uint64_t nonce, int in_bits, const uint64_t* thr,
                          int num_thr, const uint8_t seed[16], uint8_t* blob);
void orc_packed_eval(const uint8_t* keys, size_t key_bytes, int broadcast,
                     const uint64_t* xs, size_t n, uint64_t* out);
size_t orc_lut_key_bytes(int intervals, int out_words);
void orc_lut_build_key(int party, uint64_t nonce, int in_bits, int out_words,
                       const uint64_t* cuts, int intervals, const uint64_t* payload,
                       const uint8_t seed[16], uint8_t* blob);
void orc_lut_eval(const uint8_t* keys, size_t key_bytes, int broadcast,
                  const uint64_t* xs, size_t n, uint64_t* out);
/* The same for elements idx0 .. idx0 + n - 1 of a larger batch (the keystream
 * counter depends on the element index). */
void orc_lut_eval_at(const uint8_t* keys, size_t key_bytes, int broadcast,
                     const uint64_t* xs, size_t n, size_t idx0, uint64_t* out);

/* ---------------- ring postprocessing (cuda/cuda_primitives.cu) ---------------- */
void orc_beaver_mul(int party, const uint64_t* a, const uint64_t* b, const uint64_t* c,
                    const uint64_t* d, const uint64_t* e, uint64_t* out, size_t n);
void orc_trunc_postproc(int party, int kind_gapars, int frac_bits, uint64_t r_hi_share,
                        uint64_t m_share, const uint64_t* hatx, const uint64_t* arith,
                        size_t arith_stride, int arith_idx, const uint64_t* bools,
                        size_t bool_stride, int carry_idx, int sign_idx, int wrap_idx,
                        uint64_t* out, size_t n);
void orc_horner_cubic(const uint64_t* x, const uint64_t* c0, const uint64_t* c1,
                      const uint64_t* c2, const uint64_t* c3, uint64_t* out, size_t n);
void orc_add_rout_aos(uint64_t* out, size_t elems, int out_words, const uint64_t* r_out,
                      int r_out_words);
void orc_row_broadcast_mul(int party, const uint64_t* A, const uint64_t* B_rows,
                           const uint64_t* C, const uint64_t* d, const uint64_t* e_rows,
                           int rows, int cols, const int* valid_lens, uint64_t* out);
void orc_row_sum(const uint64_t* mat, int rows, int cols, const int* valid_lens,
                 uint64_t* out);
void orc_row_sum_ragged(const uint64_t* vals, const int* row_offsets, int rows,
                        uint64_t* out);
void orc_row_variance(const uint64_t* mat, const uint64_t* mean, int rows, int cols,
                      const int* valid_lens, uint64_t* out);
uint64_t orc_beaver_scale(uint64_t acc, int has_scale, int64_t mul_const, int mul_shift);
void orc_beaver_matmul(int party, const uint64_t* D, const uint64_t* E, const uint64_t* A,
                       const uint64_t* B, const uint64_t* C, int batches, int M, int K,
                       int N, int w_transposed, int has_scale, int64_t mul_const,
                       int mul_shift, uint64_t* out, int threads);
void orc_matmul_public(const uint64_t* X, const int64_t* W, int M, int K, int N, uint64_t* Y);
void orc_row_mean(const uint64_t* mat, int rows, int cols, const int* valid_lens,
                  uint64_t* out);
void orc_open_add(const uint64_t* local, const uint64_t* remote, int eff_bits, uint64_t* out,
                  size_t n, int ring_bits, uint64_t ring_mask, int sign_extend);
void orc_pack_eff_bits(const uint64_t* in, int eff_bits, uint64_t* packed, size_t n);
void orc_unpack_eff_bits(const uint64_t* packed, int eff_bits, uint64_t* out, size_t n);

/* ---------------- truncation gate (oracle/gates.c) ---------------- */
#define ORC_TRUNC_TR 0     /* GateKind::FaithfulTR  */
#define ORC_TRUNC_ARS 1    /* GateKind::FaithfulARS */
#define ORC_TRUNC_GAPARS 2 /* GateKind::GapARS      */
#define ORC_TRUNC_RAND_WORDS 19
size_t orc_trunc_key_bytes(int kind, int frac_bits);
int orc_trunc_gen(const orc_prg_state* p, int kind, int frac_bits, const uint64_t* rnd,
                  uint8_t* key0, uint8_t* key1);
int orc_trunc_eval(const orc_prg_state* p, int kind, int frac_bits, const uint8_t* key,
                   const uint64_t* xhat, size_t n, uint64_t* y);

#ifdef __cplusplus
}
#endif
#endif
