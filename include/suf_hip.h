/*
 * suf_hip.h -- C ABI of libsuf_hip.so, the MI355X (gfx950) PFSS execution
 * backend for SUF.
 *
 * This header replaces the reference's GPU boundary:
 *   - cuda/pfss_cuda_api.hpp:6-24 (a 4-function C API whose bodies are stubs,
 *     cuda/pfss_kernels.cu:814-830) -> the sufhip_dcf_* / sufhip_packed_lt_* /
 *     sufhip_interval_lut_* evaluators below;
 *   - the device entry points of proto::PfssGpuStagedEval
 *     (include/proto/backend_gpu.hpp:157-210), whose CUDA bodies live in
 *     cuda/pfss_backend_gpu.cu:523-1378;
 *   - the extern "C" launcher set of include/runtime/cuda_primitives.hpp:13-236.
 *
 * Conventions (all entry points):
 *   - Plain pointers and sizes; no HIP or torch types.  `stream` is a
 *     hipStream_t passed as void* (NULL = the default stream).
 *   - Pointers named d_* are device pointers; all other pointers are host.
 *   - Every function returns SUFHIP_OK (0) or a negative status; the message
 *     of the last failure on the calling thread is sufhip_last_error().
 *     The reference launchers return void and silently do nothing for n == 0;
 *     here n == 0 is also a successful no-op.
 *   - Work is enqueued asynchronously on `stream` unless stated otherwise.
 *   - Ring arithmetic is over Z_2^64 (unsigned wrap-around).
 */
#ifndef SUF_HIP_H
#define SUF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SUFHIP_OK 0
#define SUFHIP_ERR_INVALID (-1) /* bad argument: size, null pointer, tag */
#define SUFHIP_ERR_HIP (-2)     /* HIP runtime error (launch, copy, sync) */
#define SUFHIP_ERR_NOMEM (-3)   /* device allocation failed */

#define SUFHIP_ABI_VERSION 1

/* DCF output groups (myl7/fss v0.7.1 src/group/): */
#define SUFHIP_GROUP_XOR 0 /* bytes.c: XOR of 16-byte blocks (the group SUF links) */
#define SUFHIP_GROUP_ADD 1 /* u128_le.c: addition mod 2^127 of little-endian blocks */

/* DCF output modes for sufhip_dcf_eval: */
#define SUFHIP_DCF_OUT_BIT 0    /* 1 byte per element: share byte 0 & 1
                                   (Myl7FssBackend::eval_dcf_many_u64,
                                   include/proto/myl7_fss_backend.hpp:73-100) */
#define SUFHIP_DCF_OUT_BYTES 1  /* out_bytes bytes per element: the first
                                   out_bytes bytes of the payload share
                                   (PfssBackendBatch::eval_dcf_many_u64 with
                                   outs_flat [N][out_bytes]) */
#define SUFHIP_DCF_OUT_PACKED 2 /* one bit per element: bit (i % 64) of u64
                                   word i / 64 is share byte 0 & 1 of element i */

/* ---------------------------------------------------------------------- */
/* Library and runtime plumbing (lets C++ host code manage device memory   */
/* and streams without including HIP headers).                             */
/* ---------------------------------------------------------------------- */
int sufhip_abi_version(void);
const char* sufhip_last_error(void);
/* Selects the device for the calling thread and loads the kernels. */
int sufhip_init(int device);
/* Keystream policy of the two-party LUT evaluations (gate chains, the
 * softmax and LayerNorm blocks, the max tree).  SUF's dealer gives both
 * parties of a LUT gate one AES key (seed_from_id,
 * cuda/pfss_backend_gpu.cu:508-515), so with both parties in one process a
 * kernel can compute each keystream block once for both (per_party = 0, the
 * default; used only where the two blobs' keys, nonce, mask and cut points
 * compare equal on the device).  per_party = 1 makes every kernel compute
 * each party's keystream and interval search from that party's own blob, as
 * two parties in separate processes do: the same shares, the two-process
 * cost.  Process-wide; read when a launch is issued, so a captured HIP graph
 * keeps the policy it was captured with.  No counterpart in the reference
 * (its parties never share a process). */
int sufhip_set_keystream_per_party(int per_party);
int sufhip_keystream_per_party(void);
int sufhip_device_count(int* count);
int sufhip_stream_create(void** stream);
int sufhip_stream_destroy(void* stream);
int sufhip_stream_synchronize(void* stream);
int sufhip_malloc(void** d_ptr, size_t bytes);
int sufhip_free(void* d_ptr);
int sufhip_host_alloc(void** h_ptr, size_t bytes); /* pinned host memory */
int sufhip_host_free(void* h_ptr);
int sufhip_memcpy_h2d(void* d_dst, const void* src, size_t bytes, void* stream);
int sufhip_memcpy_d2h(void* dst, const void* d_src, size_t bytes, void* stream);
int sufhip_memcpy_d2d(void* d_dst, const void* d_src, size_t bytes, void* stream);

/* Timed region helpers: records an event pair around nothing; the caller
 * records `start` and `stop` on the stream and reads the elapsed ms. */
int sufhip_event_create(void** ev);
int sufhip_event_destroy(void* ev);
int sufhip_event_record(void* ev, void* stream);
int sufhip_event_elapsed_ms(void* start, void* stop, float* ms);
/* Blocks the calling thread until the recorded work of `ev` has completed. */
int sufhip_event_synchronize(void* ev);

/* ---------------------------------------------------------------------- */
/* AES-128 and the myl7 PRG                                                 */
/* ---------------------------------------------------------------------- */
/* AES-128-CTR keystream: block i = AES_k(le64(ctr_lo + i) || le64(ctr_hi)).
 * Replaces the aes128_ctr_kernel launch of src/demo/test_cuda_prg.cpp:93
 * (kernel cuda/pfss_kernels.cu:169-184).  round_keys: 176 bytes (FIPS-197
 * key schedule); d_out: [blocks][16]. */
int sufhip_aes128_ctr(uint8_t* d_out, const uint8_t* round_keys, uint64_t ctr_lo,
                      uint64_t ctr_hi, size_t blocks, void* stream);
/* The same keystream (the same reference kernel replaced) computed bitsliced
 * on the VALU: 32 counter blocks per lane as 128 32-bit slices, the S-box as
 * tower-field inversion and affine map, no tables; d_out 16-byte aligned.
 * It is the measured alternative to the LDS T-table AES that every other
 * kernel uses (the DCF profile compares the two by counters). */
int sufhip_aes128_ctr_bitsliced(uint8_t* d_out, const uint8_t* round_keys, uint64_t ctr_lo,
                                uint64_t ctr_hi, size_t blocks, void* stream);

/* myl7 PRG (third_party/myl7_fss/src/prg/aes128_mmo.c:41-52) on n seeds:
 * d_out[i][16 j .. 16 j + 16) = AES_{K_j}(seed_i) xor seed_i, j < out_blocks
 * (out_blocks <= 8), K_j = prg_state[16 j .. 16 j + 16). */
int sufhip_prg_mmo(const uint8_t* prg_state, const uint8_t* d_seeds, size_t n, int out_blocks,
                   uint8_t* d_out, void* stream);

/* ---------------------------------------------------------------------- */
/* DCF in the myl7 adapter key format                                       */
/* (include/proto/myl7_fss_backend.hpp:131-213):                            */
/*   [in_bits u8][num_chunks u8][party u8][0][payload_len u32 LE]           */
/*   then per 16-byte payload chunk: [seed 16][cw 33 x in_bits][cw_np1 16]  */
/* Keys are flat [N][key_bytes]; `key_broadcast` = 1 means one key for all  */
/* N points (PfssGpuStagedEval::*_broadcast, backend_gpu.hpp:166-175).      */
/* prg_state is the 128-byte myl7 PRG state (prg_init, aes128_mmo.c:16-31). */
/* ---------------------------------------------------------------------- */
size_t sufhip_dcf_key_bytes(int in_bits, int payload_len);

/* Dealer: N comparison keys f_i(x) = payload_i * 1[x < alpha_i] on in_bits
 * bits (myl7 dcf_gen, third_party/myl7_fss/src/dcf.c:42-142, via
 * Myl7FssBackend::gen_dcf, myl7_fss_backend.hpp:134-213).
 * d_alpha [N] u64; d_payload [payload_len] (payload_broadcast = 1) or
 * [N][payload_len]; d_seeds [N][num_chunks][2][16] (party-0 then party-1
 * seed of each chunk).  Writes d_keys0, d_keys1 [N][key_bytes]. */
int sufhip_dcf_gen(int group, int in_bits, const uint8_t* prg_state, const uint64_t* d_alpha,
                   const uint8_t* d_payload, int payload_len, int payload_broadcast,
                   const uint8_t* d_seeds, size_t n, uint8_t* d_keys0, uint8_t* d_keys1,
                   void* stream);

/* Evaluator: one party's shares at N points (myl7 dcf_eval, dcf.c:146-193;
 * Myl7FssBackend::eval_dcf / eval_dcf_many_u64, myl7_fss_backend.hpp:73-100,
 * 215-256; PfssGpuStagedEval::eval_dcf_many_u64_device[_broadcast],
 * backend_gpu.hpp:159-175).  The party is read from each key's header.
 * key_bytes must equal sufhip_dcf_key_bytes(in_bits, payload_len).
 * out_mode SUFHIP_DCF_OUT_BIT: d_out [N] bytes; SUFHIP_DCF_OUT_BYTES:
 * d_out [N][out_bytes], 1 <= out_bytes <= payload_len;
 * SUFHIP_DCF_OUT_PACKED: d_out [ceil(N/64)] u64 words. */
int sufhip_dcf_eval(int group, int in_bits, int payload_len, const uint8_t* prg_state,
                    const uint8_t* d_keys, size_t key_bytes, int key_broadcast,
                    const uint64_t* d_xs, size_t n, int out_mode, int out_bytes, void* d_out,
                    void* stream);

/* ---------------------------------------------------------------------- */
/* Truncation gate (one instance, scalar input mask r), both halves of SUF's */
/* trunc pipeline: keygen composite_gen_trunc_gate                           */
/* (include/gates/composite_fss.hpp:645-833) and the online evaluation that  */
/* SUF runs as composite_eval_batch_backend's AddU64 branch                  */
/* (composite_fss.hpp:1385-1638) followed by the trunc postproc hook         */
/* (include/gates/postproc_hooks.hpp:172-373; launch_trunc_postproc_kernel,  */
/* include/runtime/cuda_primitives.hpp:47-63).                               */
/* Keys are device blobs (8-byte aligned): a 64-byte header (tag "STG1",     */
/* kind, frac_bits, party, key flags, shares of r_in, r_hi, r_out, the       */
/* carry / sign rotation bits and GapARS's m) followed by the f-bit carry    */
/* DCF key and, for TR / ARS, the 64-bit wrap (and ARS sign) DCF keys, all   */
/* in the myl7 adapter format with an 8-byte additive payload.               */
/* ---------------------------------------------------------------------- */
#define SUFHIP_TRUNC_TR 0     /* GateKind::FaithfulTR  */
#define SUFHIP_TRUNC_ARS 1    /* GateKind::FaithfulARS */
#define SUFHIP_TRUNC_GAPARS 2 /* GateKind::GapARS      */
#define SUFHIP_TRUNC_RAND_WORDS 19

/* 0 for an unknown kind or frac_bits outside [1, 62]. */
size_t sufhip_trunc_key_bytes(int kind, int frac_bits);

/* Dealer: both parties' keys for one gate.  rnd: SUFHIP_TRUNC_RAND_WORDS
 * host u64 words at fixed positions: 0 r | 1 r_in split | 2 r_out split |
 * 3 carry-rotation split | 4 sign-rotation split | 5 r_hi split | 6 m split |
 * 7..10, 11..14, 15..18 seeds of the carry, wrap and sign DCF keys (party-0
 * seed = words 0,1 LE; party-1 seed = words 2,3).  A split of v gives party 0
 * the word s and party 1 v - s.  Writes d_key0, d_key1
 * [sufhip_trunc_key_bytes(kind, frac_bits)]. */
int sufhip_trunc_gen(int kind, int frac_bits, const uint8_t* prg_state, const uint64_t* rnd,
                     uint8_t* d_key0, uint8_t* d_key1, void* stream);

/* Device workspace sufhip_trunc_eval needs for N points (0 = none). */
size_t sufhip_trunc_work_bytes(int frac_bits, size_t n);

/* One party: d_y[i] = this party's share of trunc(x_i) given the public
 * d_xhat[i] = x_i + r.  kind / frac_bits must be the ones the key was made
 * with; the party is read from the key.  d_work: >= sufhip_trunc_work_bytes
 * bytes, 16-byte aligned, clobbered.  Equals sufhip_trunc_prepare followed
 * by sufhip_trunc_finish on the same stream. */
int sufhip_trunc_eval(int kind, int frac_bits, const uint8_t* prg_state, const uint8_t* d_key,
                      size_t key_bytes, const uint64_t* d_xhat, size_t n, uint64_t* d_y,
                      void* d_work, size_t work_bytes, void* stream);
/* sufhip_trunc_eval without a workspace argument and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  The carry frontier lives in a static per-GPU array
 * of sufhip_trunc_noalloc_max_work_bytes() = 1 MiB: enough for any n when
 * frac_bits <= 14, and for n < 2^16 above that; a (frac_bits, n) whose
 * sufhip_trunc_work_bytes() exceeds it is rejected with SUFHIP_ERR_INVALID.
 * Every call on one GPU uses that GPU's one array, which keeps the last
 * call's contents: calls that overlap on one GPU (other streams, other host
 * threads) race and must be serialised by the caller.  Same shares as
 * sufhip_trunc_eval. */
size_t sufhip_trunc_noalloc_max_work_bytes(void);
int sufhip_trunc_eval_noalloc(int kind, int frac_bits, const uint8_t* prg_state,
                              const uint8_t* d_key, size_t key_bytes, const uint64_t* d_xhat,
                              size_t n, uint64_t* d_y, void* stream);
/* The two halves of sufhip_trunc_eval.  prepare reads only the key (it fills
 * d_work with the carry DCF's prefix frontier for a batch of n points), so a
 * caller may run it before the inputs exist, e.g. on another stream while
 * earlier rounds execute; finish needs the same n, key and d_work. */
int sufhip_trunc_prepare(int kind, int frac_bits, const uint8_t* prg_state, const uint8_t* d_key,
                         size_t key_bytes, size_t n, void* d_work, size_t work_bytes,
                         void* stream);
int sufhip_trunc_finish(int kind, int frac_bits, const uint8_t* prg_state, const uint8_t* d_key,
                        size_t key_bytes, const uint64_t* d_xhat, size_t n, uint64_t* d_y,
                        const void* d_work, size_t work_bytes, void* stream);

/* Both parties' finish in one launch (keys d_key0 / d_key1 of the same gate,
 * each with the workspace its prepare filled); the same shares as two
 * sufhip_trunc_finish calls. */
int sufhip_trunc_finish2(int kind, int frac_bits, const uint8_t* prg_state, const uint8_t* d_key0,
                         const uint8_t* d_key1, size_t key_bytes, const uint64_t* d_xhat, size_t n,
                         uint64_t* d_y0, uint64_t* d_y1, const void* d_work0,
                         const void* d_work1, size_t work_bytes, void* stream);

/* The key-only halves of many gates (any kinds, widths and batch sizes) in
 * one walk launch plus one launch per level expanded beyond depth 12; each
 * job's workspace ends as sufhip_trunc_prepare would leave it.  For
 * frac_bits <= 14 the workspace holds the full-domain table of the carry
 * share, so the finish is one table read per element. */
typedef struct sufhip_trunc_job {
  int kind;
  int frac_bits;
  const uint8_t* d_key;
  size_t key_bytes;
  size_t n;
  void* d_work;
  size_t work_bytes;
} sufhip_trunc_job;
int sufhip_trunc_prepare_batch(const uint8_t* prg_state, const sufhip_trunc_job* jobs, int count,
                               void* stream);

/* A truncation folded into the launch that produces its masked open: for a
 * GapARS gate with frac_bits <= 14 whose keys were prepared (full-domain
 * tables), y[p][i] receives party p's truncated share at the open value
 * (plus add[p][i] when add is given: a residual folded into the same write)
 * instead of the open being written.  key / table: both parties' key blobs
 * (8-byte aligned) and prepared workspaces (16-byte aligned) of
 * work_bytes >= sufhip_trunc_work_bytes(frac_bits, n) each.  A key that is
 * not a GapARS key for frac_bits yields zeros.  The whole-chain and block
 * entry points take no addend. */
typedef struct sufhip_trunc_epilogue {
  const uint8_t* key[2];
  const void* table[2];
  size_t work_bytes;
  int frac_bits;
  uint64_t* y[2];
  const uint64_t* add[2];
} sufhip_trunc_epilogue;

/* ---------------------------------------------------------------------- */
/* Two-party steps with both parties on one GPU (SUF's local channel: an    */
/* open is an exchange of masked shares and an add).  Each call does both   */
/* parties' local work of one round plus the open.  They stand in for the   */
/* host loops of MulTask / TruncTask / CubicPolyTask                        */
/* (include/runtime/phase_tasks.hpp:198-402, 2962-3061) when SUF runs both  */
/* parties in one process; they have no launcher in cuda_primitives.hpp.   */
/* ---------------------------------------------------------------------- */
/* d_xhat[i] = (d_x0[i] + r0) + (d_x1[i] + r1): the masked open of a gate input. */
int sufhip_open2_masked(const uint64_t* d_x0, const uint64_t* d_x1, uint64_t r0, uint64_t r1,
                        size_t n, uint64_t* d_xhat, void* stream);

/* d_open[i] = (d_x0[i] - d_a0[i]) + (d_x1[i] - d_a1[i]): a Beaver open (the
 * D = X - A and E = W - B of a matmul, attention_block.cpp:452-900). */
int sufhip_open2_diff(const uint64_t* d_x0, const uint64_t* d_x1, const uint64_t* d_a0,
                      const uint64_t* d_a1, size_t n, uint64_t* d_open, void* stream);

/* One Beaver product for both parties.  Per element i and party p:
 *   u_p = u[p][i*u_stride + u_off] (+ u_add[p][i*u_add_stride + u_add_off] << u_add_shift)
 *   v_p = v[p][i];   (a_p, b_p, c_p) = triples[p][3i], [3i+1], [3i+2]
 *   d = (u_0 - a_0) + (u_1 - a_1),  e = (v_0 - b_0) + (v_1 - b_1)        (the open)
 *   z_p = c_p + d*b_p + e*a_p + [p == 0] d*e
 *         (+ z_add[p][i*z_add_stride + z_add_off] << z_add_shift)
 * zhat == NULL: z[p][i] = z_p.  Otherwise only the masked open of the
 * product is written: zhat[i] = z_0 + z_1 + open_mask[0] + open_mask[1].
 * u_add / z_add: both parties' pointers or neither. */
typedef struct sufhip_mul2_args {
  const uint64_t* u[2];
  size_t u_stride;
  size_t u_off;
  const uint64_t* u_add[2];
  size_t u_add_stride;
  size_t u_add_off;
  int u_add_shift;
  const uint64_t* v[2];
  const uint64_t* triples[2];
  const uint64_t* z_add[2];
  size_t z_add_stride;
  size_t z_add_off;
  int z_add_shift;
  uint64_t* z[2];
  uint64_t* zhat;
  uint64_t open_mask[2];
} sufhip_mul2_args;
int sufhip_mul2(const sufhip_mul2_args* args, size_t n, void* stream);

/* d_out[i] = d_y[i] + (d_add[i*add_stride + add_off] << shift) (one party). */
int sufhip_add_shifted(const uint64_t* d_y, const uint64_t* d_add, size_t add_stride,
                       size_t add_off, int shift, size_t n, uint64_t* d_out, void* stream);

/* Generalised operands for the row-wise tasks of SUF's softmax and LayerNorm
 * (SoftmaxBlockTask, include/nn/softmax_block_task.hpp:33-450; LayerNormTask,
 * RecipTask, RsqrtTask, MulRowBroadcastTask, include/runtime/phase_tasks.hpp:
 * 1383-2668, 3140-3653), whose factors are affine in stored shares: x - mu[row],
 * 2 - xy, 1.5 - h/2, t + c0, inv[row].
 *
 * A term reads, for element i and party p, p[p][j * stride + off] with
 * j = index ? index[i] : i (index: int32, e.g. the row of element i),
 * multiplies it by the public `mul` (mod 2^64), shifts it left by `shift` and
 * subtracts it when `negate` is set.  An absent term has
 * p[0] == p[1] == NULL; a present one needs both.  j is clamped to
 * [0, len), so no index value reads outside the arrays; without an index,
 * len must be >= n. */
typedef struct sufhip_term2 {
  const uint64_t* p[2];
  const int32_t* index;
  size_t len;    /* rows j the arrays hold (j is clamped below len) */
  size_t stride; /* >= 1 */
  size_t off;    /* < stride */
  int shift;     /* 0..63 */
  int negate;
  uint64_t mul;  /* public multiplier applied before the shift (0 acts as 1) */
} sufhip_term2;

/* Per element and party: t[0] + t[1] + [p == 0] party0_const, i.e. the
 * shared value sum_terms + party0_const (a public constant is added to party
 * 0's share only). */
typedef struct sufhip_operand2 {
  sufhip_term2 t[2];
  uint64_t party0_const;
} sufhip_operand2;

/* Evaluates an operand for both parties: d_out0 / d_out1 (either may be NULL)
 * receive the shares, and d_xhat (may be NULL) the masked open
 * xhat[i] = x_0 + x_1 + mask of a gate input (mask = r_0 + r_1).  With
 * `trunc` (may be NULL) the open feeds that truncation gate, whose outputs
 * are written instead of d_xhat. */
int sufhip_lin2(const sufhip_operand2* x, size_t n, uint64_t* d_out0, uint64_t* d_out1,
                uint64_t* d_xhat, uint64_t mask, const sufhip_trunc_epilogue* trunc,
                void* stream);

/* Up to 4 independent sufhip_lin2 evaluations (each with the meaning of
 * sufhip_lin2's arguments) in one launch: opens of one protocol round that
 * do not depend on each other. */
/* Optional output of an open as the digit planes of a two-party Beaver
 * product's operand (sufhip_kb_split_batch's layout): element i of the
 * [batches][rows x cols] open goes to planes [8][batches][K/32][R][32] with
 * (K, R) = (cols, rows) for k_is_col = 1 and (rows, cols) otherwise; rows and
 * cols multiples of 32, 16-byte aligned.  planes = NULL: none.
 * planes_a0 (optional, with a0): also the planes of open[i] + a0[i], a0
 * indexed like the open -- party 0's own value D + A_0 after the open of
 * D = X - A, the left operand of its product with E in the balanced form of
 * sufhip_beaver_matmul2_mfma_ex (Xp). */
typedef struct sufhip_kb_planes {
  int8_t* planes;
  int batches, rows, cols;
  int k_is_col;
  int8_t* planes_a0;
  const uint64_t* a0;
} sufhip_kb_planes;
typedef struct sufhip_lin2_job {
  sufhip_operand2 x;
  size_t n;
  uint64_t* out[2];
  uint64_t* xhat;
  uint64_t mask;
  const sufhip_trunc_epilogue* trunc;
  sufhip_kb_planes xhat_planes; /* the open also as digit planes (n = batches rows cols) */
} sufhip_lin2_job;
int sufhip_lin2_batch(const sufhip_lin2_job* jobs, int count, void* stream);

/* Beaver product for both parties with general operands (MulTask and
 * MulRowBroadcastTask, phase_tasks.hpp:198-402, 1810-2185; beaver_mul_kernel
 * and row_broadcast_mul_kernel, cuda/cuda_primitives.cu:114-139, 303-336):
 *   d = open(u - a), e = open(v - b),
 *   z_p = c_p + d*b_p + e*a_p + [p == 0] d*e + z_add_p.
 * a, b, c are the triple shares as terms (shift 0, not negated; an index on b
 * gives the row-broadcast triple of MulRowBroadcastTask, whose e is then one
 * value per row).  z_add's terms may be absent.  zhat == NULL: z[p][i] = z_p;
 * otherwise only zhat[i] = z_0 + z_1 + open_mask is written (the masked open
 * of the product for the next truncation gate); with `trunc` that gate's
 * outputs are written instead. */
typedef struct sufhip_mul2x_args {
  sufhip_operand2 u;
  sufhip_operand2 v;
  sufhip_term2 a;
  sufhip_term2 b;
  sufhip_term2 c;
  sufhip_operand2 z_add;
  uint64_t* z[2];
  uint64_t* zhat;
  uint64_t open_mask;
  const sufhip_trunc_epilogue* trunc; /* the open feeds this gate (replaces zhat) */
} sufhip_mul2x_args;
int sufhip_mul2x(const sufhip_mul2x_args* args, size_t n, void* stream);

/* Row sums for both parties (launch_row_sum_kernel / launch_row_sum_ragged_kernel,
 * cuda_primitives.cu:339-389, run for both parties, followed by the public
 * scaling of LayerNormTask's mean and variance, phase_tasks.hpp:2293-2470):
 *   s_p[r] = mul_const * sum_{i in row r} x_p[i]  (mod 2^64)
 * Row r covers elements [d_row_offsets[r], d_row_offsets[r+1]) when
 * d_row_offsets (int32 [rows + 1], non-decreasing) is given, else
 * [r * cols, (r + 1) * cols).  d_sum0 / d_sum1 / d_hat may each be NULL;
 * d_hat[r] = s_0[r] + s_1[r] + mask (masked open of the scaled sum); with
 * `trunc` the truncation gate's outputs are written instead of d_hat. */
int sufhip_row_sum2(const sufhip_operand2* x, int rows, int cols, const int32_t* d_row_offsets,
                    uint64_t mul_const, uint64_t* d_sum0, uint64_t* d_sum1, uint64_t* d_hat,
                    uint64_t mask, const sufhip_trunc_epilogue* trunc, void* stream);

/* Both parties' broadcast interval-LUT keys of one gate in one launch (the
 * coefficient LUT of a composite gate evaluated by both parties), at the
 * masked open xhat = x_0 + x_1 + mask of the operand x, or at d_xhat when x
 * is NULL.  Same shares as sufhip_interval_lut_eval with each key; for small
 * gates (intervals <= 64, intervals * out_words <= 512).  d_out0 / d_out1:
 * [n][out_words]. */
int sufhip_interval_lut_eval2(const uint8_t* d_key0, const uint8_t* d_key1, size_t key_bytes,
                              int intervals, int out_words, const sufhip_operand2* x,
                              const uint64_t* d_xhat, uint64_t mask, size_t n, uint64_t* d_out0,
                              uint64_t* d_out1, void* stream);

/* A whole elementwise gate chain for both parties in one launch: the
 * coefficient LUT at the masked open of x, every Beaver product (opens
 * summed in registers) and every truncation (table gates, f-bit, the
 * rsqrt's third f + 1), per element.  The shares equal those of the
 * round-by-round evaluation with the same material.
 *   SUFHIP_CHAIN_CUBIC  CubicPolyTask (include/runtime/phase_tasks.hpp:
 *     2718-3066), 4-word LUT (c0..c3), 3 products, 3 truncations:
 *     y = tr((c3 x + c2 << f) x); y2 = tr((y + c1 << f) x); out = tr(y2 + c0 << f)
 *   SUFHIP_CHAIN_RECIP  RecipTask with one NR step (phase_tasks.hpp:3140-3653),
 *     2-word LUT (c0, c1): y = tr(c1 x) + c0; out = tr(y (2 << f - tr(y x)))
 *   SUFHIP_CHAIN_RSQRT  RsqrtTask with one NR step (phase_tasks.hpp:1383-1700),
 *     2-word LUT: y = tr(c1 x) + c0; y2 = tr(y y); h = tr_(f+1)(x y2);
 *     out = tr(y (3 << (f - 1) - h))  (4 products, 4 truncations)
 * a / b / c: the products' triple shares as terms (shift 0); trunc[k]: the
 * truncation gates in order (y ignored), trunc_mask[k] their masks;
 * frac_bits in [1, 13]; intervals <= 64. */
/* Optional output of a producer as the left operand of a following
 * public-weight product (sufhip_matmul_public2_planes): element i = m cols + k
 * of party p goes to the balanced base-256 digit planes [8][cols/32][2 rows]
 * [32] int8 (rows = n / cols; party 0's rows first), 16-byte aligned, cols
 * and rows multiples of 32.  planes = NULL: none. */
typedef struct sufhip_x_planes {
  int8_t* planes;
  int cols;
} sufhip_x_planes;

#define SUFHIP_CHAIN_CUBIC 0
#define SUFHIP_CHAIN_RECIP 1
#define SUFHIP_CHAIN_RSQRT 2
typedef struct sufhip_chain2_args {
  int kind;
  int frac_bits;
  size_t n;
  sufhip_operand2 x;
  const uint8_t* lut[2];
  size_t lut_key_bytes;
  int intervals;
  uint64_t lut_mask;
  sufhip_term2 a[4];
  sufhip_term2 b[4];
  sufhip_term2 c[4];
  sufhip_trunc_epilogue trunc[4];
  uint64_t trunc_mask[4];
  uint64_t* out[2];        /* may be NULL when out_planes is given */
  sufhip_x_planes out_planes;
} sufhip_chain2_args;
int sufhip_gate_chain2(const sufhip_chain2_args* args, void* stream);

/* Both parties' shares of one Beaver triple set: a, b, c device arrays per
 * party (b per row for a row-broadcast triple). */
typedef struct sufhip_triple2 {
  const uint64_t* a[2];
  const uint64_t* b[2];
  const uint64_t* c[2];
} sufhip_triple2;

/* LayerNormTask whole (include/runtime/phase_tasks.hpp:2186-2668, with
 * RsqrtTask :1383-1700, as transformer_layer_forward builds it,
 * src/nn/transformer_layer.cpp:626-760: no gamma/beta, one NR step) for both
 * parties in one launch, one workgroup per row of the row-major
 * [rows x cols] input x (cols <= 2048):
 *   mu  = tr_mean(inv_len * sum_row x)          open masked by mean_mask
 *   d   = x - mu[row];  q = d * d               Beaver, triple sq (per element)
 *   va  = tr_var[0](inv_len * sum_row q)        open masked by var_mask[0]
 *   var = tr_var[1](va)                         open masked by var_mask[1]
 *   rs  = rsqrt chain at var + eps (party 0 adds eps); its LUT, triples and
 *         truncations as sufhip_gate_chain2 with kind SUFHIP_CHAIN_RSQRT and
 *         n = rows (x and out of that struct are ignored)
 *   out = tr_norm(d * rs[row])                  row-broadcast triple norm,
 *                                               open masked by norm_mask
 * Every tr_* is a prepared GapARS table gate (frac_bits <= 14; y ignored).
 * The shares equal those of the launch-per-step evaluation (sufhip_row_sum2,
 * sufhip_mul2x, sufhip_lin2, sufhip_gate_chain2 with the same material). */
typedef struct sufhip_layernorm2_args {
  const uint64_t* x[2];
  int rows;
  int cols;
  uint64_t inv_len;
  uint64_t eps;
  sufhip_trunc_epilogue tr_mean;
  sufhip_trunc_epilogue tr_var[2];
  sufhip_trunc_epilogue tr_norm;
  uint64_t mean_mask;
  uint64_t var_mask[2];
  uint64_t norm_mask;
  sufhip_triple2 sq;
  sufhip_triple2 norm;
  sufhip_chain2_args rsqrt;
  uint64_t* out[2];        /* may be NULL when out_planes is given */
  sufhip_x_planes out_planes;
  /* Optional (in_slices != NULL; x is then ignored): the input is the
   * truncation of a public-weight product whose k-slices
   * sufhip_matmul_public2_planes_partial left unreduced,
   *   x_p[i] = tr_in_p(sum_z in_slices[(2 z) mn + i] + in_slices[(2 z + 1) mn + i]
   *                    + in_mask) + tr_in.add[p][i]   (mn = rows cols),
   * written to tr_in.y[p][i] and then normalised: the product's reduction and
   * its truncation epilogue (the residual r1 = tr(ctx Wout) + x of
   * transformer_layer_forward, src/nn/transformer_layer.cpp:626-760) run in
   * this launch instead of their own.  2..8 slices; tr_in a prepared GapARS
   * table gate with outputs (and optionally an addend). */
  const uint64_t* in_slices;
  int in_slice_count;
  sufhip_trunc_epilogue tr_in;
  uint64_t in_mask;
  /* Optional (walk_count > 0): the key-only halves of other truncation gates,
   * as sufhip_trunc_prepare_batch(walk_prg_state, walk_jobs, walk_count)
   * would write them, for gates that later launches evaluate (the prepare of
   * transformer_layer_forward's later truncations, src/nn/
   * transformer_layer.cpp:435-830).  Up to 24 table-gate jobs (f <= 14) run
   * as extra workgroups of this launch, on the CUs its rows leave free (rows
   * of up to 1024 elements); other job sets and longer rows go through
   * sufhip_trunc_prepare_batch on the same stream first.
   * The results are byte-equal either way. */
  const sufhip_trunc_job* walk_jobs;
  int walk_count;
  const uint8_t* walk_prg_state;
} sufhip_layernorm2_args;
int sufhip_layernorm2(const sufhip_layernorm2_args* args, void* stream);

/* RowMaxDiffTask whole (include/nn/row_maxdiff_task.hpp:49-165) for both
 * parties in one launch: every round of the pairwise-max tree over the packed
 * rows [d_row_offsets[r], d_row_offsets[r+1]) (1 <= length <= max_row <= 512,
 * 2^rounds >= max_row), then d_delta_p[i] = max_p(row) - x_p[i].  Round k
 * uses keys[k] (both parties' ReLU LUT blobs, as sufhip_relu_max_round2)
 * and counts its LUT slots like the per-round evaluation:
 * d_round_offsets[k * rows + r] = the row's first output slot in round k.
 * Same shares as the per-round kernels followed by the delta step. */
typedef struct sufhip_relu_round_key {
  const uint8_t* key[2];
  size_t key_bytes;
  int intervals; /* <= 8 */
  uint64_t mask;
} sufhip_relu_round_key;
int sufhip_relu_max_tree2(const uint64_t* d_x0, const uint64_t* d_x1, int rows,
                          const int32_t* d_row_offsets, int max_row, int rounds,
                          const int32_t* d_round_offsets, const sufhip_relu_round_key* keys,
                          uint64_t* d_delta0, uint64_t* d_delta1, void* stream);

/* SoftmaxBlockTask whole (include/nn/softmax_block_task.hpp:97-450, fed by
 * RowMaxDiffTask, include/nn/row_maxdiff_task.hpp:49-165) for both parties in
 * one launch, one wavefront per packed row [d_row_offsets[r],
 * d_row_offsets[r+1]) (1 <= length <= max_row <= 512):
 *   s     = x at the row's elements; with pre_truncs = 1 or 2, s is replaced
 *           by pre[q](open of s masked by pre_mask[q]) in turn (the scores'
 *           truncations of attention_forward)
 *   max   = the ReLU pairwise-max tree over s (rounds <= 10, keys and
 *           d_round_offsets as sufhip_relu_max_tree2)
 *   e     = nexp chain at max - s (sufhip_gate_chain2 material, kind CUBIC,
 *           n = the packed element count; x and out of that struct ignored;
 *           its triple shares plain arrays: no index, multiplier, shift or
 *           negation, all of stride 1 or all of stride 3, else
 *           SUFHIP_ERR_INVALID)
 *   inv   = recip chain at the row sum of e (kind RECIP, n = rows)
 *   prob  = tr_norm(e * inv[row]) (row-broadcast triple norm, open masked
 *           by norm_mask)
 * and writes prob to out (if given) and/or, with d_dense given, the open
 * P - A of the next Beaver product over the dense [rows x dense_cols]
 * layout: d_dense[r * dense_cols + j] = (prob_0 - a_0) + (prob_1 - a_1) for
 * j < length, (0 - a_0) + (0 - a_1) for length <= j < dense_cols
 * (dense_a[p] [rows * dense_cols]).  Shares equal those of the launch-per-
 * step evaluation with the same material. */
typedef struct sufhip_softmax2_args {
  sufhip_operand2 x;
  int pre_truncs;
  sufhip_trunc_epilogue pre[2];
  uint64_t pre_mask[2];
  int rows;
  const int32_t* d_row_offsets;
  int max_row;
  int rounds;
  const int32_t* d_round_offsets;
  sufhip_relu_round_key keys[10];
  sufhip_chain2_args nexp;
  sufhip_chain2_args recip;
  sufhip_triple2 norm;
  sufhip_trunc_epilogue tr_norm;
  uint64_t norm_mask;
  uint64_t* out[2];
  uint64_t* d_dense;
  const uint64_t* dense_a[2];
  int dense_cols;
  sufhip_kb_planes dense_planes; /* the dense open also as digit planes, rows x dense_cols */
} sufhip_softmax2_args;
int sufhip_softmax2(const sufhip_softmax2_args* args, void* stream);

/* One pairwise-max round of RowMaxDiffTask (include/nn/row_maxdiff_task.hpp:
 * 49-150), max(a, b) = b + ReLU(a - b), for both parties.  For output slot j:
 *   src_b[j] < 0: next_p[j] = cur_p[src_a[j]] (odd element carried);
 *   else: d_p = cur_p[src_a[j]] - cur_p[src_b[j]], xhat = d_0 + d_1 + mask,
 *         (q0_p, q1_p) = interval LUT share of party p at xhat (element index
 *         j of the batch, out_words = 2, the ReLU SUF's coefficients shifted
 *         to the public xhat: q0 + q1 xhat = ReLU(d)),
 *         next_p[j] = cur_p[src_b[j]] + q0_p + q1_p * xhat.
 * d_lut0 / d_lut1: the parties' broadcast interval-LUT blobs (format of
 * sufhip_interval_lut_build_key; intervals <= 64, key_bytes =
 * sufhip_interval_lut_key_bytes(intervals, 2)).  Source indices outside
 * [0, n_in) yield 0 instead of a read. */
int sufhip_relu_max_round2(const uint64_t* d_cur0, const uint64_t* d_cur1, size_t n_in,
                           const int32_t* d_src_a, const int32_t* d_src_b, size_t n_out,
                           const uint8_t* d_lut0, const uint8_t* d_lut1, size_t key_bytes,
                           int intervals, uint64_t mask, uint64_t* d_next0, uint64_t* d_next1,
                           void* stream);

/* ---------------------------------------------------------------------- */
/* Interval LUT and packed compare in the reference GPU blob formats        */
/* (cuda/pfss_backend_gpu.cu:75-94, 189-288), evaluated with the kernel     */
/* counter convention of cuda/pfss_kernels.cu:240-719.  They replace        */
/* GpuPfssBackend::eval_interval_lut_many_device[_broadcast] and            */
/* eval_packed_lt_many_device[_broadcast] (PfssGpuStagedEval,               */
/* include/proto/backend_gpu.hpp:176-201) and PfssIntervalLutExt::          */
/* eval_interval_lut_many_u64 / PackedLtBackend::eval_packed_lt_many        */
/* (pfss_interval_lut_ext.hpp:17-27, packed_backend.hpp:15-23).             */
/* Keys are device blobs: [N][key_bytes] or one blob (key_broadcast = 1),   */
/* 8-byte aligned; key_bytes must equal the *_key_bytes() of the stated     */
/* geometry.  Outputs are u64 [N][out_words].                               */
/* ---------------------------------------------------------------------- */
/* seed_from_id (cuda/pfss_backend_gpu.cu:189-194): 16 bytes, byte i = low
 * byte of the i-th output of std::mt19937_64(id ^ tweak * 0x9e3779b97f4a7c15). */
void sufhip_seed_from_id(uint64_t id, uint64_t tweak, uint8_t* seed16);
size_t sufhip_interval_lut_key_bytes(int intervals, int out_words);
/* Host: one party's LUT blob (build_interval_key, pfss_backend_gpu.cu:223-255).
 * cuts [intervals + 1], payload [intervals][out_words]. */
int sufhip_interval_lut_build_key(int party, uint64_t nonce, int in_bits, int out_words,
                                  const uint64_t* cuts, int intervals, const uint64_t* payload,
                                  const uint8_t* seed16, uint8_t* blob);
int sufhip_interval_lut_eval(const uint8_t* d_keys, size_t key_bytes, int key_broadcast,
                             int intervals, int out_words, const uint64_t* d_xs, size_t n,
                             uint64_t* d_out, void* stream);
size_t sufhip_packed_lt_key_bytes(int num_thr);
/* Host: one party's packed-compare blob (build_packed_cmp_key,
 * pfss_backend_gpu.cu:257-288); thresholds are stored masked to in_bits and
 * the sorted flag is derived. */
int sufhip_packed_lt_build_key(int party, uint64_t nonce, int in_bits, const uint64_t* thresholds,
                               int num_thr, const uint8_t* seed16, uint8_t* blob);
/* out_words must be ceil(num_thr / 64). */
int sufhip_packed_lt_eval(const uint8_t* d_keys, size_t key_bytes, int key_broadcast, int num_thr,
                          int out_words, const uint64_t* d_xs, size_t n, uint64_t* d_out,
                          void* stream);

/* ---------------------------------------------------------------------- */
/* Ring postprocessing, Beaver products, row reductions and open packing.   */
/* Each replaces the launcher of the same name in                          */
/* include/runtime/cuda_primitives.hpp (line numbers below) with the same   */
/* argument list, a status return, and the kernel formula of               */
/* cuda/cuda_primitives.cu.                                                 */
/* ---------------------------------------------------------------------- */
/* launch_beaver_mul_kernel (:15-25): out = c + d*b + e*a (+ d*e if party 0).
 * d_x, d_y are accepted for signature parity and not read. */
int sufhip_beaver_mul(int party, const uint64_t* d_x, const uint64_t* d_y, const uint64_t* d_a,
                      const uint64_t* d_b, const uint64_t* d_c, const uint64_t* d_d_open,
                      const uint64_t* d_e_open, uint64_t* d_out, size_t n, void* stream);
/* launch_beaver_mul_aos_kernel (:29-35): triples are {u64 a, b, c} per element. */
int sufhip_beaver_mul_aos(int party, const void* d_triples, const uint64_t* d_d_open,
                          const uint64_t* d_e_open, uint64_t* d_out, size_t n, void* stream);
/* launch_trunc_shift_kernel (:39-43): out = x >> frac_bits. */
int sufhip_trunc_shift(const uint64_t* d_in, uint64_t* d_out, int frac_bits, size_t n,
                       void* stream);
/* launch_trunc_postproc_kernel (:48-64): faithful TR/ARS (kind_gapars = 0) or
 * GapARS (1) output share from the PFSS base word, carry/sign/wrap bool words
 * and the public xhat (formulas of include/gates/postproc_hooks.hpp:172-373).
 * A bool index is used only when 0 <= idx < bool_stride and d_bools != NULL. */
int sufhip_trunc_postproc(int party, int kind_gapars, int frac_bits, uint64_t r_hi_share,
                          uint64_t m_share, const uint64_t* d_hatx_public, const uint64_t* d_arith,
                          size_t arith_stride, int arith_idx, const uint64_t* d_bools,
                          size_t bool_stride, int carry_idx, int sign_idx, int wrap_idx,
                          uint64_t* d_out, size_t n, void* stream);
/* launch_horner_cubic_kernel (:68-75): ((c3 x + c2) x + c1) x + c0. */
int sufhip_horner_cubic(const uint64_t* d_x, const uint64_t* d_c0, const uint64_t* d_c1,
                        const uint64_t* d_c2, const uint64_t* d_c3, uint64_t* d_out, size_t n,
                        void* stream);
/* launch_add_rout_aos_kernel (:79-84): out[i*out_words + j] += r_out[j] for
 * j < r_out_words; r_out is a host array.  Up to 64 words (the reference
 * launcher silently does nothing above 8; here that is an error above 64). */
int sufhip_add_rout_aos(uint64_t* d_out, size_t elems, int out_words, const uint64_t* r_out,
                        size_t r_out_words, void* stream);
/* launch_row_broadcast_mul_kernel (:91-102). */
int sufhip_row_broadcast_mul(int party, const uint64_t* d_A, const uint64_t* d_B_rows,
                             const uint64_t* d_C, const uint64_t* d_d_open,
                             const uint64_t* d_e_open_rows, int rows, int cols,
                             const int* d_valid_lens, uint64_t* d_out, size_t n, void* stream);
/* launch_row_sum_kernel (:106-111); valid_lens (optional) are clamped to cols. */
int sufhip_row_sum(const uint64_t* d_mat, int rows, int cols, const int* d_valid_lens,
                   uint64_t* d_out_rows, void* stream);
/* launch_row_sum_ragged_kernel (:117-121). */
int sufhip_row_sum_ragged(const uint64_t* d_vals, const int* d_row_offsets, int rows,
                          uint64_t* d_out_rows, void* stream);
/* launch_beaver_matmul2d_kernel (:133-147): out = C + D*B + A*E (+ D*E for
 * party 0) mod 2^64; A, D [M x K]; B, E [K x N] (or [N x K] when
 * w_transposed); C, out [M x N]; optional (out * mul_const) >> mul_shift on the
 * signed 128-bit product when has_scale. */
int sufhip_beaver_matmul2d(int party, const uint64_t* d_D_open, const uint64_t* d_E_open,
                           const uint64_t* d_A_tri_share, const uint64_t* d_B_tri_share,
                           const uint64_t* d_C_tri_share, int M, int K, int N, int w_transposed,
                           int has_scale, int64_t mul_const, int mul_shift, uint64_t* d_out,
                           void* stream);
/* The same product as sufhip_beaver_matmul2d (w_transposed = 0, no scale) on
 * the int8 matrix cores: operands split into balanced base-256 digits and
 * the 36 digit-plane GEMMs with i + j < 8 accumulated exactly in int32
 * (v_mfma_i32_32x32x32_i8), recombined mod 2^64.  Requires M % 32 == 0,
 * N % 64 == 0, K % 32 == 0 and K <= 8191 (work_bytes() is 0 otherwise).
 * d_work: 16-byte aligned device scratch of
 * sufhip_beaver_matmul2d_mfma_work_bytes(M, K, N) bytes (the digit planes,
 * 16 (M + N) K bytes, plus k-slice partial sums for small grids), clobbered. */
size_t sufhip_beaver_matmul2d_mfma_work_bytes(int M, int K, int N);
int sufhip_beaver_matmul2d_mfma(int party, const uint64_t* d_D_open, const uint64_t* d_E_open,
                                const uint64_t* d_A_tri_share, const uint64_t* d_B_tri_share,
                                const uint64_t* d_C_tri_share, int M, int K, int N,
                                uint64_t* d_out, void* d_work, size_t work_bytes, void* stream);
/* launch_beaver_matmul2d_batched_kernel (:151-166): D [batches][M x K],
 * E [batches][K x N]; the same A, B, C for every batch; out [batches][M x N]. */
int sufhip_beaver_matmul2d_batched(int party, const uint64_t* d_D_open, const uint64_t* d_E_open,
                                   const uint64_t* d_A_tri_share, const uint64_t* d_B_tri_share,
                                   const uint64_t* d_C_tri_share, int batches, int M, int K, int N,
                                   int w_transposed, int has_scale, int64_t mul_const,
                                   int mul_shift, uint64_t* d_out, void* stream);
/* Two-party batched Beaver product with one triple per batch instance (the
 * per-head QK^T and PV products of attention_forward,
 * src/nn/attention_block.cpp:1590-1850, as BatchedMatmul2DTask runs them; the
 * reference's batched launcher reuses one triple for every batch,
 * cuda_primitives.hpp:149-150): for batch b and party p,
 *   out_p[b] = C_p[b] + D[b] * B_p[b] + A_p[b] * E[b] (+ D[b] * E[b] for p = 0)
 * with D [b][M x K], E [b][K x N], A_p [b][M x K], B_p [b][K x N],
 * C_p and out_p [b][M x N], row-major, mod 2^64.  Small launches split the
 * 2K inner dimension over slices summed by a second pass: d_work of
 * sufhip_beaver_matmul2_batched_work_bytes() bytes (0: none needed). */
size_t sufhip_beaver_matmul2_batched_work_bytes(int batches, int M, int K, int N);
int sufhip_beaver_matmul2_batched(const uint64_t* d_D_open, const uint64_t* d_E_open,
                                  const uint64_t* d_A0, const uint64_t* d_A1,
                                  const uint64_t* d_B0, const uint64_t* d_B1,
                                  const uint64_t* d_C0, const uint64_t* d_C1, int batches, int M,
                                  int K, int N, uint64_t* d_out0, uint64_t* d_out1, void* d_work,
                                  size_t work_bytes, void* stream);

/* The same two-party batched product on the int8 matrix cores, exact
 * (36 int8 digit GEMMs per operand pair): every operand as balanced
 * base-256 digit planes, the triple shares' made once with the triples and
 * the opens' per call.  sufhip_kb_split_batch writes up to
 * SUFHIP_KB_SPLIT_JOBS operands' planes in one launch: src [batches][rows x
 * cols] u64 row-major -> planes [8][batches][K/32][R][32] int8 with
 * (K, R) = (cols, rows) for a left operand (k_is_col = 1: D, A_p) and
 * (rows, cols) for a right one (k_is_col = 0: E, B_p); rows and cols
 * multiples of 32, planes of sufhip_kb_planes_bytes() bytes, 16-byte
 * aligned.  sufhip_beaver_matmul2_mfma_batched: the planes of D, E, A_p,
 * B_p and C_p, out_p as in sufhip_beaver_matmul2_batched; M, K, N multiples
 * of 32, K <= 4096 (exact int32 accumulation).  planes_a0 (optional, with
 * a0): also the planes of src[i] + a0[i] (as in sufhip_kb_planes). */
#define SUFHIP_KB_SPLIT_JOBS 8
typedef struct sufhip_kb_split_job {
  const uint64_t* src;
  int8_t* planes;
  int batches, rows, cols;
  int k_is_col;
  int8_t* planes_a0;
  const uint64_t* a0;
} sufhip_kb_split_job;
/* sufhip_beaver_matmul2_mfma_ex: the same product with options.  merge_heads:
 * outputs at [m][b N + n] (heads side by side, as attention_forward merges
 * the heads' context) instead of [b][m][n].  trunc (optional): the open
 * out_0 + out_1 + mask feeds this prepared GapARS table gate (no addend),
 * whose outputs trunc->y are written at the output positions instead of
 * out (which may be NULL).  out_planes (optional, merge_heads only, cols =
 * batches N): the (truncated) outputs also as the digit planes of a
 * following public-weight product.  Xp (optional): the planes of D + A_0
 * (party 0's own value after the open, sufhip_kb_planes.planes_a0).  With
 * it each party's share takes two operand products per k-step,
 *   out_0 = C_0 + (D + A_0) E + D B_0,   out_1 = C_1 + A_1 E + D B_1,
 * the same shares as the three-product form that runs without it. */
typedef struct sufhip_beaver_mfma2_args {
  const int8_t* Dp;
  const int8_t* Ep;
  const int8_t* Ap[2];
  const int8_t* Bp[2];
  const uint64_t* C[2];
  int batches, M, K, N;
  uint64_t* out[2];
  int merge_heads;
  const sufhip_trunc_epilogue* trunc;
  uint64_t mask;
  sufhip_x_planes out_planes;
  const int8_t* Xp;
} sufhip_beaver_mfma2_args;
int sufhip_beaver_matmul2_mfma_ex(const sufhip_beaver_mfma2_args* args, void* stream);
size_t sufhip_kb_planes_bytes(int batches, int rows, int cols);
int sufhip_kb_split_batch(const sufhip_kb_split_job* jobs, int count, void* stream);
/* sufhip_kb_open_split_batch: up to SUFHIP_KB_SPLIT_JOBS masked opens of
 * Beaver operands written straight as their digit planes, with no u64 open
 * in memory: element i is a[0][i] + a[1][i] - b[0][i] - b[1][i] (D = X - A
 * or E = W - B from both parties' shares: materialize_open of the Beaver
 * matmul, src/nn/matmul_beaver.cpp:34-53), laid out as in
 * sufhip_kb_split_batch.  a[0]
 * and a[1] are required; b[p] = NULL subtracts nothing.
 * a_stride: an optional strided view of a[0] and a[1] (u64 units, each >= 0):
 * element (batch, row, col) of a[p] is read at a[p][a_stride[0] * batch +
 * a_stride[1] * row + a_stride[2] * col], e.g. one head's Q, K^T or V inside
 * the [seq x 3d] rows of a QKV product (attention_block.cpp:1517-1531 splits
 * them by copies).  All three zero: a[p] is [batches][rows][cols] like b[p].
 * The caller keeps every viewed element inside a[p]'s allocation. */
typedef struct sufhip_kb_open_job {
  const uint64_t* a[2];
  const uint64_t* b[2];
  int8_t* planes;
  int batches, rows, cols;
  int k_is_col;
  int8_t* planes_a0; /* optional, with a0: planes of the open + a0[i] */
  const uint64_t* a0;
  int64_t a_stride[3];
} sufhip_kb_open_job;
int sufhip_kb_open_split_batch(const sufhip_kb_open_job* jobs, int count, void* stream);
/* sufhip_kb_open_split_prepare: sufhip_trunc_prepare_batch(prg_state, tjobs,
 * tcount) followed by sufhip_kb_open_split_batch(jobs, count), with the same
 * results, in one launch when every truncation job is a table gate
 * (frac_bits <= 14) and at most 8 jobs whose walks cover at most three
 * quarters of one full walk workgroup per CU: the walks' dependent levels then
 * run beside the split's memory stream.  Other truncation jobs take
 * sufhip_trunc_prepare_batch's own launches first.  The two calls it replaces
 * stand for the Beaver matmul's materialize_open (src/nn/matmul_beaver.cpp:
 * 34-53) and the key-dependent DCF evaluation of the truncation that follows
 * it (include/gates/composite_fss.hpp:1508-1515); the reference issues them
 * separately.  tcount = 0 is the open split alone. */
int sufhip_kb_open_split_prepare(const sufhip_kb_open_job* jobs, int count,
                                 const uint8_t* prg_state, const sufhip_trunc_job* tjobs,
                                 int tcount, void* stream);
int sufhip_beaver_matmul2_mfma_batched(const int8_t* d_Dp, const int8_t* d_Ep,
                                       const int8_t* d_Ap0, const int8_t* d_Ap1,
                                       const int8_t* d_Bp0, const int8_t* d_Bp1,
                                       const uint64_t* d_C0, const uint64_t* d_C1, int batches,
                                       int M, int K, int N, uint64_t* d_out0, uint64_t* d_out1,
                                       void* stream);

/* Share x public weight for both parties (nn::matmul_publicW_gpu,
 * src/nn/matmul_gpu.cu:388-720; CPU form src/nn/matmul_publicW.cpp:17-36):
 * Y_p = X_p * W mod 2^64, X_p [M x K] u64 shares, W [K x N] public int64, on
 * the int8 matrix cores with W in `digits` balanced base-256 digit planes.
 * sufhip_public_w_digits: host helper, the digits the weights need (1..8).
 * sufhip_public_w_prepare: W's planes, k-blocked [digits][K/32][N][32] int8
 * (done once per weight; d_planes of sufhip_public_w_planes_bytes bytes,
 * 16-byte aligned; an opaque layout for sufhip_matmul_public2).
 * sufhip_matmul_public2: M, K, N multiples of 32, digits in 1..4 with
 * digits * K < 2^17 (exact int32 accumulation); writes the shares
 * (d_out0 and d_out1) and/or the masked open d_zhat = Y_0 + Y_1 + mask that
 * the following truncation gate consumes (with `trunc`: that gate's outputs
 * instead of d_zhat).  d_work: 16-byte aligned, of
 * sufhip_matmul_public2_work_bytes(M, K, N) bytes (0 for a bad shape). */
int sufhip_public_w_digits(const int64_t* w, size_t n);
size_t sufhip_public_w_planes_bytes(int K, int N, int digits);
int sufhip_public_w_prepare(const int64_t* d_W, int K, int N, int digits, int8_t* d_planes,
                            void* stream);
size_t sufhip_matmul_public2_work_bytes(int M, int K, int N);
/* sufhip_matmul_public2 with X_0, X_1 already as the digit planes a
 * producer wrote (sufhip_x_planes with cols = K, rows = M); same outputs and
 * workspace. */
int sufhip_matmul_public2_planes(const int8_t* d_Xp, int M, int K, int N, const int8_t* d_planes,
                                 int digits, uint64_t* d_out0, uint64_t* d_out1, uint64_t* d_zhat,
                                 uint64_t mask, const sufhip_trunc_epilogue* trunc, void* d_work,
                                 size_t work_bytes, void* stream);
/* The number of k-slices the products above split (M, K, N) into (0 for a
 * bad shape).  Above 1 each slice's partial shares pass through the
 * workspace and a reduction launch; sufhip_matmul_public2_planes_partial
 * stops before that launch and leaves the reduction (with the truncation) to
 * the consumer, sufhip_layernorm2's in_slices. */
int sufhip_matmul_public2_slices(int M, int K, int N);
/* sufhip_matmul_public2_planes without the reduction: on return *d_slices
 * points at the partial shares inside d_work, [slices][2][M N] u64 (slice z,
 * party p at (2 z + p) M N), valid once the launch has run and until the
 * workspace's next use.  Needs sufhip_matmul_public2_slices(M, K, N) > 1.
 * The product is the reference's public-weight matmul
 * (src/nn/matmul_publicW.cpp:17-36) before the truncation that follows it. */
int sufhip_matmul_public2_planes_partial(const int8_t* d_Xp, int M, int K, int N,
                                         const int8_t* d_planes, int digits, void* d_work,
                                         size_t work_bytes, const uint64_t** d_slices,
                                         void* stream);
/* The attention's opens written by the QKV product's launch.  For the
 * [seq x 3d] product Y = trunc(X Wqkv) (d = heads dh; M = seq, N = 3d) the
 * launch writes no Y: element (m, c), head h and column k of the head in
 * region j = c / d, goes as Y_0 + Y_1 - sub[j][0] - sub[j][1] to the digit
 * planes out[j] (sufhip_kb_planes).  Every sub[j][p] is indexed
 * [heads][seq][dh] like the head split of Y: A of QK^T, its B transposed per
 * head, and B of PV.  The planes:
 *   j = 0: Q_h - A    (heads, seq, dh, k_is_col 1; planes_a0 with a0 = A_0)
 *   j = 1: K_h^T - B  (heads, dh, seq, k_is_col 0)
 *   j = 2: V_h - B2   (heads, seq, dh, k_is_col 0)
 * the same planes as sufhip_kb_open_split_batch over strided views of Y
 * after sufhip_matmul_public2_planes with `trunc` (the head split of
 * attention_block.cpp:1517-1531 and materialize_open of
 * src/nn/matmul_beaver.cpp:34-53, in the product's epilogue).  trunc is
 * required (a prepared table gate; its y pointers are not written); dh a
 * multiple of 32, d of 64; the product unsliced. */
typedef struct sufhip_qkv_opens {
  int heads, seq, dh;
  const uint64_t* sub[3][2];
  sufhip_kb_planes out[3];
} sufhip_qkv_opens;
int sufhip_matmul_public2_planes_qkv(const int8_t* d_Xp, int M, int K, int N,
                                     const int8_t* d_planes, int digits, uint64_t mask,
                                     const sufhip_trunc_epilogue* trunc,
                                     const sufhip_qkv_opens* opens, void* d_work,
                                     size_t work_bytes, void* stream);
int sufhip_matmul_public2(const uint64_t* d_X0, const uint64_t* d_X1, int M, int K, int N,
                          const int8_t* d_planes, int digits, uint64_t* d_out0, uint64_t* d_out1,
                          uint64_t* d_zhat, uint64_t mask, const sufhip_trunc_epilogue* trunc,
                          void* d_work, size_t work_bytes, void* stream);

/* launch_row_mean_kernel (:169-174): sum >> log2(L) for power-of-two L, else
 * the u64 sum divided by L as a plain integer (the reference's formula). */
int sufhip_row_mean(const uint64_t* d_mat, int rows, int cols, const int* d_valid_lens,
                    uint64_t* d_out_rows, void* stream);
/* launch_row_variance_kernel (:179-185): sum over active columns of (x - mean)^2. */
int sufhip_row_variance(const uint64_t* d_mat, const uint64_t* d_mean, int rows, int cols,
                        const int* d_valid_lens, uint64_t* d_out_rows, void* stream);
/* launch_unpack_eff_bits_kernel (:189-193) / launch_pack_eff_bits_kernel
 * (:197-201): LSB-first bitstream of eff_bits-wide values in u64 words;
 * the packed buffer holds ceil(n * eff_bits / 64) words. */
int sufhip_unpack_eff_bits(const uint64_t* d_packed, int eff_bits, uint64_t* d_out, size_t n,
                           void* stream);
int sufhip_pack_eff_bits(const uint64_t* d_in, int eff_bits, uint64_t* d_packed, size_t n,
                         void* stream);
/* launch_open_add_to_signed_kernel (:206-212), launch_unpack_add_to_signed_kernel
 * (:217-224), launch_unpack_add_mod_kernel (:229-236). */
int sufhip_open_add_to_signed(const uint64_t* d_local_share, const uint64_t* d_remote_share,
                              uint64_t* d_out_signed, size_t n, int ring_bits, uint64_t ring_mask,
                              void* stream);
int sufhip_unpack_add_to_signed(const uint64_t* d_local_share, const uint64_t* d_packed_remote,
                                int eff_bits, uint64_t* d_out_signed, size_t n, int ring_bits,
                                uint64_t ring_mask, void* stream);
int sufhip_unpack_add_mod(const uint64_t* d_local_share, const uint64_t* d_packed_remote,
                          int eff_bits, uint64_t* d_out_mod, size_t n, int ring_bits,
                          uint64_t ring_mask, void* stream);

/* ---------------------------------------------------------------------- */
/* Composite gates with boolean outputs (SUF l_out > 0), both parties on one */
/* GPU: the selector network and boolean-DAG Beaver evaluation of            */
/* composite_eval_batch_backend (include/gates/composite_fss.hpp:2132-2456,  */
/* selectors_from_cutbits_block :893-974, eval_bool_xor_view                 */
/* include/gates/bool_dag_xor.hpp:13-104), and the bucket staging of x^      */
/* that PfssSuperBatch::flush_eval does (src/runtime/pfss_superbatch.cpp:    */
/* 740-930).                                                                 */
/* ---------------------------------------------------------------------- */

/* One job's masked inputs in a bucket: len values from src (device; plain
 * u64 when eff_bits == 64, else an LSB-first bitstream of eff_bits-wide
 * values in u64 words, the pack_eff_bits layout) to bucket[dst, dst + len). */
#define SUFHIP_STAGE_MAX_SEGS 64
typedef struct sufhip_stage_seg {
  const void* src;
  size_t len;
  size_t dst;
  int eff_bits;
} sufhip_stage_seg;
/* All of a bucket's segments in one launch (segments may not overlap). */
int sufhip_stage_hatx(const sufhip_stage_seg* segs, int count, uint64_t* d_bucket,
                      size_t bucket_len, void* stream);

/* Boolean program instructions (int32: opcode in bits 0-3, operand above),
 * postfix over XOR-shared bits: VAR pushes predicate query q's bit, WRAP
 * the low bit of wrap bit w's additive share, CONST a constant (party 0's
 * share); NOT, XOR, AND, OR pop their operands (AND and OR take one bit
 * triple each, in program order). */
#define SUFHIP_BOOL_VAR 0
#define SUFHIP_BOOL_WRAP 1
#define SUFHIP_BOOL_CONST 2
#define SUFHIP_BOOL_NOT 3
#define SUFHIP_BOOL_XOR 4
#define SUFHIP_BOOL_AND 5
#define SUFHIP_BOOL_OR 6
#define SUFHIP_BOOL_MAX_STACK 16
#define SUFHIP_COMPOSITE_MAX_ELL 8
#define SUFHIP_COMPOSITE_MAX_CUTS 31
#define SUFHIP_COMPOSITE_MAX_WRAP 32
#define SUFHIP_COMPOSITE_MAX_PROG 384

/* The x^-domain segments of the gate are delimited by `cuts` cut points; cut
 * bit k of element i is 1[xhat_i < cut_k] (XOR-shared bytes, bit 0).
 * Segment s's output j is program k = s ell + j: instructions
 * prog[prog_off[k], prog_off[k + 1]).  Triples (additive u64, [T][3][n] per
 * party: a, b, c) are consumed by index: cut k's b2a at k; the chain product
 * of selector s (1 <= s < cuts) at cuts + s - 1; output bit (s, j)'s b2a at
 * B + k and its selector product at B + (cuts + 1) ell + k, B = max(0,
 * 2 cuts - 1); T = sufhip_composite_bool_triples(cuts, ell).  Bit triples
 * ([and_count][n] bytes per party, bit 0 a, bit 1 b, bit 2 c = a AND b over
 * both parties' XOR shares) in program order.  out[p]: [n][ell] additive
 * shares of the boolean outputs. */
typedef struct sufhip_composite_bool_args {
  size_t n;
  int queries;
  int cuts;
  int ell;
  int wraps;
  int and_count;
  int prog_len;
  const uint8_t* pred[2];    /* [queries][n] */
  const uint8_t* cut[2];     /* [cuts][n] */
  const uint8_t* bit_tri[2]; /* [and_count][n] */
  const uint64_t* tri[2];    /* [T][3][n] */
  uint64_t* out[2];          /* [n][ell] */
  uint64_t wrap[2][SUFHIP_COMPOSITE_MAX_WRAP];
  int16_t prog_off[(SUFHIP_COMPOSITE_MAX_CUTS + 1) * SUFHIP_COMPOSITE_MAX_ELL + 1];
  int32_t prog[SUFHIP_COMPOSITE_MAX_PROG];
} sufhip_composite_bool_args;
size_t sufhip_composite_bool_triples(int cuts, int ell);
int sufhip_composite_bool2(const sufhip_composite_bool_args* args, void* stream);

/* One flush of a two-party open collector (the device path of
 * OpenCollector::flush, src/runtime/open_collector.cpp:357-791): the
 * requests' shares (device, both parties) are gathered, party 1's are
 * packed to eff_bits (the message it sends: launch_pack_eff_bits_kernel),
 * and party 0's own shares plus party 1's unpacked message give the opened
 * values (launch_unpack_add_mod_kernel; launch_unpack_add_to_signed_kernel
 * when sign_extend), masked to ring_bits, back to back in request order in
 * d_opened: (s0 + (s1 mod 2^eff_bits)) mod 2^ring_bits, exact when
 * eff_bits >= ring_bits or party 1's shares fit eff_bits.  Launches:
 * 2 * ceil(count / 64) gathers, one pack, one unpack-add (four for up to 64
 * requests).  d_work: 8-byte aligned,
 * sufhip_open_flush2_work_bytes(total, eff_bits) bytes. */
typedef struct sufhip_open_req {
  const uint64_t* share[2];
  size_t len;
} sufhip_open_req;
size_t sufhip_open_flush2_work_bytes(size_t total, int eff_bits);
int sufhip_open_flush2(const sufhip_open_req* reqs, int count, int eff_bits, int ring_bits,
                       int sign_extend, uint64_t* d_opened, void* d_work, size_t work_bytes,
                       void* stream);

/* ---------------------------------------------------------------------- */
/* Host-side helpers for seeded synthetic inputs                            */
/* ---------------------------------------------------------------------- */
/* out[i] = the i-th output of std::mt19937_64(seed). */
int sufhip_host_mt19937_64(uint64_t seed, uint64_t* out, size_t n);
/* out[i] = llround(clip(sigma * z_i, -clip, clip) * 2^frac_bits) as a
 * two's-complement u64, z_i standard normal by Box-Muller on
 * std::mt19937_64(seed) words (clip <= 0 disables clipping). */
int sufhip_host_normal_fixed(uint64_t seed, double sigma, double clip, int frac_bits,
                             uint64_t* out, size_t n);

#ifdef __cplusplus
}
#endif
#endif /* SUF_HIP_H */
