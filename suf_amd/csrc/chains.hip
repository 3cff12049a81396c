// Whole elementwise gate chains for two parties on one GPU in one launch.
//
// With both parties in one process an open is a local sum, so the rounds of
// an elementwise task chain need no grid-wide synchronisation between them:
// element i's rounds depend only on element i.  One kernel therefore runs,
// per element and for both parties, the coefficient LUT at the masked open,
// every Beaver product (each d / e open summed in registers) and every
// truncation gate (table lookup at the product's masked open), and writes
// only the final shares.  The arithmetic, element indices (LUT keystream
// counters), triples and keys are those of the round-by-round evaluation,
// so the shares are bit-identical to it.
//
//   CUBIC  CubicPolyTask (include/runtime/phase_tasks.hpp:2718-3066):
//          m = c3 x + c2 << f; y = tr(m x); y2 = tr((y + c1 << f) x);
//          out = tr(y2 + c0 << f)                (trunc_2f + c0 as two tr_f)
//   RECIP  RecipTask, one NR step (phase_tasks.hpp:3140-3653):
//          y = tr(c1 x) + c0; xy = tr(y x); out = tr(y (2 << f - xy))
//   RSQRT  RsqrtTask, one NR step (phase_tasks.hpp:1383-1700):
//          y = tr(c1 x) + c0; y2 = tr(y y); h = tr'(x y2);
//          out = tr(y (3 << (f - 1) - h))        (tr' truncates by f + 1)
#include <hip/hip_runtime.h>

#include "aes_lds.hpp"
#include "operand_device.hpp"
#include "suf_hip.h"
#include "sufhip_internal.hpp"
#include "trunc_device.hpp"

namespace sufhip {
namespace {

constexpr int kBlock = 256;
constexpr int kCopies = 32;
constexpr size_t kLutHdr = 216;
constexpr int kMaxIntervals = 64;
constexpr int kMaxWords = 4;

struct ChainArgs {
  sufhip_operand2 x;
  const uint8_t* lut[2];
  uint64_t lut_mask;
  int intervals;
  int f;
  sufhip_term2 a[4], b[4], c[4];
  const uint8_t* tkey[4][2];
  const uint4* ttab[4][2];
  uint64_t tmask[4];
  int tf[4];
  uint64_t* out[2];
  size_t n;
};

__device__ __forceinline__ uint64_t mask_bits(int bits) {
  return bits <= 0 ? 0 : (bits >= 64 ? ~uint64_t(0) : (uint64_t(1) << bits) - 1);
}

struct Two {
  uint64_t v[2];
};

// Beaver product k of the chain for both parties, opens summed in place.
__device__ __forceinline__ Two beaver(const ChainArgs& A, int k, size_t i, Two u, Two v) {
  const uint64_t a0 = term_at(A.a[k], 0, i), a1 = term_at(A.a[k], 1, i);
  const uint64_t b0 = term_at(A.b[k], 0, i), b1 = term_at(A.b[k], 1, i);
  const uint64_t c0 = term_at(A.c[k], 0, i), c1 = term_at(A.c[k], 1, i);
  const uint64_t d = (u.v[0] - a0) + (u.v[1] - a1);
  const uint64_t e = (v.v[0] - b0) + (v.v[1] - b1);
  return Two{{c0 + d * b0 + e * a0 + d * e, c1 + d * b1 + e * a1}};
}

// Truncation gate j at the masked open of z, both parties.
__device__ __forceinline__ Two trunc(const ChainArgs& A, int j, Two z) {
  const uint64_t zh = z.v[0] + z.v[1] + A.tmask[j];
  return Two{{trunc_table_eval(A.tkey[j][0], A.ttab[j][0], A.tf[j], zh),
              trunc_table_eval(A.tkey[j][1], A.ttab[j][1], A.tf[j], zh)}};
}

template <int kKind>
__global__ void __launch_bounds__(kBlock) gate_chain_kernel(ChainArgs A) {
  constexpr int W = kKind == SUFHIP_CHAIN_CUBIC ? 4 : 2;
  __shared__ __align__(16) uint32_t tab[256 * kCopies];
  __shared__ uint4 rk[2][11];
  __shared__ uint64_t cuts[2][kMaxIntervals];
  __shared__ uint64_t pay[2][kMaxIntervals * kMaxWords];
  fill_ttable<kCopies>(tab, kTDev.v);
  const int nint = A.intervals;
  for (int p = 0; p < 2; ++p) {
    const uint8_t* k = A.lut[p];
    const uint32_t* rkg = reinterpret_cast<const uint32_t*>(k + 40);
    for (int i = threadIdx.x; i < 11; i += blockDim.x)
      rk[p][i] = make_uint4(rkg[4 * i], rkg[4 * i + 1], rkg[4 * i + 2], rkg[4 * i + 3]);
    const uint64_t* cg = reinterpret_cast<const uint64_t*>(k + kLutHdr);
    const uint64_t* pg = cg + (nint + 1);
    for (int i = threadIdx.x; i < nint; i += blockDim.x) cuts[p][i] = cg[i];
    for (int i = threadIdx.x; i < nint * W; i += blockDim.x) pay[p][i] = pg[i];
  }
  __syncthreads();
  const AesLds<kCopies> aes{tab, threadIdx.x % kCopies};
  uint64_t m[2], nonce[2];
  int party[2];
  for (int p = 0; p < 2; ++p) {
    m[p] = mask_bits(*reinterpret_cast<const uint16_t*>(A.lut[p]));
    party[p] = A.lut[p][8];
    nonce[p] = *reinterpret_cast<const uint64_t*>(A.lut[p] + 16);
  }
  const int f = A.f;
  for (size_t i = size_t(blockIdx.x) * kBlock + threadIdx.x; i < A.n;
       i += size_t(gridDim.x) * kBlock) {
    const Two x{{operand_at(A.x, 0, i), operand_at(A.x, 1, i)}};
    const uint64_t xh = x.v[0] + x.v[1] + A.lut_mask;
    // Coefficient rows of both parties (interval LUT, pfss_kernels.cu:545-719).
    uint64_t cf[2][W];
    for (int p = 0; p < 2; ++p) {
      const uint64_t xm = xh & m[p];
      int lo = 0, hi = nint;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if ((cuts[p][mid] & m[p]) <= xm)
          lo = mid + 1;
        else
          hi = mid;
      }
      int iv = lo - 1;
      if (iv < 0) iv = 0;
#pragma unroll
      for (int w = 0; w < W; w += 2) {
        const uint64_t ctr = nonce[p] ^ (uint64_t(i) << 32) ^ (uint64_t(iv) * W + uint64_t(w));
        uint32_t s0 = uint32_t(ctr), s1 = uint32_t(ctr >> 32), s2 = 0, s3 = 0;
        aes.encrypt(s0, s1, s2, s3, rk[p]);
        const uint64_t k0 = uint64_t(s0) | uint64_t(s1) << 32;
        const uint64_t k1 = uint64_t(s2) | uint64_t(s3) << 32;
        const uint64_t* row = pay[p] + size_t(iv) * W;
        cf[p][w] = party[p] == 0 ? k0 : row[w] - k0;
        cf[p][w + 1] = party[p] == 0 ? k1 : row[w + 1] - k1;
      }
    }
    Two res;
    if constexpr (kKind == SUFHIP_CHAIN_CUBIC) {
      Two mm = beaver(A, 0, i, Two{{cf[0][3], cf[1][3]}}, x);
      mm.v[0] += cf[0][2] << f;
      mm.v[1] += cf[1][2] << f;
      const Two y = trunc(A, 0, beaver(A, 1, i, mm, x));
      const Two q{{y.v[0] + (cf[0][1] << f), y.v[1] + (cf[1][1] << f)}};
      const Two y2 = trunc(A, 1, beaver(A, 2, i, q, x));
      res = trunc(A, 2, Two{{y2.v[0] + (cf[0][0] << f), y2.v[1] + (cf[1][0] << f)}});
    } else {
      const Two t = trunc(A, 0, beaver(A, 0, i, Two{{cf[0][1], cf[1][1]}}, x));
      const Two y{{t.v[0] + cf[0][0], t.v[1] + cf[1][0]}};
      if constexpr (kKind == SUFHIP_CHAIN_RECIP) {
        const Two xy = trunc(A, 1, beaver(A, 1, i, y, x));
        const Two two{{(uint64_t(2) << f) - xy.v[0], uint64_t(0) - xy.v[1]}};
        res = trunc(A, 2, beaver(A, 2, i, y, two));
      } else {
        const Two y2 = trunc(A, 1, beaver(A, 1, i, y, y));
        const Two h = trunc(A, 2, beaver(A, 2, i, x, y2));
        const Two inner{{(uint64_t(3) << (f - 1)) - h.v[0], uint64_t(0) - h.v[1]}};
        res = trunc(A, 3, beaver(A, 3, i, y, inner));
      }
    }
    A.out[0][i] = res.v[0];
    A.out[1][i] = res.v[1];
  }
}

unsigned int chain_grid(size_t n) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const size_t need = (n + kBlock - 1) / kBlock;
  const size_t cap = size_t(cus) * 4;
  return static_cast<unsigned int>(need < cap ? need : cap);
}

}  // namespace
}  // namespace sufhip

using namespace sufhip;

extern "C" {

int sufhip_gate_chain2(const sufhip_chain2_args* args, void* stream) {
  SUFHIP_REQUIRE(args != nullptr, "sufhip_gate_chain2: null args");
  const sufhip_chain2_args& g = *args;
  SUFHIP_REQUIRE(g.kind == SUFHIP_CHAIN_CUBIC || g.kind == SUFHIP_CHAIN_RECIP ||
                     g.kind == SUFHIP_CHAIN_RSQRT,
                 "sufhip_gate_chain2: unknown kind");
  const int W = g.kind == SUFHIP_CHAIN_CUBIC ? 4 : 2;
  const int prods = g.kind == SUFHIP_CHAIN_RSQRT ? 4 : 3;
  SUFHIP_REQUIRE(g.frac_bits >= 1 && g.frac_bits <= kTruncTableBits - 1,
                 "sufhip_gate_chain2: frac_bits in [1, 13]");
  SUFHIP_REQUIRE(g.intervals >= 1 && g.intervals <= kMaxIntervals,
                 "sufhip_gate_chain2: intervals in [1, 64]");
  SUFHIP_REQUIRE(g.lut_key_bytes == sufhip_interval_lut_key_bytes(g.intervals, W),
                 "sufhip_gate_chain2: LUT key_bytes does not match (intervals, words)");
  if (g.n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(g.n < (size_t(1) << 40), "sufhip_gate_chain2: n too large");
  SUFHIP_REQUIRE(g.lut[0] && g.lut[1] && g.out[0] && g.out[1],
                 "sufhip_gate_chain2: null LUT key or output");
  SUFHIP_REQUIRE((reinterpret_cast<uintptr_t>(g.lut[0]) & 7) == 0 &&
                     (reinterpret_cast<uintptr_t>(g.lut[1]) & 7) == 0,
                 "sufhip_gate_chain2: LUT keys must be 8-byte aligned");
  if (int rc = check_operand(g.x, g.n, "sufhip_gate_chain2 x")) return rc;
  ChainArgs A{};
  A.x = g.x;
  A.lut[0] = g.lut[0];
  A.lut[1] = g.lut[1];
  A.lut_mask = g.lut_mask;
  A.intervals = g.intervals;
  A.f = g.frac_bits;
  A.n = g.n;
  A.out[0] = g.out[0];
  A.out[1] = g.out[1];
  for (int k = 0; k < prods; ++k) {
    SUFHIP_REQUIRE(g.a[k].p[0] && g.b[k].p[0] && g.c[k].p[0],
                   "sufhip_gate_chain2: a product's triple is missing");
    if (int rc = check_term(g.a[k], g.n, false, "sufhip_gate_chain2 a")) return rc;
    if (int rc = check_term(g.b[k], g.n, false, "sufhip_gate_chain2 b")) return rc;
    if (int rc = check_term(g.c[k], g.n, false, "sufhip_gate_chain2 c")) return rc;
    A.a[k] = g.a[k];
    A.b[k] = g.b[k];
    A.c[k] = g.c[k];
    const int want_f = (g.kind == SUFHIP_CHAIN_RSQRT && k == 2) ? g.frac_bits + 1 : g.frac_bits;
    SUFHIP_REQUIRE(g.trunc[k].frac_bits == want_f,
                   "sufhip_gate_chain2: truncation gate of the wrong width");
    sufhip_trunc_epilogue t = g.trunc[k];
    uint64_t dummy = 0;
    t.y[0] = t.y[1] = &dummy;  // outputs are the chain's own
    TruncEpi e;
    if (int rc = make_epi(&t, g.n, "sufhip_gate_chain2 trunc", &e)) return rc;
    A.tkey[k][0] = e.key[0];
    A.tkey[k][1] = e.key[1];
    A.ttab[k][0] = e.table[0];
    A.ttab[k][1] = e.table[1];
    A.tmask[k] = g.trunc_mask[k];
    A.tf[k] = e.f;
  }
  const dim3 grid(chain_grid(g.n)), block(kBlock);
  hipStream_t s = as_stream(stream);
  if (g.kind == SUFHIP_CHAIN_CUBIC)
    hipLaunchKernelGGL(gate_chain_kernel<SUFHIP_CHAIN_CUBIC>, grid, block, 0, s, A);
  else if (g.kind == SUFHIP_CHAIN_RECIP)
    hipLaunchKernelGGL(gate_chain_kernel<SUFHIP_CHAIN_RECIP>, grid, block, 0, s, A);
  else
    hipLaunchKernelGGL(gate_chain_kernel<SUFHIP_CHAIN_RSQRT>, grid, block, 0, s, A);
  return check_launch("gate_chain_kernel");
}

}  // extern "C"
