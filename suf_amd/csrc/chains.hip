// Whole elementwise gate chains for two parties on one GPU in one launch.
//
// With both parties in one process an open is a local sum, so the rounds of
// an elementwise task chain need no grid-wide synchronisation between them:
// element i's rounds depend only on element i.  One kernel therefore runs,
// per element and for both parties, the coefficient LUT at the masked open,
// every Beaver product and every truncation gate (chain_device.hpp), and
// writes only the final shares.  The arithmetic, element indices (LUT
// keystream counters), triples and keys are those of the round-by-round
// evaluation, so the shares are bit-identical to it.
#include <hip/hip_runtime.h>

#include "chain_device.hpp"

namespace sufhip {
namespace {

constexpr int kBlock = 512;  // two workgroups of the 72 KB LDS footprint per CU
constexpr int kCopies = 32;
using ChainAes = AesLds2<kCopies>;

// kPlain: x and the triple shares are plain arrays (ChainArgs::plain and
// plain_x), read through plain pointers.
template <int kKind, bool kPlain>
__global__ void __launch_bounds__(kBlock) gate_chain_kernel(ChainArgs A) {
  constexpr int W = kKind == SUFHIP_CHAIN_CUBIC ? 4 : 2;
  constexpr int kProds = chain_products<kKind>();
  __shared__ __align__(16) uint32_t tab[ChainAes::kSpanWords];
  __shared__ ChainLds L;
  __shared__ TruncHdr th[kProds][2];
  // Staging in one pass: the span's slots, the LUT items and the gates'
  // key headers all loaded before the first LDS store.
  {
    TruncHdrStager<kProds> hs;
    ChainAes::Filler<kBlock> tf;
    ChainStager<kBlock, 2> cs;
    hs.load(A, 0);
    tf.load(kTDev.v);
    cs.load(A, W);
    cs.store(A, W, L);
    tf.store(tab);
    hs.store(th);
  }
  __syncthreads();
  chain_compare(A, L);
  __syncthreads();
  const ChainAes aes = ChainAes::make(tab);
  const ChainKeyInfo K = chain_key_info(A, L);
  for (size_t i = size_t(blockIdx.x) * kBlock + threadIdx.x; i < A.n;
       i += size_t(gridDim.x) * kBlock) {
    Two res;
    if constexpr (kPlain) {
      const Two x{{plain_x(A, 0, i), plain_x(A, 1, i)}};
      res = chain_eval<kKind, ChainAes>(A, L, K, aes, i, x, plain_loader<kKind>{&A, i}, th);
    } else {
      const Two x{{operand_at(A.x, 0, i), operand_at(A.x, 1, i)}};
      res = chain_eval<kKind, ChainAes>(A, L, K, aes, i, x, chain_loader<kKind>{&A, i}, th);
    }
    if (A.out[0]) {
      A.out[0][i] = res.v[0];
      A.out[1][i] = res.v[1];
    }
    if (A.xp.planes) {
      const size_t rows = A.n / size_t(A.xp.cols);
      put_x_digits(A.xp, rows, i, 0, res.v[0]);
      put_x_digits(A.xp, rows, i, 1, res.v[1]);
    }
  }
}

unsigned int chain_grid(size_t n) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const size_t need = (n + kBlock - 1) / kBlock;
  const size_t cap = size_t(cus) * 2;
  return static_cast<unsigned int>(need < cap ? need : cap);
}

}  // namespace
}  // namespace sufhip

using namespace sufhip;

extern "C" {

int sufhip_gate_chain2(const sufhip_chain2_args* args, void* stream) {
  SUFHIP_REQUIRE(args != nullptr, "sufhip_gate_chain2: null args");
  const sufhip_chain2_args& g = *args;
  ChainArgs A;
  if (int rc = make_chain_args(g, true, "sufhip_gate_chain2", &A)) return rc;
  if (g.n == 0) return SUFHIP_OK;
  const dim3 grid(chain_grid(g.n)), block(kBlock);
  hipStream_t s = as_stream(stream);
  const bool plain = A.plain && A.plain_x;
  if (g.kind == SUFHIP_CHAIN_CUBIC && plain)
    hipLaunchKernelGGL((gate_chain_kernel<SUFHIP_CHAIN_CUBIC, true>), grid, block, 0, s, A);
  else if (g.kind == SUFHIP_CHAIN_CUBIC)
    hipLaunchKernelGGL((gate_chain_kernel<SUFHIP_CHAIN_CUBIC, false>), grid, block, 0, s, A);
  else if (g.kind == SUFHIP_CHAIN_RECIP && plain)
    hipLaunchKernelGGL((gate_chain_kernel<SUFHIP_CHAIN_RECIP, true>), grid, block, 0, s, A);
  else if (g.kind == SUFHIP_CHAIN_RECIP)
    hipLaunchKernelGGL((gate_chain_kernel<SUFHIP_CHAIN_RECIP, false>), grid, block, 0, s, A);
  else if (plain)
    hipLaunchKernelGGL((gate_chain_kernel<SUFHIP_CHAIN_RSQRT, true>), grid, block, 0, s, A);
  else
    hipLaunchKernelGGL((gate_chain_kernel<SUFHIP_CHAIN_RSQRT, false>), grid, block, 0, s, A);
  return check_launch("gate_chain_kernel");
}

}  // extern "C"
