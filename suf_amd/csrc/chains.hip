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

// Two forms.  The narrow one runs two 512-lane workgroups per CU on the
// two-table AES span (64 KB of LDS each).  The wide one runs one 1024-lane
// workgroup per CU (four waves per SIMD, at most 128 VGPRs) on the
// four-table AES (128 KB): two 3-input XORs per column where the two-table
// span needs a rotate and three XORs, a quarter fewer VALU operations per
// round on the pipe that bounds the chain, at twice the staging per
// workgroup and without a second workgroup to overlap it.  Batches of at
// least two full passes of the chip take the wide form.
template <bool kWide>
struct ChainCfg {
  static constexpr int kBlock = 512;
  using Aes = AesLds2<32>;
  static constexpr int kTabWords = Aes::kSpanWords;
  static constexpr int kPerCu = 2;
};
template <>
struct ChainCfg<true> {
  static constexpr int kBlock = 1024;
  using Aes = AesLds4;
  static constexpr int kTabWords = Aes::kWords;
  static constexpr int kPerCu = 1;
};

// kPlain: x and the triple shares are plain arrays (ChainArgs::plain and
// plain_x), read through plain pointers.
template <int kKind, bool kPlain, bool kWide>
__global__ void __launch_bounds__(ChainCfg<kWide>::kBlock) gate_chain_kernel(ChainArgs A) {
  using Cfg = ChainCfg<kWide>;
  using ChainAes = typename Cfg::Aes;
  constexpr int kBlock = Cfg::kBlock;
  constexpr int W = kKind == SUFHIP_CHAIN_CUBIC ? 4 : 2;
  constexpr int kProds = chain_products<kKind>();
  __shared__ __align__(16) uint32_t tab[Cfg::kTabWords];
  __shared__ ChainLds L;
  __shared__ TruncHdr th[kProds][2];
  // Staging in one pass: the tables' slots, the LUT items and the gates'
  // key headers all loaded before the first LDS store.
  {
    TruncHdrStager<kProds> hs;
    typename ChainAes::template Filler<kBlock> tf;
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

int cu_count() {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  return cus;
}

template <int kKind, bool kPlain>
void launch_chain(const ChainArgs& A, hipStream_t s) {
  const size_t cus = size_t(cu_count());
  const bool wide = A.n >= 2 * cus * size_t(ChainCfg<true>::kBlock);
  const size_t block = wide ? ChainCfg<true>::kBlock : ChainCfg<false>::kBlock;
  const size_t cap = cus * (wide ? ChainCfg<true>::kPerCu : ChainCfg<false>::kPerCu);
  const size_t need = (A.n + block - 1) / block;
  const dim3 grid(unsigned(need < cap ? need : cap));
  if (wide)
    hipLaunchKernelGGL((gate_chain_kernel<kKind, kPlain, true>), grid, dim3(block), 0, s, A);
  else
    hipLaunchKernelGGL((gate_chain_kernel<kKind, kPlain, false>), grid, dim3(block), 0, s, A);
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
  hipStream_t s = as_stream(stream);
  const bool plain = A.plain && A.plain_x;
  if (g.kind == SUFHIP_CHAIN_CUBIC && plain)
    launch_chain<SUFHIP_CHAIN_CUBIC, true>(A, s);
  else if (g.kind == SUFHIP_CHAIN_CUBIC)
    launch_chain<SUFHIP_CHAIN_CUBIC, false>(A, s);
  else if (g.kind == SUFHIP_CHAIN_RECIP && plain)
    launch_chain<SUFHIP_CHAIN_RECIP, true>(A, s);
  else if (g.kind == SUFHIP_CHAIN_RECIP)
    launch_chain<SUFHIP_CHAIN_RECIP, false>(A, s);
  else if (plain)
    launch_chain<SUFHIP_CHAIN_RSQRT, true>(A, s);
  else
    launch_chain<SUFHIP_CHAIN_RSQRT, false>(A, s);
  return check_launch("gate_chain_kernel");
}

}  // extern "C"
