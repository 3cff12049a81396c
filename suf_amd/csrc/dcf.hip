// myl7/fss v0.7.1 DCF (lambda = 16, AES-128-MMO PRG) on CDNA4: batched key
// generation and evaluation over SUF's myl7 adapter key blobs.
//
// Evaluation (third_party/myl7_fss/src/dcf.c:146-193) walks the tree from
// bit in_bits-1 down to bit 0.  At each level the reference expands the seed
// into four blocks (sl, vl, sr, vr) with four AES calls, then keeps only the
// side selected by the input bit.  Here each lane computes just the two
// blocks on that side -- AES_{K_{2b}} for the next seed and AES_{K_{2b+1}}
// for the value block, b = x_i -- which halves the AES work without changing
// any output byte.  When only share byte 0 bit 0 is needed (the
// eval_dcf_many_u64 contract, include/proto/myl7_fss_backend.hpp:88-99), the
// value block is reduced to its first byte: bit 0 of a sum or XOR depends
// only on bit 0 of the terms, and bit 0 of -v equals bit 0 of v, so this
// holds for both output groups.
//
// One element per lane; each lane streams its own key front to back
// (33 bytes per level), so successive levels hit the same cache lines.
//
// The evaluation kernels run 1024 lanes per CU (four waves per SIMD): their
// walks keep the round keys in scalar registers and fit in the 128 VGPRs
// that allows, and the table lookups that bound them overlap better with
// more waves.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstring>

#include "dcf_device.hpp"

namespace sufhip {
namespace {

struct DcfEvalArgs {
  Prg4 prg;
  const uint8_t* keys;
  const uint64_t* xs;
  void* out;
  size_t key_bytes;
  size_t n;
  int broadcast;
  int in_bits;
  int chunks;     // chunks to evaluate (1 for the bit modes)
  int out_bytes;  // bytes per element (OUT_BYTES)
  DcfKeySel key_sel;  // the bit modes' round keys (scalar loads)
};

constexpr int kDcfBitBlock = 1024;

template <int kMode>
__global__ void __launch_bounds__(kDcfBitBlock) dcf_eval_bit_kernel(DcfEvalArgs a) {
  SUFHIP_DCF_TABLE_SETUP();
  const KeySelPtr keys = kernarg_key_sel(offsetof(DcfEvalArgs, key_sel));
  const size_t stride = size_t(gridDim.x) * kDcfBitBlock;
  for (size_t base = size_t(blockIdx.x) * kDcfBitBlock; base < a.n; base += stride) {
    const size_t e = base + threadIdx.x;
    uint32_t bit = 0;
    if (e < a.n) {
      const uint8_t* key = a.broadcast ? a.keys : a.keys + e * a.key_bytes;
      const uint32_t party = key[2] & 1u;
      uint64_t x = a.xs[e];
      if (a.in_bits < 64) x &= (uint64_t(1) << a.in_bits) - 1;
      bit = walk_bit(aes, keys, key + 8, a.in_bits, x, party);
    }
    if constexpr (kMode == SUFHIP_DCF_OUT_BIT) {
      if (e < a.n) static_cast<uint8_t*>(a.out)[e] = uint8_t(bit);
    } else {
      // Waves cover 64 consecutive elements starting at a multiple of 64.
      const uint64_t word = __ballot(bit != 0);
      if ((threadIdx.x & 63) == 0 && e < a.n) static_cast<uint64_t*>(a.out)[e >> 6] = word;
    }
  }
}

template <int kGroup>
__global__ void __launch_bounds__(kDcfBitBlock) dcf_eval_bytes_kernel(DcfEvalArgs a) {
  SUFHIP_DCF_TABLE_SETUP();
  const KeySelPtr keys = kernarg_key_sel(offsetof(DcfEvalArgs, key_sel));
  const size_t stride = size_t(gridDim.x) * kDcfBitBlock;
  const size_t chunk_bytes = 32 + 33 * size_t(a.in_bits);
  for (size_t e = size_t(blockIdx.x) * kDcfBitBlock + threadIdx.x; e < a.n; e += stride) {
    const uint8_t* key = a.broadcast ? a.keys : a.keys + e * a.key_bytes;
    const uint32_t party = key[2] & 1u;
    uint64_t x = a.xs[e];
    if (a.in_bits < 64) x &= (uint64_t(1) << a.in_bits) - 1;
    uint8_t* out = static_cast<uint8_t*>(a.out) + e * size_t(a.out_bytes);
    for (int c = 0; c < a.chunks; ++c) {
      const bool more = (c + 1) * chunk_bytes + 8 < a.key_bytes;
      U128 r = walk_full<kGroup>(aes, keys, key + 8 + c * chunk_bytes, a.in_bits, x, party, more);
      const int base = 16 * c;
      const int take = a.out_bytes - base < 16 ? a.out_bytes - base : 16;
      for (int b = 0; b < take; ++b) {
        const uint64_t word = b < 8 ? r.lo : r.hi;
        out[base + b] = uint8_t(word >> (8 * (b & 7)));
      }
    }
  }
}

// ---------------------------------------------------------------- keygen --

struct DcfGenArgs {
  Prg4 prg;
  const uint64_t* alpha;
  const uint8_t* payload;
  const uint8_t* seeds;
  uint8_t* keys0;
  uint8_t* keys1;
  size_t key_bytes;
  size_t n;
  int payload_bcast;
  int payload_len;
  int in_bits;
  int chunks;
};

// myl7 dcf_gen (third_party/myl7_fss/src/dcf.c:42-142) for kLtAlpha, one key
// pair per lane, written in the adapter layout (myl7_fss_backend.hpp:156-210).
template <int kGroup>
__global__ void __launch_bounds__(kDcfBlock) dcf_gen_kernel(DcfGenArgs a) {
  SUFHIP_DCF_LDS_SETUP(a.prg);
  const size_t stride = size_t(gridDim.x) * kDcfBlock;
  for (size_t e = size_t(blockIdx.x) * kDcfBlock + threadIdx.x; e < a.n; e += stride) {
    const uint8_t* pay = a.payload_bcast ? a.payload : a.payload + e * size_t(a.payload_len);
    gen_key<kGroup>(aes, rkl, a.in_bits, a.chunks, a.payload_len, a.alpha[e], pay,
                    a.seeds + e * size_t(a.chunks) * 32, a.keys0 + e * a.key_bytes,
                    a.keys1 + e * a.key_bytes);
  }
}

constexpr size_t kMaxElems = size_t(1) << 38;

}  // namespace
}  // namespace sufhip

using namespace sufhip;

extern "C" {

size_t sufhip_dcf_key_bytes(int in_bits, int payload_len) {
  if (in_bits <= 0 || in_bits > 64 || payload_len <= 0) return 0;
  const size_t chunks = (size_t(payload_len) + 15) / 16;
  if (chunks > 255) return 0;
  return 8 + chunks * (32 + 33 * size_t(in_bits));
}

int sufhip_dcf_gen(int group, int in_bits, const uint8_t* prg_state, const uint64_t* d_alpha,
                   const uint8_t* d_payload, int payload_len, int payload_broadcast,
                   const uint8_t* d_seeds, size_t n, uint8_t* d_keys0, uint8_t* d_keys1,
                   void* stream) {
  SUFHIP_REQUIRE(group == SUFHIP_GROUP_XOR || group == SUFHIP_GROUP_ADD,
                 "sufhip_dcf_gen: unknown group");
  SUFHIP_REQUIRE(in_bits >= 1 && in_bits <= 64, "sufhip_dcf_gen: in_bits out of range");
  SUFHIP_REQUIRE(payload_len >= 1 && payload_len <= 255 * 16,
                 "sufhip_dcf_gen: payload_len out of range");
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(n < kMaxElems, "sufhip_dcf_gen: n too large");
  SUFHIP_REQUIRE(prg_state && d_alpha && d_payload && d_seeds && d_keys0 && d_keys1,
                 "sufhip_dcf_gen: null pointer");
  DcfGenArgs a{};
  fill_prg4(prg_state, &a.prg);
  a.alpha = d_alpha;
  a.payload = d_payload;
  a.seeds = d_seeds;
  a.keys0 = d_keys0;
  a.keys1 = d_keys1;
  a.key_bytes = sufhip_dcf_key_bytes(in_bits, payload_len);
  a.n = n;
  a.payload_bcast = payload_broadcast ? 1 : 0;
  a.payload_len = payload_len;
  a.in_bits = in_bits;
  a.chunks = (payload_len + 15) / 16;
  unsigned int g = 0;
  if (int rc = dcf_grid(n, &g)) return rc;
  if (group == SUFHIP_GROUP_XOR)
    hipLaunchKernelGGL((dcf_gen_kernel<SUFHIP_GROUP_XOR>), dim3(g), dim3(kDcfBlock), 0,
                       as_stream(stream), a);
  else
    hipLaunchKernelGGL((dcf_gen_kernel<SUFHIP_GROUP_ADD>), dim3(g), dim3(kDcfBlock), 0,
                       as_stream(stream), a);
  return check_launch("dcf_gen_kernel");
}

int sufhip_dcf_eval(int group, int in_bits, int payload_len, const uint8_t* prg_state,
                    const uint8_t* d_keys, size_t key_bytes, int key_broadcast,
                    const uint64_t* d_xs, size_t n, int out_mode, int out_bytes, void* d_out,
                    void* stream) {
  SUFHIP_REQUIRE(group == SUFHIP_GROUP_XOR || group == SUFHIP_GROUP_ADD,
                 "sufhip_dcf_eval: unknown group");
  SUFHIP_REQUIRE(in_bits >= 1 && in_bits <= 64, "sufhip_dcf_eval: in_bits out of range");
  SUFHIP_REQUIRE(payload_len >= 1 && payload_len <= 255 * 16,
                 "sufhip_dcf_eval: payload_len out of range");
  SUFHIP_REQUIRE(key_bytes == sufhip_dcf_key_bytes(in_bits, payload_len),
                 "sufhip_dcf_eval: key_bytes does not match (in_bits, payload_len)");
  SUFHIP_REQUIRE(out_mode == SUFHIP_DCF_OUT_BIT || out_mode == SUFHIP_DCF_OUT_BYTES ||
                     out_mode == SUFHIP_DCF_OUT_PACKED,
                 "sufhip_dcf_eval: unknown out_mode");
  if (out_mode == SUFHIP_DCF_OUT_BYTES)
    SUFHIP_REQUIRE(out_bytes >= 1 && out_bytes <= payload_len,
                   "sufhip_dcf_eval: out_bytes must be in [1, payload_len]");
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(n < kMaxElems, "sufhip_dcf_eval: n too large");
  SUFHIP_REQUIRE(prg_state && d_keys && d_xs && d_out, "sufhip_dcf_eval: null pointer");
  DcfEvalArgs a{};
  fill_prg4(prg_state, &a.prg);
  a.keys = d_keys;
  a.xs = d_xs;
  a.out = d_out;
  a.key_bytes = key_bytes;
  a.n = n;
  a.broadcast = key_broadcast ? 1 : 0;
  a.in_bits = in_bits;
  a.chunks = 1;
  a.out_bytes = out_mode == SUFHIP_DCF_OUT_BYTES ? out_bytes : 1;
  hipStream_t s = as_stream(stream);
  fill_key_sel(a.prg, &a.key_sel);
  if (out_mode != SUFHIP_DCF_OUT_BYTES) {
    unsigned int g = 0;
    if (int rc = dcf_grid(n, &g, kDcfBitBlock)) return rc;
    const dim3 grid(g), block(kDcfBitBlock);
    if (out_mode == SUFHIP_DCF_OUT_BIT) {
      hipLaunchKernelGGL((dcf_eval_bit_kernel<SUFHIP_DCF_OUT_BIT>), grid, block, 0, s, a);
    } else {
      SUFHIP_REQUIRE((reinterpret_cast<uintptr_t>(d_out) & 7) == 0,
                     "sufhip_dcf_eval: packed output must be 8-byte aligned");
      hipLaunchKernelGGL((dcf_eval_bit_kernel<SUFHIP_DCF_OUT_PACKED>), grid, block, 0, s, a);
    }
  } else {
    unsigned int g = 0;
    if (int rc = dcf_grid(n, &g, kDcfBitBlock)) return rc;
    const dim3 grid(g), block(kDcfBitBlock);
    a.chunks = (out_bytes + 15) / 16;
    if (group == SUFHIP_GROUP_XOR)
      hipLaunchKernelGGL((dcf_eval_bytes_kernel<SUFHIP_GROUP_XOR>), grid, block, 0, s, a);
    else
      hipLaunchKernelGGL((dcf_eval_bytes_kernel<SUFHIP_GROUP_ADD>), grid, block, 0, s, a);
  }
  return check_launch("dcf_eval kernel");
}

}  // extern "C"
