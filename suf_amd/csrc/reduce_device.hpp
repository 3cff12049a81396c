// Wave64 and workgroup sums of u64 words (mod 2^64) for the row kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sufhip {

// Sum over the 64 lanes of a wavefront, returned to every lane (xor
// butterfly on the two 32-bit halves).
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t lo = __shfl_xor(uint32_t(v), off, 64);
    const uint32_t hi = __shfl_xor(uint32_t(v >> 32), off, 64);
    v += uint64_t(lo) | uint64_t(hi) << 32;
  }
  return v;
}

// Sums of two words over a workgroup of kWaves wavefronts, returned to every
// thread.  red: LDS scratch [2][kWaves]; contains two barriers, so every
// thread of the workgroup must call it.
template <int kWaves>
__device__ __forceinline__ void block_sum2_u64(uint64_t& a, uint64_t& b, uint64_t (*red)[kWaves]) {
  a = wave_sum_u64(a);
  b = wave_sum_u64(b);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[0][w] = a;
    red[1][w] = b;
  }
  __syncthreads();
  a = 0;
  b = 0;
#pragma unroll
  for (int k = 0; k < kWaves; ++k) {
    a += red[0][k];
    b += red[1][k];
  }
  __syncthreads();
}

}  // namespace sufhip
