// Balanced base-256 digit planes for the exact int8 matrix-core products
// over Z_2^64 (matmul_public.hip, matmul_mfma.hip, beaver_mfma2.hip).
//
// v = sum_{i<8} d_i 256^i mod 2^64 with d_i in [-128, 127]: d_i is the low
// byte as a signed value and v becomes (v - d_i) / 256.  A k-blocked plane
// stores a [rows x K] operand as [K / 32][rows][32] int8, so the 32 rows x
// 32 k of one MFMA step are a contiguous 1 KB block and one 16-byte load per
// lane fetches its row's half of it.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "suf_hip.h"

namespace sufhip {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kDigitPlanes = 8;

// The eight digits of v, each as its byte (two's complement) in d[i].
__device__ __forceinline__ void digits8(uint64_t v, uint32_t (&d)[kDigitPlanes]) {
#pragma unroll
  for (int i = 0; i < kDigitPlanes; ++i) {
    const uint32_t b = uint32_t(v) & 0xffu;
    d[i] = b;
    v = (v >> 8) + (b >> 7);  // borrow when the digit is negative
  }
}

// Byte offset of (row, k) in a k-blocked plane of `rows` rows.
__device__ __forceinline__ size_t kblock_off(size_t row, int k, size_t rows) {
  return (size_t(k >> 5) * rows + row) * 32 + size_t(k & 31);
}

__device__ __forceinline__ v4i load16(const int8_t* p) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  v4i r;
  r.x = int(u.x);
  r.y = int(u.y);
  r.z = int(u.z);
  r.w = int(u.w);
  return r;
}

// Party p's element i of a producer's output into its sufhip_x_planes
// (rows = the output's row count).
__device__ __forceinline__ void put_x_digits(const sufhip_x_planes& xp, size_t rows, size_t i,
                                             int p, uint64_t v) {
  const size_t cols = size_t(xp.cols);
  const size_t m = i / cols;
  const int k = int(i - m * cols);
  const size_t off = kblock_off(size_t(p) * rows + m, k, 2 * rows);
  const size_t plane = 2 * rows * cols;
  uint32_t d[kDigitPlanes];
  digits8(v, d);
#pragma unroll
  for (int q = 0; q < kDigitPlanes; ++q) xp.planes[q * plane + off] = int8_t(d[q]);
}

// Element i of a [batches][rows x cols] open into its sufhip_kb_planes.
__device__ __forceinline__ void put_kb_digits(const sufhip_kb_planes& o, size_t i, uint64_t v) {
  const size_t rc = size_t(o.rows) * size_t(o.cols);
  const size_t b = i / rc, rem = i - b * rc;
  const int r = int(rem / size_t(o.cols)), c = int(rem - size_t(r) * size_t(o.cols));
  const bool kc = o.k_is_col != 0;
  const size_t R = size_t(kc ? o.rows : o.cols);
  const size_t off = b * rc + kblock_off(size_t(kc ? r : c), kc ? c : r, R);
  const size_t plane = size_t(o.batches) * rc;
  uint32_t d[kDigitPlanes];
  digits8(v, d);
#pragma unroll
  for (int q = 0; q < kDigitPlanes; ++q) o.planes[q * plane + off] = int8_t(d[q]);
  if (o.planes_a0) {
    digits8(v + o.a0[i], d);
#pragma unroll
    for (int q = 0; q < kDigitPlanes; ++q) o.planes_a0[q * plane + off] = int8_t(d[q]);
  }
}

// Host: checks an optional sufhip_kb_planes for an open of n elements.
inline bool kb_planes_ok(const sufhip_kb_planes& o, size_t n) {
  if (!o.planes) return !o.planes_a0;
  if ((o.planes_a0 == nullptr) != (o.a0 == nullptr)) return false;
  return o.batches >= 1 && o.rows >= 32 && o.cols >= 32 && o.rows % 32 == 0 &&
         o.cols % 32 == 0 && size_t(o.batches) * size_t(o.rows) * size_t(o.cols) == n &&
         (reinterpret_cast<uintptr_t>(o.planes) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(o.planes_a0) & 15) == 0;
}

// Host: checks an optional sufhip_x_planes for an output of n elements.
inline bool x_planes_ok(const sufhip_x_planes& xp, size_t n) {
  if (!xp.planes) return true;
  if (xp.cols < 32 || xp.cols % 32 || n % size_t(xp.cols)) return false;
  const size_t rows = n / size_t(xp.cols);
  return rows % 32 == 0 && (reinterpret_cast<uintptr_t>(xp.planes) & 15) == 0;
}

}  // namespace sufhip
