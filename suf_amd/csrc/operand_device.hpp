// The generalised two-party operands of the C ABI (sufhip_term2,
// sufhip_operand2 in suf_hip.h): device-side evaluation and host-side
// argument checks, shared by the kernels that read operands.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "suf_hip.h"
#include "sufhip_internal.hpp"

namespace sufhip {

__device__ __forceinline__ uint64_t term_at(const sufhip_term2& t, int p, size_t i) {
  // Clamped to the arrays' rows whether or not the row comes from an index.
  size_t j = i;
  if (t.index) {
    const int32_t r = t.index[i];
    j = r < 0 ? 0 : size_t(r);
  }
  if (j >= t.len) j = t.len - 1;
  uint64_t v = t.p[p][j * t.stride + t.off];
  if (t.mul) v *= t.mul;
  v <<= t.shift;
  return t.negate ? uint64_t(0) - v : v;
}

__device__ __forceinline__ uint64_t operand_at(const sufhip_operand2& o, int p, size_t i) {
  uint64_t v = p == 0 ? o.party0_const : 0;
  if (o.t[0].p[0]) v += term_at(o.t[0], p, i);
  if (o.t[1].p[0]) v += term_at(o.t[1], p, i);
  return v;
}


// Host-side checks of the generalised operands (see sufhip_term2 in suf_hip.h).
inline int check_term(const sufhip_term2& t, size_t n, bool allow_shift, const char* what) {
  if (!t.p[0] && !t.p[1]) return SUFHIP_OK;
  if (!t.p[0] || !t.p[1]) {
    set_error(std::string(what) + ": a term needs both parties' pointers or neither");
    return SUFHIP_ERR_INVALID;
  }
  if (t.stride < 1 || t.off >= t.stride || t.shift < 0 || t.shift > 63 ||
      (!allow_shift && (t.shift != 0 || t.negate || t.mul > 1))) {
    set_error(std::string(what) + ": bad term stride/offset/shift/negate/mul");
    return SUFHIP_ERR_INVALID;
  }
  if (t.len == 0 || (!t.index && t.len < n)) {
    set_error(std::string(what) + ": term len smaller than the element count");
    return SUFHIP_ERR_INVALID;
  }
  return SUFHIP_OK;
}

inline int check_operand(const sufhip_operand2& o, size_t n, const char* what) {
  for (int k = 0; k < 2; ++k)
    if (int rc = check_term(o.t[k], n, true, what)) return rc;
  return SUFHIP_OK;
}

}  // namespace sufhip
