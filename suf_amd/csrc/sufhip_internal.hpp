// Internal helpers shared by the HIP translation units of libsuf_hip.so:
// status codes and the thread-local error message behind the C ABI, HIP
// error checks, and launch-shape helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "suf_hip.h"

namespace sufhip {

void set_error(const std::string& msg);
void clear_error();

// Returns SUFHIP_ERR_HIP with a message when `st` is not hipSuccess.
int hip_status(hipError_t st, const char* what);

#define SUFHIP_CHECK(expr, what)                                \
  do {                                                          \
    hipError_t _st = (expr);                                    \
    if (_st != hipSuccess) return ::sufhip::hip_status(_st, what); \
  } while (0)

#define SUFHIP_REQUIRE(cond, msg)                 \
  do {                                            \
    if (!(cond)) {                                \
      ::sufhip::set_error(msg);                   \
      return SUFHIP_ERR_INVALID;                  \
    }                                             \
  } while (0)

// Checks the launch that was just issued.
int check_launch(const char* what);

// sufhip_set_keystream_per_party's policy: true when every two-party LUT
// kernel computes each party's keystream from its own blob.
bool keystream_per_party();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline unsigned int grid_for(size_t n, unsigned int block) {
  size_t g = (n + block - 1) / block;
  return static_cast<unsigned int>(g);
}

// Upper bound on grid.x for 1-D launches (the hardware limit is 2^31-1; keep
// a margin and switch to grid-stride loops above it).
constexpr size_t kMaxGrid = 1u << 30;

}  // namespace sufhip
