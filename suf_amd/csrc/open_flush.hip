// One flush of a two-party open collector on the GPU: the device path of
// OpenCollector::flush (src/runtime/open_collector.cpp:357-791) for both
// parties in one process.  The requests' shares are gathered into one
// bucket per party (sufhip_stage_hatx, up to 64 requests a launch), party
// 1's bucket is packed to eff_bits -- the message it sends
// (launch_pack_eff_bits_kernel) -- and party 0's view adds that unpacked
// message to its own shares (launch_unpack_add_mod_kernel, or the
// sign-extending form).  Party 0's message is not formed: with both parties
// in one process the opened values are shared, and nothing would read it.
// That is 2 * ceil(count / 64) gather launches, one pack and one unpack-add
// (four launches for up to 64 requests).  The opened values stay on the
// device, back to back in request order, for the PFSS evaluation that
// consumes them (OpenCollector::view_device_u64).
#include <hip/hip_runtime.h>

#include <string>

#include "suf_hip.h"
#include "sufhip_internal.hpp"

namespace sufhip {
namespace {

size_t packed_words_of(size_t n, int eff_bits) {
  return (n * size_t(eff_bits) + 63) / 64;
}

}  // namespace
}  // namespace sufhip

using namespace sufhip;

extern "C" {

size_t sufhip_open_flush2_work_bytes(size_t total, int eff_bits) {
  if (eff_bits < 1 || eff_bits > 64) return 0;
  return 2 * total * 8 + (packed_words_of(total, eff_bits) + 1) * 8;
}

int sufhip_open_flush2(const sufhip_open_req* reqs, int count, int eff_bits, int ring_bits,
                       int sign_extend, uint64_t* d_opened, void* d_work, size_t work_bytes,
                       void* stream) {
  SUFHIP_REQUIRE(count >= 0 && (count == 0 || reqs), "sufhip_open_flush2: bad requests");
  SUFHIP_REQUIRE(eff_bits >= 1 && eff_bits <= 64 && ring_bits >= 1 && ring_bits <= 64,
                 "sufhip_open_flush2: eff_bits and ring_bits in [1, 64]");
  size_t total = 0;
  for (int i = 0; i < count; ++i) {
    SUFHIP_REQUIRE(reqs[i].len == 0 || (reqs[i].share[0] && reqs[i].share[1]),
                   "sufhip_open_flush2: request " + std::to_string(i) + " has a null share");
    total += reqs[i].len;
  }
  if (total == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_opened && d_work, "sufhip_open_flush2: null output or workspace");
  SUFHIP_REQUIRE(work_bytes >= sufhip_open_flush2_work_bytes(total, eff_bits),
                 "sufhip_open_flush2: workspace smaller than sufhip_open_flush2_work_bytes()");
  SUFHIP_REQUIRE((reinterpret_cast<uintptr_t>(d_work) & 7) == 0,
                 "sufhip_open_flush2: workspace must be 8-byte aligned");
  uint64_t* bucket[2] = {static_cast<uint64_t*>(d_work), static_cast<uint64_t*>(d_work) + total};
  uint64_t* msg1 = bucket[1] + total;
  // Gather both parties' shares, 64 requests per launch and party.
  for (int p = 0; p < 2; ++p) {
    size_t pos = 0;
    for (int base = 0; base < count; base += SUFHIP_STAGE_MAX_SEGS) {
      const int m = count - base < SUFHIP_STAGE_MAX_SEGS ? count - base : SUFHIP_STAGE_MAX_SEGS;
      sufhip_stage_seg segs[SUFHIP_STAGE_MAX_SEGS];
      for (int i = 0; i < m; ++i) {
        const sufhip_open_req& r = reqs[base + i];
        segs[i] = sufhip_stage_seg{r.share[p], r.len, pos, 64};
        pos += r.len;
      }
      if (int rc = sufhip_stage_hatx(segs, m, bucket[p], total, stream)) return rc;
    }
  }
  // Party 1's message; party 0 opens with it.
  if (int rc = sufhip_pack_eff_bits(bucket[1], eff_bits, msg1, total, stream)) return rc;
  const uint64_t mask = ring_bits >= 64 ? ~uint64_t(0) : (uint64_t(1) << ring_bits) - 1;
  return sign_extend
             ? sufhip_unpack_add_to_signed(bucket[0], msg1, eff_bits, d_opened, total, ring_bits,
                                           mask, stream)
             : sufhip_unpack_add_mod(bucket[0], msg1, eff_bits, d_opened, total, ring_bits, mask,
                                     stream);
}

}  // extern "C"
