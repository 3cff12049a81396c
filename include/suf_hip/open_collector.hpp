// Batched opens on the GPU, both parties in one process: the device path of
// SUF's runtime::OpenCollector (include/runtime/open_collector.hpp:52-163,
// src/runtime/open_collector.cpp:324-985) with the opened values kept on the
// device (the reference's SUF_OPEN_PACK_DEVICE / DEVICE_KEEP_OPENED path),
// where the PFSS evaluation that consumes x^ reads them.
//
// Method names, handles, generations, limits and stats follow the
// reference.  The differences come from holding both parties' shares:
//   * reserve() hands out device views for party 0 and party 1 (the
//     caller's kernels fill them); enqueue() takes two device share vectors,
//     which it reads at flush() without copying them first;
//   * flush() takes no party or channel: party 1's shares are packed to
//     eff_bits (the message it would send) and party 0 adds that unpacked
//     message to its own, on the collector's stream (sufhip_open_flush2:
//     2 * ceil(requests / 64) gather launches, one pack, one unpack-add).  It returns without waiting for the GPU:
//     view_device_u64() pointers are valid in that stream's order; view() and
//     view_u64() copy the opened values to the host once per flush and wait.
//   * Stats::wire_bytes_sent counts one party's packed message, the bytes it
//     would put on the channel; flush_ns is the host time to issue a flush.
//
// A flush's opened value is (s0 + (s1 mod 2^eff_bits)) mod 2^ring_bits:
// exact when eff_bits >= ring_bits (the reference's fixed packing packs to
// the ring's width, the default here) or when party 1's shares fit eff_bits
// (its dynamic packing).  view() sign-extends from ring_bits
// (proto::to_signed).
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <vector>

namespace suf_hip {

enum class OpenKind : uint8_t { kOther = 0, kBeaver = 1, kMask = 2, kCount = 3 };

struct OpenHandle {
  uint64_t gen = 0;  // generation at enqueue; a flush or clear() starts the next one
  size_t offset = 0;
  size_t len = 0;
};

// A read-only window onto host memory owned by the collector.
template <typename T>
struct ConstView {
  const T* ptr = nullptr;
  size_t n = 0;
  const T* data() const { return ptr; }
  size_t size() const { return n; }
  bool empty() const { return n == 0; }
  const T& operator[](size_t i) const { return ptr[i]; }
  const T* begin() const { return ptr; }
  const T* end() const { return ptr + n; }
};

class DeviceOpenCollector {
 public:
  struct Stats {
    size_t flushes = 0;
    size_t opened_words = 0;
    std::array<size_t, static_cast<size_t>(OpenKind::kCount)> opened_words_by_kind{};
    uint64_t wire_bytes_sent = 0;
    size_t max_pending_words = 0;
    uint64_t flush_ns = 0;
  };
  struct Limits {
    size_t max_pending_words = size_t(1) << 24;
  };
  // Device views of a reserved open, one per party; valid until the next
  // flush() or clear().  The memory is reused by the next flush's reserves,
  // so fill them on the collector's stream (or a stream ordered after it).
  struct Reserve {
    OpenHandle handle;
    uint64_t* diff[2] = {nullptr, nullptr};
  };

  // ring_bits: shares live in Z_2^ring_bits; eff_bits: the packed width of
  // each party's message, 0 for ring_bits.
  explicit DeviceOpenCollector(int ring_bits = 64, int eff_bits = 0);
  ~DeviceOpenCollector();
  DeviceOpenCollector(const DeviceOpenCollector&) = delete;
  DeviceOpenCollector& operator=(const DeviceOpenCollector&) = delete;

  // Both parties' shares of one vector, device pointers; they must hold
  // their values until the flush that reads them has run on the stream.
  OpenHandle enqueue(const uint64_t* d_share0, const uint64_t* d_share1, size_t len,
                     OpenKind kind = OpenKind::kOther);
  Reserve reserve(size_t len, OpenKind kind = OpenKind::kOther);
  void flush();

  size_t pending_words() const { return pending_words_; }
  const Limits& limits() const { return limits_; }
  void set_limits(const Limits& lim) { limits_ = lim; }

  ConstView<int64_t> view(const OpenHandle& h) const;
  ConstView<uint64_t> view_u64(const OpenHandle& h) const;
  const uint64_t* view_device_u64(const OpenHandle& h) const;

  bool empty() const { return requests_.empty(); }
  bool has_pending() const { return !requests_.empty(); }
  bool ready(const OpenHandle& h) const;
  void clear();

  // Non-owning; nullptr is the default stream.
  void set_cuda_stream(void* stream) { stream_ = stream; }
  const Stats& stats() const { return stats_; }
  void reset_stats() { stats_ = Stats{}; }
  int ring_bits() const { return ring_bits_; }
  int eff_bits() const { return eff_bits_; }

 private:
  struct Request {
    const uint64_t* share[2];
    size_t len;
    OpenKind kind;
  };
  // Pending arena for reserve(): device chunks per party, kept across
  // flushes so a steady stream of opens allocates nothing.
  struct Chunk {
    uint64_t* d[2] = {nullptr, nullptr};
    size_t cap = 0, used = 0;
  };
  void grow(void** d, size_t* cap, size_t bytes);

  int ring_bits_, eff_bits_;
  void* stream_ = nullptr;
  Limits limits_;
  Stats stats_;
  std::vector<Request> requests_;
  std::vector<Chunk> chunks_;
  size_t pending_words_ = 0;
  uint64_t generation_ = 0;
  uint64_t opened_generation_ = ~uint64_t(0);
  bool opened_ready_ = false;
  size_t opened_words_ = 0;
  void* d_opened_ = nullptr;
  size_t opened_cap_ = 0;
  void* d_work_ = nullptr;
  size_t work_cap_ = 0;
  mutable std::vector<uint64_t> host_u64_;
  mutable std::vector<int64_t> host_signed_;
  mutable bool host_u64_ok_ = false, host_signed_ok_ = false;
};

}  // namespace suf_hip
