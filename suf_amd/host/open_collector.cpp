// DeviceOpenCollector (include/suf_hip/open_collector.hpp): request
// bookkeeping on the host, the flush in sufhip_open_flush2.
#include "suf_hip/open_collector.hpp"

#include <chrono>
#include <stdexcept>
#include <string>

#include "suf_hip.h"

namespace suf_hip {

namespace {

void hip_ok(int rc, const char* what) {
  if (rc != SUFHIP_OK) {
    const char* m = sufhip_last_error();
    throw std::runtime_error(std::string("DeviceOpenCollector: ") + what + ": " +
                             (m ? m : "sufhip error"));
  }
}

constexpr size_t kChunkWords = size_t(1) << 20;

}  // namespace

DeviceOpenCollector::DeviceOpenCollector(int ring_bits, int eff_bits)
    : ring_bits_(ring_bits), eff_bits_(eff_bits == 0 ? ring_bits : eff_bits) {
  if (ring_bits_ < 1 || ring_bits_ > 64 || eff_bits_ < 1 || eff_bits_ > 64)
    throw std::runtime_error("DeviceOpenCollector: ring_bits and eff_bits in [1, 64]");
}

DeviceOpenCollector::~DeviceOpenCollector() {
  // Frees wait for the device, so no flush still reads these buffers.
  for (Chunk& c : chunks_)
    for (int p = 0; p < 2; ++p)
      if (c.d[p]) sufhip_free(c.d[p]);
  if (d_opened_) sufhip_free(d_opened_);
  if (d_work_) sufhip_free(d_work_);
}

OpenHandle DeviceOpenCollector::enqueue(const uint64_t* d_share0, const uint64_t* d_share1,
                                        size_t len, OpenKind kind) {
  if (len && (!d_share0 || !d_share1))
    throw std::runtime_error("DeviceOpenCollector: null share");
  if (limits_.max_pending_words > 0 && pending_words_ + len > limits_.max_pending_words)
    throw std::runtime_error("DeviceOpenCollector: pending open budget exceeded");
  OpenHandle h;
  h.gen = generation_;
  h.offset = pending_words_;
  h.len = len;
  if (static_cast<size_t>(kind) >= static_cast<size_t>(OpenKind::kCount)) kind = OpenKind::kOther;
  requests_.push_back(Request{{d_share0, d_share1}, len, kind});
  pending_words_ += len;
  if (pending_words_ > stats_.max_pending_words) stats_.max_pending_words = pending_words_;
  return h;
}

DeviceOpenCollector::Reserve DeviceOpenCollector::reserve(size_t len, OpenKind kind) {
  if (limits_.max_pending_words > 0 && pending_words_ + len > limits_.max_pending_words)
    throw std::runtime_error("DeviceOpenCollector: pending open budget exceeded");
  Chunk* c = nullptr;
  for (Chunk& k : chunks_)
    if (k.cap - k.used >= len) {
      c = &k;
      break;
    }
  if (!c) {
    Chunk k;
    k.cap = len > kChunkWords ? len : kChunkWords;
    for (int p = 0; p < 2; ++p) {
      void* d = nullptr;
      const int rc = sufhip_malloc(&d, k.cap * sizeof(uint64_t));
      if (rc != SUFHIP_OK) {
        if (k.d[0]) sufhip_free(k.d[0]);
        hip_ok(rc, "pending arena");
      }
      k.d[p] = static_cast<uint64_t*>(d);
    }
    chunks_.push_back(k);
    c = &chunks_.back();
  }
  Reserve r;
  r.diff[0] = c->d[0] + c->used;
  r.diff[1] = c->d[1] + c->used;
  c->used += len;
  r.handle = enqueue(r.diff[0], r.diff[1], len, kind);
  return r;
}

void DeviceOpenCollector::grow(void** d, size_t* cap, size_t bytes) {
  if (bytes <= *cap) return;
  if (*d) hip_ok(sufhip_free(*d), "free");
  *d = nullptr;
  *cap = 0;
  hip_ok(sufhip_malloc(d, bytes), "device allocation");
  *cap = bytes;
}

void DeviceOpenCollector::flush() {
  if (requests_.empty()) return;
  const auto t0 = std::chrono::steady_clock::now();
  const size_t total = pending_words_;
  std::vector<sufhip_open_req> reqs;
  reqs.reserve(requests_.size());
  for (const Request& r : requests_) {
    sufhip_open_req q{};
    q.share[0] = r.share[0];
    q.share[1] = r.share[1];
    q.len = r.len;
    reqs.push_back(q);
  }
  if (total) {
    grow(&d_opened_, &opened_cap_, total * sizeof(uint64_t));
    const size_t wb = sufhip_open_flush2_work_bytes(total, eff_bits_);
    grow(&d_work_, &work_cap_, wb);
    hip_ok(sufhip_open_flush2(reqs.data(), int(reqs.size()), eff_bits_, ring_bits_, 0,
                              static_cast<uint64_t*>(d_opened_), d_work_, work_cap_, stream_),
           "flush");
  }
  stats_.flushes += 1;
  stats_.opened_words += total;
  for (const Request& r : requests_) stats_.opened_words_by_kind[size_t(r.kind)] += r.len;
  stats_.wire_bytes_sent += uint64_t((total * size_t(eff_bits_) + 63) / 64) * 8;
  requests_.clear();
  pending_words_ = 0;
  for (Chunk& c : chunks_) c.used = 0;
  opened_words_ = total;
  opened_ready_ = true;
  opened_generation_ = generation_;
  generation_ += 1;
  host_u64_ok_ = host_signed_ok_ = false;
  stats_.flush_ns += uint64_t(std::chrono::duration_cast<std::chrono::nanoseconds>(
                                  std::chrono::steady_clock::now() - t0)
                                  .count());
}

bool DeviceOpenCollector::ready(const OpenHandle& h) const {
  return opened_ready_ && h.gen == opened_generation_ && h.offset + h.len <= opened_words_;
}

const uint64_t* DeviceOpenCollector::view_device_u64(const OpenHandle& h) const {
  if (!ready(h) || !d_opened_) return nullptr;
  return static_cast<const uint64_t*>(d_opened_) + h.offset;
}

ConstView<uint64_t> DeviceOpenCollector::view_u64(const OpenHandle& h) const {
  if (!ready(h)) throw std::runtime_error("DeviceOpenCollector: view_u64 out of range");
  if (!host_u64_ok_) {
    host_u64_.resize(opened_words_);
    if (opened_words_) {
      hip_ok(sufhip_memcpy_d2h(host_u64_.data(), d_opened_, opened_words_ * sizeof(uint64_t),
                               stream_),
             "copy to host");
      hip_ok(sufhip_stream_synchronize(stream_), "sync");
    }
    host_u64_ok_ = true;
  }
  return ConstView<uint64_t>{host_u64_.data() + h.offset, h.len};
}

ConstView<int64_t> DeviceOpenCollector::view(const OpenHandle& h) const {
  if (!ready(h)) throw std::runtime_error("DeviceOpenCollector: view out of range");
  if (!host_signed_ok_) {
    view_u64(h);
    host_signed_.resize(opened_words_);
    const int k = ring_bits_;
    for (size_t i = 0; i < opened_words_; ++i) {
      const uint64_t v = host_u64_[i];
      host_signed_[i] = k >= 64 ? int64_t(v) : int64_t(v << (64 - k)) >> (64 - k);
    }
    host_signed_ok_ = true;
  }
  return ConstView<int64_t>{host_signed_.data() + h.offset, h.len};
}

void DeviceOpenCollector::clear() {
  requests_.clear();
  pending_words_ = 0;
  for (Chunk& c : chunks_) c.used = 0;
  opened_ready_ = false;
  opened_generation_ = ~uint64_t(0);
  opened_words_ = 0;
  host_u64_ok_ = host_signed_ok_ = false;
  generation_ += 1;
}

}  // namespace suf_hip
