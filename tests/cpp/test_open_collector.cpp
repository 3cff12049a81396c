// DeviceOpenCollector (include/suf_hip/open_collector.hpp).
//   test_open_collector cpu
//     handles, generations, the pending budget and the empty/ready/view
//     rules, with no GPU call (enqueue takes pointers without reading them).
//   test_open_collector gpu
//     secrets split into shares open to themselves through reserve() and
//     enqueue() requests mixed in one flush, over several flushes that reuse
//     the pending arena; views of an old generation are refused; the signed
//     view sign-extends from the ring; stats count words, kinds and the
//     packed message bytes.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "suf_hip.h"
#include "suf_hip/open_collector.hpp"

using namespace suf_hip;

static int g_fail = 0;
#define CHECK(cond, ...)                 \
  do {                                   \
    if (!(cond)) {                       \
      std::fprintf(stderr, __VA_ARGS__); \
      std::fprintf(stderr, "\n");        \
      ++g_fail;                          \
    }                                    \
  } while (0)

template <typename F>
static bool throws(F f) {
  try {
    f();
  } catch (const std::runtime_error&) {
    return true;
  }
  return false;
}

static void ok(int rc, const char* what) {
  if (rc != SUFHIP_OK) {
    const char* m = sufhip_last_error();
    throw std::runtime_error(std::string(what) + ": " + (m ? m : "?"));
  }
}

static void test_cpu() {
  DeviceOpenCollector c(50);
  CHECK(c.eff_bits() == 50 && c.ring_bits() == 50, "eff_bits defaults to ring_bits");
  CHECK(throws([] { DeviceOpenCollector bad(0); }), "ring_bits 0 accepted");
  CHECK(throws([] { DeviceOpenCollector bad(64, 65); }), "eff_bits 65 accepted");
  CHECK(c.empty() && !c.has_pending() && c.pending_words() == 0, "fresh collector not empty");
  // Enqueue records device pointers without touching them.
  static uint64_t fake[2][8];
  OpenHandle a = c.enqueue(fake[0], fake[1], 5, OpenKind::kMask);
  OpenHandle b = c.enqueue(fake[0], fake[1], 3, OpenKind::kBeaver);
  CHECK(a.offset == 0 && a.len == 5 && b.offset == 5 && b.len == 3, "offsets %zu %zu", a.offset,
        b.offset);
  CHECK(a.gen == b.gen, "one generation before a flush");
  CHECK(c.pending_words() == 8 && c.has_pending(), "pending words %zu", c.pending_words());
  CHECK(!c.ready(a) && c.view_device_u64(a) == nullptr, "ready before a flush");
  CHECK(throws([&] { c.view_u64(a); }) && throws([&] { c.view(a); }), "view before a flush");
  CHECK(throws([&] { c.enqueue(nullptr, fake[1], 2); }), "null share accepted");
  c.enqueue(nullptr, nullptr, 0);  // an empty request needs no pointers
  DeviceOpenCollector::Limits lim;
  lim.max_pending_words = 10;
  c.set_limits(lim);
  CHECK(throws([&] { c.enqueue(fake[0], fake[1], 3); }), "pending budget not enforced");
  CHECK(c.pending_words() == 8, "a refused enqueue changed the pending words");
  c.clear();
  CHECK(c.empty() && c.pending_words() == 0, "clear left requests");
  OpenHandle d = c.enqueue(fake[0], fake[1], 2);
  CHECK(d.gen != a.gen && d.offset == 0, "clear did not start a new generation");
  c.clear();
  c.flush();  // nothing pending: no GPU call, no generation change
  CHECK(c.stats().flushes == 0, "an empty flush counted");
  CHECK(c.stats().max_pending_words == 8, "max pending %zu", c.stats().max_pending_words);
}

struct Dev {
  void* p = nullptr;
  explicit Dev(size_t bytes) { ok(sufhip_malloc(&p, bytes ? bytes : 8), "malloc"); }
  ~Dev() { sufhip_free(p); }
  uint64_t* u() const { return static_cast<uint64_t*>(p); }
};

static void test_gpu() {
  ok(sufhip_init(0), "init");
  void* stream = nullptr;
  ok(sufhip_stream_create(&stream), "stream");
  std::mt19937_64 rng(2024);
  for (int ring : {64, 50, 13}) {
    DeviceOpenCollector c(ring);
    c.set_cuda_stream(stream);
    const uint64_t mask = ring >= 64 ? ~uint64_t(0) : (uint64_t(1) << ring) - 1;
    uint64_t prev_gen = ~uint64_t(0);
    OpenHandle stale;
    for (int round = 0; round < 3; ++round) {
      // Requests: reserve()d (filled by copies on the stream) and enqueue()d
      // external buffers, mixed, lengths ragged, one empty.
      const std::vector<size_t> lens = {1000, 1, 0, size_t(70000 + round), 33};
      std::vector<std::vector<uint64_t>> xs, s0, s1;
      std::vector<OpenHandle> hs;
      std::vector<Dev*> ext;
      for (size_t i = 0; i < lens.size(); ++i) {
        const size_t n = lens[i];
        std::vector<uint64_t> x(n), a(n), b(n);
        for (size_t j = 0; j < n; ++j) {
          x[j] = rng() & mask;
          b[j] = rng() & mask;
          a[j] = (x[j] - b[j]) & mask;
        }
        const OpenKind kind = i % 2 ? OpenKind::kBeaver : OpenKind::kMask;
        if ((i + round) % 2 == 0) {
          DeviceOpenCollector::Reserve r = c.reserve(n, kind);
          if (n) {
            ok(sufhip_memcpy_h2d(r.diff[0], a.data(), n * 8, stream), "h2d");
            ok(sufhip_memcpy_h2d(r.diff[1], b.data(), n * 8, stream), "h2d");
          }
          hs.push_back(r.handle);
        } else {
          Dev* d0 = new Dev(n * 8);
          Dev* d1 = new Dev(n * 8);
          ext.push_back(d0);
          ext.push_back(d1);
          if (n) {
            ok(sufhip_memcpy_h2d(d0->p, a.data(), n * 8, stream), "h2d");
            ok(sufhip_memcpy_h2d(d1->p, b.data(), n * 8, stream), "h2d");
          }
          hs.push_back(c.enqueue(d0->u(), d1->u(), n, kind));
        }
        xs.push_back(x);
      }
      c.flush();
      CHECK(!c.has_pending() && c.pending_words() == 0, "flush left requests");
      CHECK(hs[0].gen != prev_gen, "generation did not advance");
      if (round > 0) {
        CHECK(!c.ready(stale) && c.view_device_u64(stale) == nullptr,
              "a view of the previous flush is still ready");
        CHECK(throws([&] { c.view_u64(stale); }), "view_u64 of the previous flush");
      }
      for (size_t i = 0; i < hs.size(); ++i) {
        CHECK(c.ready(hs[i]), "request %zu not ready", i);
        ConstView<uint64_t> v = c.view_u64(hs[i]);
        CHECK(v.size() == xs[i].size(), "view length");
        size_t bad = 0;
        for (size_t j = 0; j < v.size(); ++j) bad += v[j] != xs[i][j];
        CHECK(bad == 0, "ring %d round %d request %zu: %zu opened values differ", ring, round, i,
              bad);
        // The device view holds the same values.
        if (!xs[i].empty()) {
          std::vector<uint64_t> back(xs[i].size());
          ok(sufhip_memcpy_d2h(back.data(), c.view_device_u64(hs[i]), back.size() * 8, stream),
             "d2h");
          ok(sufhip_stream_synchronize(stream), "sync");
          CHECK(back == xs[i], "device view differs (request %zu)", i);
        }
        ConstView<int64_t> sv = c.view(hs[i]);
        bool sx_ok = true;
        for (size_t j = 0; j < sv.size(); ++j) {
          const uint64_t x = xs[i][j];
          const bool neg = ring < 64 && ((x >> (ring - 1)) & 1);
          const uint64_t want = neg ? (x | ~mask) : x;
          sx_ok &= uint64_t(sv[j]) == want;
        }
        CHECK(sx_ok, "signed view of request %zu", i);
      }
      stale = hs[0];
      prev_gen = hs[0].gen;
      ok(sufhip_stream_synchronize(stream), "sync");
      for (Dev* d : ext) delete d;
    }
    const DeviceOpenCollector::Stats& st = c.stats();
    size_t words = 0;
    for (int r = 0; r < 3; ++r) words += 1000 + 1 + 70000 + r + 33;
    CHECK(st.flushes == 3 && st.opened_words == words, "stats: %zu flushes, %zu words",
          st.flushes, st.opened_words);
    CHECK(st.opened_words_by_kind[size_t(OpenKind::kMask)] +
                  st.opened_words_by_kind[size_t(OpenKind::kBeaver)] ==
              words,
          "words by kind");
    uint64_t wire = 0;
    for (int r = 0; r < 3; ++r) wire += ((71034 + r) * uint64_t(ring) + 63) / 64 * 8;
    CHECK(st.wire_bytes_sent == wire, "wire bytes %llu, want %llu",
          (unsigned long long)st.wire_bytes_sent, (unsigned long long)wire);
  }
  ok(sufhip_stream_destroy(stream), "stream destroy");
}

int main(int argc, char** argv) {
  const std::string mode = argc > 1 ? argv[1] : "cpu";
  try {
    if (mode == "cpu")
      test_cpu();
    else if (mode == "gpu")
      test_gpu();
    else
      throw std::runtime_error("mode: cpu | gpu");
  } catch (const std::exception& e) {
    std::fprintf(stderr, "exception: %s\n", e.what());
    return 2;
  }
  if (g_fail) {
    std::printf("%d checks failed\n", g_fail);
    return 1;
  }
  std::printf("open collector %s: passed\n", mode.c_str());
  return 0;
}
