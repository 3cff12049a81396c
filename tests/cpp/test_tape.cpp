// Tape records, composite party-key tapes and key arrays streamed from a tape
// into device memory (include/suf_hip/tape.hpp).
//   test_tape cpu <tests/golden/tape_records.bin>
//     the records written here are byte-equal to the reference TapeWriter's
//     tape, which reads back to the same values; tag and length checks;
//     composite-tape round trips and every truncation refused; key-array
//     sections parse back.
//   test_tape gpu <scratch dir>
//     DCF keys made on the GPU and a truncation gate's keys go to a tape file
//     in blocks; DeviceKeyArray streams them back into device buffers (small
//     staging buffers, several refills) byte-equal to the originals; the
//     tape-loaded DCF keys reconstruct 1[x < alpha] and the tape-loaded
//     truncation keys give the shares of the original keys.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "suf_hip.h"
#include "suf_hip/tape.hpp"

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

static std::vector<uint8_t> read_file(const std::string& path) {
  std::FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) throw std::runtime_error("cannot open " + path);
  std::vector<uint8_t> b;
  uint8_t buf[4096];
  size_t n;
  while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0) b.insert(b.end(), buf, buf + n);
  std::fclose(f);
  return b;
}

static void test_records(const std::string& golden) {
  BufferSink sink;
  TapeWriter w(sink);
  w.write_u64(0x0123456789abcdefull);
  const uint64_t v[4] = {1, 2, 3, ~uint64_t(0)};
  w.write_u64_vec(v, 4);
  const uint8_t hello[5] = {'h', 'e', 'l', 'l', 'o'};
  w.write_bytes(hello, 5);
  w.write_bytes(nullptr, 0);
  const Triple64 t1{1, 2, 3};
  w.write_triples(&t1, 1);
  const Triple64 t2[2] = {{4, 5, 6}, {7, 8, 9}};
  w.write_triples(t2, 2);
  w.write_u64(0);
  const std::vector<uint8_t> ref = read_file(golden);
  CHECK(sink.bytes == ref, "records differ from the reference TapeWriter's (%zu vs %zu bytes)",
        sink.bytes.size(), ref.size());
  FileSource src(golden);
  TapeReader r(src);
  CHECK(r.read_u64() == 0x0123456789abcdefull, "u64");
  CHECK(r.read_u64_vec() == std::vector<uint64_t>(v, v + 4), "u64 vec");
  CHECK(r.read_bytes() == std::vector<uint8_t>(hello, hello + 5), "bytes");
  CHECK(r.read_bytes().empty(), "empty bytes");
  auto a = r.read_triples();
  CHECK(a.size() == 1 && a[0].a == 1 && a[0].b == 2 && a[0].c == 3, "triple");
  auto b = r.read_triples();
  CHECK(b.size() == 2 && b[1].a == 7 && b[1].c == 9, "triples");
  CHECK(r.read_u64() == 0 && r.eof(), "tail");
  // Tag and size checks, and reads past the end.
  BufferSource s1(ref.data(), ref.size());
  TapeReader r1(s1);
  CHECK(throws([&] { r1.read_bytes(); }), "a u64 record read as bytes must throw");
  BufferSource s2(ref.data(), 12);
  TapeReader r2(s2);
  CHECK(throws([&] { r2.read_u64(); }), "a truncated record must throw");
}

static CompositeTapeKey random_key(std::mt19937_64& g) {
  CompositeTapeKey k;
  k.r_in_share = g();
  for (int i = 0; i < 3; ++i) k.r_in_share_vec.push_back(g());
  k.r_out_share = {g(), g()};
  for (int i = 0; i < 5; ++i) k.wrap_share.push_back(g());
  k.r_hi_share = g();
  k.wrap_sign_share = g();
  k.extra_params = {g()};
  k.pred_meta = {1, 2, 8};
  k.cut_pred_meta = {0, 1, 1};
  k.coeff_bit_order = 1;
  k.coeff_sem = 2;
  for (int i = 0; i < 3; ++i) {
    std::vector<uint8_t> blob(100 + 37 * i);
    for (auto& x : blob) x = uint8_t(g());
    k.pred_keys.push_back(blob);
  }
  k.cut_pred_keys.push_back(std::vector<uint8_t>(5, 7));
  k.base_coeff_share = {g(), g(), g(), g()};
  k.total_delta_share = {g(), g(), g(), g()};
  for (int i = 0; i < 7; ++i) k.triples.push_back({g(), g(), g()});
  for (int i = 0; i < 9; ++i) k.bit_triples.push_back({uint8_t(g() & 1), uint8_t(g() & 1), uint8_t(g() & 1)});
  return k;
}

static void test_composite_tape() {
  std::mt19937_64 g(11);
  const CompositeTapeKey k = random_key(g);
  const std::vector<uint8_t> t = write_composite_tape(k);
  // Field order and sizes of gates::write_composite_tape: 8 + (4 + 24) +
  // (4 + 16) + (4 + 40) + 8 + 8 + (4 + 8) + 6 + 6 + 2, then the key lists,
  // coefficient shares, triples and bit triples.
  size_t want = 8 + 28 + 20 + 44 + 16 + 12 + 14;
  want += 4 + (4 + 100) + (4 + 137) + (4 + 174) + 4 + (4 + 5) + 4;
  want += (4 + 32) + (4 + 32) + (4 + 7 * 24) + (4 + 9 * 3);
  CHECK(t.size() == want, "composite tape size %zu, want %zu", t.size(), want);
  CHECK(t[0] == uint8_t(k.r_in_share) && t[8] == 3 && t[12] == uint8_t(k.r_in_share_vec[0]),
        "composite tape head");
  const CompositeTapeKey b = read_composite_tape(t.data(), t.size());
  CHECK(write_composite_tape(b) == t, "composite tape round trip");
  CHECK(b.pred_keys == k.pred_keys && b.wrap_share == k.wrap_share && b.triples.size() == 7 &&
            b.bit_triples[8].c == k.bit_triples[8].c && b.pred_meta.out_bytes == 8,
        "composite tape fields");
  int refused = 0;
  for (size_t len = 0; len < t.size(); ++len)
    refused += throws([&] { read_composite_tape(t.data(), len); }) ? 1 : 0;
  CHECK(size_t(refused) == t.size(), "every truncation must be refused (%d of %zu)", refused,
        t.size());
}

static void test_key_array_cpu() {
  std::vector<uint8_t> keys(10 * 13);
  for (size_t i = 0; i < keys.size(); ++i) keys[i] = uint8_t(i * 7);
  BufferSink sink;
  TapeWriter w(sink);
  write_key_array(w, keys.data(), 10, 13, 4);
  BufferSource src(sink.bytes.data(), sink.bytes.size());
  TapeReader r(src);
  CHECK(r.read_u64() == 10 && r.read_u64() == 13, "key array header");
  std::vector<uint8_t> back;
  while (!r.eof()) {
    auto blk = r.read_bytes();
    CHECK(blk.size() % 13 == 0 && blk.size() <= 4 * 13, "key block size");
    back.insert(back.end(), blk.begin(), blk.end());
  }
  CHECK(back == keys, "key array round trip");
}

static void ok(int rc, const char* what) {
  if (rc != SUFHIP_OK) throw std::runtime_error(std::string(what) + ": " + sufhip_last_error());
}

static std::vector<uint8_t> d2h(const void* d, size_t n) {
  std::vector<uint8_t> h(n);
  ok(sufhip_memcpy_d2h(h.data(), d, n, nullptr), "d2h");
  ok(sufhip_stream_synchronize(nullptr), "sync");
  return h;
}

static void* h2d(const void* h, size_t n) {
  void* d = nullptr;
  ok(sufhip_malloc(&d, n), "malloc");
  ok(sufhip_memcpy_h2d(d, h, n, nullptr), "h2d");
  return d;
}

static void test_gpu(const std::string& dir) {
  ok(sufhip_init(0), "init");
  uint8_t state[128];
  std::mt19937_64 g(3);
  for (auto& b : state) b = uint8_t(g() & 0xff);
  // DCF keys for 5000 points, written to a tape file in blocks of 777 keys.
  const size_t n = 5000;
  const size_t kb = sufhip_dcf_key_bytes(64, 1);
  std::vector<uint64_t> alpha(n), xs(n);
  std::vector<uint8_t> seeds(n * 32);
  for (size_t i = 0; i < n; ++i) {
    alpha[i] = g();
    xs[i] = alpha[i] + (g() % 5) - 2;
  }
  for (auto& s : seeds) s = uint8_t(g());
  const uint8_t one = 1;
  void *da = h2d(alpha.data(), n * 8), *dsd = h2d(seeds.data(), seeds.size()), *dp = h2d(&one, 1);
  void *dk0 = nullptr, *dk1 = nullptr;
  ok(sufhip_malloc(&dk0, n * kb), "malloc");
  ok(sufhip_malloc(&dk1, n * kb), "malloc");
  ok(sufhip_dcf_gen(SUFHIP_GROUP_XOR, 64, state, static_cast<uint64_t*>(da),
                    static_cast<uint8_t*>(dp), 1, 1, static_cast<uint8_t*>(dsd), n,
                    static_cast<uint8_t*>(dk0), static_cast<uint8_t*>(dk1), nullptr),
     "dcf_gen");
  const std::vector<uint8_t> k0 = d2h(dk0, n * kb), k1 = d2h(dk1, n * kb);
  // A truncation gate's two keys as single-key arrays on the same tape.
  const int f = 12;
  const size_t tkb = sufhip_trunc_key_bytes(SUFHIP_TRUNC_GAPARS, f);
  std::vector<uint64_t> rnd(SUFHIP_TRUNC_RAND_WORDS);
  for (auto& w : rnd) w = g();
  void *dt0 = nullptr, *dt1 = nullptr;
  ok(sufhip_malloc(&dt0, tkb), "malloc");
  ok(sufhip_malloc(&dt1, tkb), "malloc");
  ok(sufhip_trunc_gen(SUFHIP_TRUNC_GAPARS, f, state, rnd.data(), static_cast<uint8_t*>(dt0),
                      static_cast<uint8_t*>(dt1), nullptr),
     "trunc_gen");
  const std::vector<uint8_t> t0 = d2h(dt0, tkb), t1 = d2h(dt1, tkb);
  const std::string path = dir + "/keys.tape";
  {
    FileSink sink(path);
    TapeWriter w(sink);
    write_key_array(w, k0.data(), n, kb, 777);
    write_key_array(w, k1.data(), n, kb, 777);
    write_key_array(w, t0.data(), 1, tkb, 1);
    write_key_array(w, t1.data(), 1, tkb, 1);
    w.flush();
  }
  FileSource src(path);
  TapeReader r(src);
  void* stream = nullptr;
  ok(sufhip_stream_create(&stream), "stream");
  DeviceKeyArray a0(r, stream, 3 * kb + 5);  // staging holds 3 keys: many refills
  DeviceKeyArray a1(r, stream, 64 << 10);
  DeviceKeyArray ta0(r, stream), ta1(r, stream);
  CHECK(a0.size() == n && a0.key_bytes() == kb && r.eof(), "key array headers");
  CHECK(d2h(a0.data(), n * kb) == k0 && d2h(a1.data(), n * kb) == k1, "DCF keys from the tape");
  CHECK(d2h(ta0.data(), tkb) == t0 && d2h(ta1.data(), tkb) == t1, "truncation keys from the tape");
  // Evaluate the tape-loaded keys.
  void* dx = h2d(xs.data(), n * 8);
  void *o0 = nullptr, *o1 = nullptr;
  ok(sufhip_malloc(&o0, n), "malloc");
  ok(sufhip_malloc(&o1, n), "malloc");
  ok(sufhip_dcf_eval(SUFHIP_GROUP_XOR, 64, 1, state, a0.data(), kb, 0, static_cast<uint64_t*>(dx),
                     n, SUFHIP_DCF_OUT_BIT, 1, o0, stream),
     "dcf_eval");
  ok(sufhip_dcf_eval(SUFHIP_GROUP_XOR, 64, 1, state, a1.data(), kb, 0, static_cast<uint64_t*>(dx),
                     n, SUFHIP_DCF_OUT_BIT, 1, o1, stream),
     "dcf_eval");
  ok(sufhip_stream_synchronize(stream), "sync");
  const std::vector<uint8_t> b0 = d2h(o0, n), b1 = d2h(o1, n);
  size_t bad = 0;
  for (size_t i = 0; i < n; ++i) bad += ((b0[i] ^ b1[i]) & 1) != (xs[i] < alpha[i] ? 1 : 0);
  CHECK(bad == 0, "tape-loaded DCF keys: %zu wrong reconstructions", bad);
  std::vector<uint64_t> xh(n);
  for (size_t i = 0; i < n; ++i) xh[i] = (g() % 100000) + rnd[0] - 50000;
  void* dxh = h2d(xh.data(), n * 8);
  void *y[4] = {nullptr, nullptr, nullptr, nullptr};
  for (auto& p : y) ok(sufhip_malloc(&p, n * 8), "malloc");
  const void* tk[4] = {ta0.data(), ta1.data(), dt0, dt1};
  for (int q = 0; q < 4; ++q)
    ok(sufhip_trunc_eval_noalloc(SUFHIP_TRUNC_GAPARS, f, state, static_cast<const uint8_t*>(tk[q]),
                                 tkb, static_cast<uint64_t*>(dxh), n, static_cast<uint64_t*>(y[q]),
                                 stream),
       "trunc_eval");
  ok(sufhip_stream_synchronize(stream), "sync");
  CHECK(d2h(y[0], n * 8) == d2h(y[2], n * 8) && d2h(y[1], n * 8) == d2h(y[3], n * 8),
        "tape-loaded truncation keys give the original keys' shares");
  for (void* p : {da, dsd, dp, dk0, dk1, dt0, dt1, dx, o0, o1, dxh, y[0], y[1], y[2], y[3]})
    sufhip_free(p);
  sufhip_stream_destroy(stream);
  std::remove(path.c_str());
}

static void write_file(const std::string& path, const std::vector<uint8_t>& v) {
  std::FILE* f = std::fopen(path.c_str(), "wb");
  if (!f || std::fwrite(v.data(), 1, v.size(), f) != v.size())
    throw std::runtime_error("cannot write " + path);
  std::fclose(f);
}

int main(int argc, char** argv) {
  // composite-rw <in> <out>: the C++ reader and writer over a composite tape
  // written elsewhere (the Python host side); composite-write <out>: a tape
  // of the random key above, for the Python reader.
  if (argc == 4 && std::string(argv[1]) == "composite-rw") {
    try {
      const std::vector<uint8_t> t = read_file(argv[2]);
      write_file(argv[3], write_composite_tape(read_composite_tape(t.data(), t.size())));
    } catch (const std::exception& e) {
      std::fprintf(stderr, "exception: %s\n", e.what());
      return 2;
    }
    return 0;
  }
  if (argc == 3 && std::string(argv[1]) == "composite-write") {
    std::mt19937_64 g(11);
    try {
      write_file(argv[2], write_composite_tape(random_key(g)));
    } catch (const std::exception& e) {
      std::fprintf(stderr, "exception: %s\n", e.what());
      return 2;
    }
    return 0;
  }
  if (argc < 3) {
    std::fprintf(stderr, "usage: test_tape cpu <golden tape> | gpu <scratch dir>\n");
    return 2;
  }
  try {
    if (std::string(argv[1]) == "cpu") {
      test_records(argv[2]);
      test_composite_tape();
      test_key_array_cpu();
    } else {
      test_gpu(argv[2]);
    }
  } catch (const std::exception& e) {
    std::fprintf(stderr, "exception: %s\n", e.what());
    return 2;
  }
  if (g_fail) {
    std::fprintf(stderr, "%d check(s) failed\n", g_fail);
    return 1;
  }
  std::printf("tape test (%s) passed\n", argv[1]);
  return 0;
}
