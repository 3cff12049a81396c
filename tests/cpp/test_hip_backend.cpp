// Two-party test of HipPfssBackend through the SUF proto interfaces, in the
// style of the reference's in-process tests (src/demo/test_pfss_gpu.cpp,
// test_cuda_packed_pfss.cpp): a dealer instance generates keys, one instance
// per party evaluates on its own thread, and the shares must reconstruct the
// closed forms (1[x < alpha], the LUT row, the threshold bitmask).
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <random>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "suf_hip.h"
#include "suf_hip/cuda_primitives.hpp"
#include "suf_hip/hip_pfss_backend.hpp"

using suf_hip::HipPfssBackend;

static int g_fail = 0;
#define CHECK(cond, ...)                   \
  do {                                     \
    if (!(cond)) {                         \
      std::fprintf(stderr, __VA_ARGS__);   \
      std::fprintf(stderr, "\n");          \
      ++g_fail;                            \
      return;                              \
    }                                      \
  } while (0)

// Runs f(party, backend) for both parties concurrently.
static void two_parties(const std::function<void(int, HipPfssBackend&)>& f) {
  HipPfssBackend b0, b1;
  std::thread t0([&] { f(0, b0); });
  std::thread t1([&] { f(1, b1); });
  t0.join();
  t1.join();
}

static std::vector<uint8_t> flatten(const proto::FssKey& k, size_t n) {
  std::vector<uint8_t> v(k.bytes.size() * n);
  for (size_t i = 0; i < n; ++i) std::memcpy(v.data() + i * k.bytes.size(), k.bytes.data(), k.bytes.size());
  return v;
}

static void test_dcf(int in_bits, size_t payload_len) {
  HipPfssBackend::Params dp;
  dp.seed = 99 + payload_len;
  HipPfssBackend dealer(dp);
  std::mt19937_64 rng(in_bits * 131 + payload_len);
  const uint64_t mask = in_bits == 64 ? ~0ull : ((1ull << in_bits) - 1);
  const size_t nkeys = 40, per = 5, n = nkeys * per;
  std::vector<uint8_t> payload(payload_len, 0);
  payload[0] = 1;  // XorBytes {1} or pack_u64_le(1) (AddU64)
  std::vector<proto::DcfKeyPair> keys;
  std::vector<uint64_t> alphas, xs;
  for (size_t k = 0; k < nkeys; ++k) {
    uint64_t a = rng() & mask;
    alphas.push_back(a);
    keys.push_back(dealer.gen_dcf(in_bits, dealer.u64_to_bits_msb(a, in_bits), payload));
    for (size_t d = 0; d < per; ++d) xs.push_back((a + d - 2) & mask);
  }
  const size_t kb = keys[0].k0.bytes.size();
  const int ob = payload_len == 1 ? 1 : 8;
  std::vector<uint8_t> outs[2], single[2];
  two_parties([&](int p, HipPfssBackend& be) {
    std::vector<uint8_t> flat(kb * n);
    for (size_t i = 0; i < n; ++i) {
      const auto& k = p ? keys[i / per].k1 : keys[i / per].k0;
      std::memcpy(flat.data() + i * kb, k.bytes.data(), kb);
    }
    outs[p].assign(n * ob, 0);
    be.eval_dcf_many_u64(in_bits, kb, flat.data(), xs, ob, outs[p].data());
    const auto& k0 = p ? keys[0].k1 : keys[0].k0;
    single[p] = be.eval_dcf(in_bits, k0, be.u64_to_bits_msb(xs[0], in_bits));
  });
  for (size_t i = 0; i < n; ++i) {
    const uint64_t lt = xs[i] < alphas[i / per];
    uint64_t rec;
    if (payload_len == 1) {
      rec = (outs[0][i] ^ outs[1][i]) & 1;
    } else {
      uint64_t a, b;
      std::memcpy(&a, &outs[0][i * 8], 8);
      std::memcpy(&b, &outs[1][i * 8], 8);
      rec = a + b;
    }
    CHECK(rec == lt, "dcf in_bits=%d plen=%zu i=%zu rec=%llu exp=%llu", in_bits, payload_len, i,
          (unsigned long long)rec, (unsigned long long)lt);
  }
  CHECK(single[0].size() == payload_len, "eval_dcf returns payload_len bytes");
}

static void test_dcf_device_broadcast() {
  HipPfssBackend dealer;
  const uint64_t alpha = 0x8000000000001234ull;
  auto kp = dealer.gen_dcf(64, dealer.u64_to_bits_msb(alpha, 64), std::vector<uint8_t>{1});
  const size_t n = 10000;
  std::vector<uint64_t> xs(n);
  std::mt19937_64 rng(5);
  for (auto& x : xs) x = rng();
  xs[0] = alpha - 1;
  xs[1] = alpha;
  std::vector<uint8_t> outs[2];
  two_parties([&](int p, HipPfssBackend& be) {
    void* d = nullptr;
    if (sufhip_malloc(&d, n * 8) || sufhip_memcpy_h2d(d, xs.data(), n * 8, nullptr) ||
        sufhip_stream_synchronize(nullptr))
      throw std::runtime_error("staging xs");
    const auto& k = p ? kp.k1 : kp.k0;
    outs[p].assign(n, 0);
    be.eval_dcf_many_u64_device_broadcast(64, k.bytes.size(), k.bytes.data(),
                                          static_cast<const uint64_t*>(d), n, 1, outs[p].data());
    // device-only call keeps the result in last_device_bools()
    be.eval_dcf_many_u64_device_broadcast(64, k.bytes.size(), k.bytes.data(),
                                          static_cast<const uint64_t*>(d), n, 1, nullptr);
    std::vector<uint8_t> dev(n);
    if (sufhip_memcpy_d2h(dev.data(), be.last_device_bools(), n, nullptr) ||
        sufhip_stream_synchronize(nullptr))
      throw std::runtime_error("reading last_device_bools");
    if (dev != outs[p]) throw std::runtime_error("last_device_bools differs from host output");
    sufhip_free(d);
  });
  for (size_t i = 0; i < n; ++i)
    CHECK(uint64_t((outs[0][i] ^ outs[1][i]) & 1) == uint64_t(xs[i] < alpha), "bcast dcf i=%zu", i);
}

static void test_lut() {
  HipPfssBackend dealer;
  proto::IntervalLutDesc desc;
  desc.in_bits = 6;
  desc.out_words = 2;
  desc.cutpoints = {0, 20, 40, 64};
  desc.payload_flat = {100, 200, 300, 400, 500, 600};
  auto kp = dealer.gen_interval_lut(desc);
  std::vector<uint64_t> xs = {0, 25, 50, 19, 20, 63};
  std::vector<uint64_t> outs[2], bouts[2];
  two_parties([&](int p, HipPfssBackend& be) {
    const auto& k = p ? kp.k1 : kp.k0;
    auto flat = flatten(k, xs.size());
    outs[p].assign(xs.size() * 2, 0);
    be.eval_interval_lut_many_u64(k.bytes.size(), flat.data(), xs, 2, outs[p].data());
    void* d = nullptr;
    if (sufhip_malloc(&d, xs.size() * 8) ||
        sufhip_memcpy_h2d(d, xs.data(), xs.size() * 8, nullptr) ||
        sufhip_stream_synchronize(nullptr))
      throw std::runtime_error("staging xs");
    bouts[p].assign(xs.size() * 2, 0);
    be.eval_interval_lut_many_device_broadcast(k.bytes.size(), k.bytes.data(),
                                               static_cast<const uint64_t*>(d), xs.size(), 2,
                                               bouts[p].data());
    sufhip_free(d);
  });
  for (size_t i = 0; i < xs.size(); ++i) {
    const size_t iv = xs[i] < 20 ? 0 : (xs[i] < 40 ? 1 : 2);
    for (int w = 0; w < 2; ++w) {
      CHECK(outs[0][i * 2 + w] + outs[1][i * 2 + w] == desc.payload_flat[iv * 2 + w], "lut i=%zu", i);
      CHECK(bouts[0][i * 2 + w] + bouts[1][i * 2 + w] == desc.payload_flat[iv * 2 + w],
            "lut bcast i=%zu", i);
    }
  }
}

static void test_packed() {
  HipPfssBackend dealer;
  std::vector<uint64_t> thr = {5, 12, 33, 48, 60};
  auto kp = dealer.gen_packed_lt(6, thr);
  std::vector<uint64_t> xs = {0, 15, 63, 33, 4};
  std::vector<uint64_t> outs[2];
  two_parties([&](int p, HipPfssBackend& be) {
    const auto& k = p ? kp.k1 : kp.k0;
    auto flat = flatten(k, xs.size());
    outs[p].assign(xs.size(), 0);
    be.eval_packed_lt_many(k.bytes.size(), flat.data(), xs, 6, 1, outs[p].data());
  });
  for (size_t i = 0; i < xs.size(); ++i) {
    uint64_t exp = 0;
    for (size_t j = 0; j < thr.size(); ++j) exp |= uint64_t(xs[i] < thr[j]) << j;
    CHECK((outs[0][i] ^ outs[1][i]) == exp, "packed i=%zu", i);
  }
}

static void test_errors() {
  HipPfssBackend be;
  bool threw = false;
  try {
    be.gen_dcf(65, std::vector<uint8_t>(65, 0), std::vector<uint8_t>{1});
  } catch (const std::runtime_error&) {
    threw = true;
  }
  CHECK(threw, "gen_dcf(in_bits=65) must throw");
  threw = false;
  try {
    std::vector<uint8_t> junk(100, 0);
    be.eval_dcf_many_u64(64, junk.size(), junk.data(), std::vector<uint64_t>{1}, 1, junk.data());
  } catch (const std::runtime_error&) {
    threw = true;
  }
  CHECK(threw, "eval on a malformed key must throw");
}

// SUF's launchers by their reference names (include/suf_hip/cuda_primitives.hpp
// over the C ABI): a Beaver product and ragged row sums reconstruct their
// closed forms, and a launch the C ABI rejects throws.
static void test_launcher_shim() {
  const size_t n = 1000;
  std::mt19937_64 rng(5);
  std::vector<uint64_t> x(n), y(n), a0(n), a1(n), b0(n), b1(n), c0(n), c1(n), d(n), e(n);
  for (size_t i = 0; i < n; ++i) {
    x[i] = rng(), y[i] = rng();
    const uint64_t a = rng(), b = rng();
    a0[i] = rng(), b0[i] = rng(), c0[i] = rng();
    a1[i] = a - a0[i], b1[i] = b - b0[i], c1[i] = a * b - c0[i];
    d[i] = x[i] - a, e[i] = y[i] - b;
  }
  auto up = [](const std::vector<uint64_t>& v) {
    void* p = nullptr;
    if (sufhip_malloc(&p, v.size() * 8) || sufhip_memcpy_h2d(p, v.data(), v.size() * 8, nullptr))
      throw std::runtime_error("upload failed");
    return static_cast<uint64_t*>(p);
  };
  uint64_t *dx = up(x), *dy = up(y), *dd = up(d), *de = up(e);
  uint64_t* da[2] = {up(a0), up(a1)};
  uint64_t* db[2] = {up(b0), up(b1)};
  uint64_t* dc[2] = {up(c0), up(c1)};
  uint64_t* dz[2] = {up(x), up(x)};
  for (int p = 0; p < 2; ++p)
    launch_beaver_mul_kernel(p, dx, dy, da[p], db[p], dc[p], dd, de, dz[p], n, nullptr);
  std::vector<uint64_t> z0(n), z1(n);
  sufhip_memcpy_d2h(z0.data(), dz[0], n * 8, nullptr);
  sufhip_memcpy_d2h(z1.data(), dz[1], n * 8, nullptr);
  sufhip_stream_synchronize(nullptr);
  for (size_t i = 0; i < n; ++i) CHECK(z0[i] + z1[i] == x[i] * y[i], "launcher Beaver product at %zu", i);
  // Ragged rows of lengths 1..40 packed back to back.
  std::vector<int> offs{0};
  for (int r = 1; r <= 40; ++r) offs.push_back(offs.back() + r);
  std::vector<uint64_t> vals(offs.back());
  for (auto& v : vals) v = rng();
  void* doffs = nullptr;
  sufhip_malloc(&doffs, offs.size() * sizeof(int));
  sufhip_memcpy_h2d(doffs, offs.data(), offs.size() * sizeof(int), nullptr);
  uint64_t* dvals = up(vals);
  uint64_t* dsum = up(std::vector<uint64_t>(40));
  launch_row_sum_ragged_kernel(dvals, static_cast<const int*>(doffs), 40, dsum, nullptr);
  std::vector<uint64_t> sums(40);
  sufhip_memcpy_d2h(sums.data(), dsum, 40 * 8, nullptr);
  sufhip_stream_synchronize(nullptr);
  for (int r = 0; r < 40; ++r) {
    uint64_t want = 0;
    for (int j = offs[r]; j < offs[r + 1]; ++j) want += vals[j];
    CHECK(sums[r] == want, "launcher ragged row sum %d", r);
  }
  bool threw = false;
  try {
    launch_pack_eff_bits_kernel(dx, 65, dz[0], n, nullptr);  // eff_bits out of range
  } catch (const std::runtime_error&) {
    threw = true;
  }
  CHECK(threw, "a launch the C ABI rejects must throw");
  for (void* p : {static_cast<void*>(dx), static_cast<void*>(dy), static_cast<void*>(dd),
                  static_cast<void*>(de), static_cast<void*>(da[0]), static_cast<void*>(da[1]),
                  static_cast<void*>(db[0]), static_cast<void*>(db[1]), static_cast<void*>(dc[0]),
                  static_cast<void*>(dc[1]), static_cast<void*>(dz[0]), static_cast<void*>(dz[1]),
                  doffs, static_cast<void*>(dvals), static_cast<void*>(dsum)})
    sufhip_free(p);
}

static void test_factory() {
  setenv("SUF_PFSS_BACKEND", "HIP", 1);
  auto be = suf_hip::make_hip_backend_from_env();
  CHECK(be != nullptr, "SUF_PFSS_BACKEND=hip must select the HIP backend");
  CHECK(dynamic_cast<proto::PfssGpuStagedEval*>(be.get()) != nullptr, "staged-eval capability");
  CHECK(dynamic_cast<proto::PackedLtBackend*>(be.get()) != nullptr, "packed capability");
  setenv("SUF_PFSS_BACKEND", "cpu", 1);
  CHECK(suf_hip::make_hip_backend_from_env() == nullptr, "other kinds are not ours");
}

static std::vector<uint8_t> unhex(const std::string& h) {
  std::vector<uint8_t> v(h.size() / 2);
  for (size_t i = 0; i < v.size(); ++i) v[i] = uint8_t(std::stoul(h.substr(2 * i, 2), nullptr, 16));
  return v;
}

// Keys the reference's own myl7 adapter made (XOR group, tests/golden/
// dcf_myl7.json, written out as text by the pytest wrapper), evaluated by an
// instance with xor_payloads: every payload share byte-equal to the
// reference's through eval_dcf, and through eval_dcf_many_u64 (share byte
// 0 & 1 on a 1-byte key, as the reference's batch), for 1-, 8- and 16-byte
// payloads.  The default instance gives the additive group for the
// multi-byte keys, so its shares differ there.
//   prg <hex 128 bytes>
//   case <in_bits> <payload_len> <key0 hex> <key1 hex> <n>
//   x <u64> <out0 hex> <out1 hex>     (n lines)
static int run_golden(const char* path) {
  std::FILE* f = std::fopen(path, "r");
  if (!f) {
    std::fprintf(stderr, "cannot open %s\n", path);
    return 2;
  }
  char tok[16];
  char buf[8192], b2[8192], b3[8192];
  if (std::fscanf(f, "%15s %8191s", tok, buf) != 2 || std::string(tok) != "prg") return 2;
  const std::vector<uint8_t> prg = unhex(buf);
  HipPfssBackend::set_prg_state(prg.data());
  HipPfssBackend::Params xp;
  xp.xor_payloads = true;
  HipPfssBackend bx(xp), bdef;
  int cases = 0, multi = 0, differ = 0;
  int in_bits, plen, n;
  while (std::fscanf(f, "%15s %d %d %8191s %8191s %d", tok, &in_bits, &plen, buf, b2, &n) == 6) {
    proto::FssKey k[2];
    k[0].bytes = unhex(buf);
    k[1].bytes = unhex(b2);
    std::vector<uint64_t> xs;
    std::vector<std::vector<uint8_t>> want[2];
    for (int i = 0; i < n; ++i) {
      unsigned long long x;
      if (std::fscanf(f, "%15s %llu %8191s %8191s", tok, &x, b2, b3) != 4) return 2;
      xs.push_back(x);
      want[0].push_back(unhex(b2));
      want[1].push_back(unhex(b3));
    }
    for (int p = 0; p < 2; ++p) {
      std::vector<uint8_t> many(size_t(n) * plen);
      bx.eval_dcf_many_u64(in_bits, k[p].bytes.size(), flatten(k[p], size_t(n)).data(), xs, plen,
                           many.data());
      for (int i = 0; i < n; ++i) {
        const std::vector<uint8_t> one = bx.eval_dcf(in_bits, k[p], bx.u64_to_bits_msb(xs[i], in_bits));
        // The batch keeps share byte 0 & 1 on a 1-byte key (the reference's
        // eval_dcf_many_u64), the payload share otherwise.
        std::vector<uint8_t> want_many = want[p][i];
        if (plen == 1) want_many[0] &= 1;
        if (one != want[p][i] || std::memcmp(many.data() + size_t(i) * plen, want_many.data(), plen)) {
          std::fprintf(stderr, "golden case %d (in_bits %d, payload %d) party %d x %d differs\n",
                       cases, in_bits, plen, p, i);
          ++g_fail;
        }
        if (plen > 1) {
          const std::vector<uint8_t> d = bdef.eval_dcf(in_bits, k[p], bdef.u64_to_bits_msb(xs[i], in_bits));
          differ += d != want[p][i];
        }
      }
    }
    ++cases;
    multi += plen > 1;
  }
  std::fclose(f);
  if (cases == 0 || multi == 0) {
    std::fprintf(stderr, "golden fixture has %d cases, %d with multi-byte payloads\n", cases, multi);
    return 1;
  }
  if (differ == 0) {
    std::fprintf(stderr, "the additive default gave the XOR shares on every multi-byte key\n");
    ++g_fail;
  }
  if (g_fail) return 1;
  std::printf("golden xor keys: %d cases (%d multi-byte) passed\n", cases, multi);
  return 0;
}

int main(int argc, char** argv) {
  if (argc > 2 && std::string(argv[1]) == "golden") {
    try {
      return run_golden(argv[2]);
    } catch (const std::exception& e) {
      std::fprintf(stderr, "exception: %s\n", e.what());
      return 2;
    }
  }
  uint8_t state[128];
  std::mt19937_64 g(3);
  for (auto& b : state) b = uint8_t(g() & 0xFF);
  HipPfssBackend::set_prg_state(state);
  try {
    test_dcf(64, 1);
    test_dcf(64, 8);
    test_dcf(12, 8);
    test_dcf(16, 1);
    test_dcf_device_broadcast();
    test_lut();
    test_packed();
    test_errors();
    test_launcher_shim();
    test_factory();
  } catch (const std::exception& e) {
    std::fprintf(stderr, "exception: %s\n", e.what());
    return 2;
  }
  if (g_fail) {
    std::fprintf(stderr, "%d check(s) failed\n", g_fail);
    return 1;
  }
  std::printf("hip backend two-party test passed\n");
  return 0;
}
