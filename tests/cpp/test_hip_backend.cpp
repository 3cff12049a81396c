// Two-party test of HipPfssBackend through the SUF proto interfaces, in the
// style of the reference's in-process tests (src/demo/test_pfss_gpu.cpp,
// test_cuda_packed_pfss.cpp): a dealer instance generates keys, one instance
// per party evaluates on its own thread, and the shares must reconstruct the
// closed forms (1[x < alpha], the LUT row, the threshold bitmask).
#include <algorithm>
#include <chrono>
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

// SUF's truncation through the unchanged per-party interfaces, as a SUF
// build with SUF_PFSS_BACKEND=hip runs it:
//   * dealer: composite_gen_trunc_gate's predicate queries
//     (include/gates/composite_fss.hpp:645-833) keyed by gen_dcf with
//     pack_u64_le(1) payloads (the AddU64 predicate semantics): carry =
//     NOT(a XOR b XOR w) over the f-bit queries 1[x^_low < r_low] and
//     1[x^_low < 0] (suf::rewrite_ltlow of build_trunc_pred_suf's threshold
//     2^f - r_low, include/suf/trunc_suf_builders.hpp:16-75,
//     include/suf/mask_rewrite.hpp:28-34), sign = a XOR b XOR w over the
//     64-bit queries 1[x^ < r + 2^63] and 1[x^ < r] (rewrite_msb_add), wrap
//     = 1[x^ < r] (src/compiler/suf_to_pfss.cpp:447-455; one query with the
//     sign's second); wrap bits, r_hi, m and the zero r_out split
//     additively;
//   * route A, the reference's own (composite_fss.hpp:1385-1638 and
//     include/runtime/phase_tasks.hpp:869-902): each query through
//     eval_dcf_many_u64_device_broadcast(..., out_bytes = 8, host outputs),
//     the bool plan on the host (one - v, b - a + w), the arithmetic and
//     bool words copied into ensure_output_buffers' device buffers and
//     launch_trunc_postproc_kernel on last_device_output() /
//     last_device_bools();
//   * route B, device-kept (GapARS: the one bool port is the carry, and
//     query a's additive share is a share of it, since b = 1[x^_low < 0] is 0
//     and w = 1): eval_dcf_many_u64_device_broadcast(..., 8, nullptr), then
//     launch_trunc_postproc_kernel straight on last_device_bools().
// Both parties reconstruct x >> f (TR: logical; ARS and GapARS:
// arithmetic, |x| < 2^62).
namespace {
enum { kTR = 0, kARS = 1, kGapARS = 2 };
constexpr uint64_t kTop = uint64_t(1) << 63;

struct TruncQuery {
  int bits;
  uint64_t theta;
  proto::FssKey key[2];
};
// Bool plan of one port (composite_fss.hpp:1416-1483's restricted forms).
struct TruncPort {
  enum Kind { kConst0, kNotRot, kRot, kVar } kind;
  int a = -1, b = -1, w = -1;  // query indexes; w: wrap-share index
};
struct TruncDeal {
  int kind, f;
  uint64_t r;
  std::vector<TruncQuery> q;
  std::vector<TruncPort> ports;
  int carry_idx = -1, sign_idx = -1, wrap_idx = -1;
  std::vector<uint64_t> wrap_share[2];
  uint64_t r_hi_share[2], m_share[2], rout_share[2];
};

std::vector<uint8_t> pack_one() {
  std::vector<uint8_t> v(8, 0);
  v[0] = 1;
  return v;
}

// rlow0: clear r's low f bits (the carry port is then the constant 0).
TruncDeal deal_trunc(HipPfssBackend& dealer, std::mt19937_64& rng, int kind, int f, bool rlow0) {
  TruncDeal d;
  d.kind = kind;
  d.f = f;
  const uint64_t mask = (uint64_t(1) << f) - 1;
  d.r = rng();
  if (rlow0) d.r &= ~mask;
  const uint64_t r_low = d.r & mask;
  auto split = [&](uint64_t v, uint64_t* s) {
    s[0] = rng();
    s[1] = v - s[0];
  };
  auto query = [&](int bits, uint64_t theta) {
    for (size_t i = 0; i < d.q.size(); ++i)
      if (d.q[i].bits == bits && d.q[i].theta == theta) return int(i);  // add_query's dedup
    TruncQuery t;
    t.bits = bits;
    t.theta = theta;
    auto kp = dealer.gen_dcf(bits, dealer.u64_to_bits_msb(theta, bits), pack_one());
    t.key[0] = kp.k0;
    t.key[1] = kp.k1;
    d.q.push_back(t);
    return int(d.q.size()) - 1;
  };
  auto wrap_bit = [&](uint64_t w) {
    uint64_t s[2];
    split(w, s);
    d.wrap_share[0].push_back(s[0]);
    d.wrap_share[1].push_back(s[1]);
    return int(d.wrap_share[0].size()) - 1;
  };
  // carry
  d.carry_idx = int(d.ports.size());
  if (r_low == 0) {
    d.ports.push_back({TruncPort::kConst0});
  } else {
    const uint64_t th0 = r_low, th1 = (r_low + ((uint64_t(1) << f) - r_low)) & mask;
    TruncPort p{TruncPort::kNotRot};
    p.a = query(f, th0);
    p.b = query(f, th1);
    p.w = wrap_bit(th1 < th0 ? 1 : 0);
    d.ports.push_back(p);
  }
  if (kind == kARS) {
    const uint64_t th0 = d.r + kTop, th1 = th0 + kTop;
    d.sign_idx = int(d.ports.size());
    TruncPort p{TruncPort::kRot};
    p.a = query(64, th0);
    p.b = query(64, th1);
    p.w = wrap_bit(th1 < th0 ? 1 : 0);
    d.ports.push_back(p);
  }
  if (kind != kGapARS) {
    d.wrap_idx = int(d.ports.size());
    TruncPort p{TruncPort::kVar};
    p.a = query(64, d.r);
    d.ports.push_back(p);
  }
  split(d.r >> f, d.r_hi_share);
  split(kind == kGapARS && (d.r >> 63) ? uint64_t(1) << (64 - f) : 0, d.m_share);
  split(0, d.rout_share);
  return d;
}

uint64_t* upload_u64(const std::vector<uint64_t>& v) {
  void* p = nullptr;
  if (sufhip_malloc(&p, v.size() * 8) || sufhip_memcpy_h2d(p, v.data(), v.size() * 8, nullptr) ||
      sufhip_stream_synchronize(nullptr))
    throw std::runtime_error("upload failed");
  return static_cast<uint64_t*>(p);
}

// Route A for one party: the reference's AddU64 branch and TruncTask's
// postproc launch, unchanged.  Writes n output words to d_out.
void trunc_route_a(HipPfssBackend& be, const TruncDeal& d, int p, const uint64_t* d_xhat,
                   size_t n, uint64_t* d_out) {
  const size_t ell = d.ports.size();
  std::vector<uint64_t> pred(d.q.size() * n);
  for (size_t qi = 0; qi < d.q.size(); ++qi) {
    const proto::FssKey& k = d.q[qi].key[p];
    be.eval_dcf_many_u64_device_broadcast(d.q[qi].bits, k.bytes.size(), k.bytes.data(), d_xhat,
                                          n, 8, reinterpret_cast<uint8_t*>(pred.data() + qi * n));
  }
  const uint64_t one = p == 0 ? 1 : 0;
  std::vector<uint64_t> bools(n * ell), haty(n, 0 + d.rout_share[p]);
  for (size_t i = 0; i < n; ++i)
    for (size_t j = 0; j < ell; ++j) {
      const TruncPort& t = d.ports[j];
      uint64_t v = 0;
      if (t.kind == TruncPort::kVar) {
        v = pred[size_t(t.a) * n + i];
      } else if (t.kind != TruncPort::kConst0) {
        v = pred[size_t(t.b) * n + i] - pred[size_t(t.a) * n + i] + d.wrap_share[p][size_t(t.w)];
        if (t.kind == TruncPort::kNotRot) v = one - v;
      }
      bools[i * ell + j] = v;
    }
  be.ensure_output_buffers(n, n * ell);
  void* s = be.device_stream();
  if (sufhip_memcpy_h2d(const_cast<uint64_t*>(be.last_device_output()), haty.data(), n * 8, s) ||
      sufhip_memcpy_h2d(const_cast<uint64_t*>(be.last_device_bools()), bools.data(),
                        n * ell * 8, s))
    throw std::runtime_error("route A: H2D of the gate outputs");
  launch_trunc_postproc_kernel(p, d.kind == kGapARS, d.f, d.r_hi_share[p], d.m_share[p], d_xhat,
                               be.last_device_output(), 1, 0, be.last_device_bools(), ell,
                               d.carry_idx, d.sign_idx, d.wrap_idx, d_out, n, s);
  if (sufhip_stream_synchronize(s)) throw std::runtime_error("route A: sync");
}

// Route B for one party (GapARS): the carry query's share stays on the
// device and feeds the postproc directly; d_arith1 holds base + r_out.
void trunc_route_b(HipPfssBackend& be, const TruncDeal& d, int p, const uint64_t* d_xhat,
                   size_t n, const uint64_t* d_arith1, uint64_t* d_out) {
  void* s = be.device_stream();
  const TruncPort& c = d.ports[size_t(d.carry_idx)];
  if (c.kind == TruncPort::kConst0) {
    launch_trunc_postproc_kernel(p, 1, d.f, d.r_hi_share[p], d.m_share[p], d_xhat, d_arith1, 0,
                                 0, nullptr, 0, -1, -1, -1, d_out, n, s);
  } else {
    const proto::FssKey& k = d.q[size_t(c.a)].key[p];
    be.eval_dcf_many_u64_device_broadcast(d.f, k.bytes.size(), k.bytes.data(), d_xhat, n, 8,
                                          nullptr);
    launch_trunc_postproc_kernel(p, 1, d.f, d.r_hi_share[p], d.m_share[p], d_xhat, d_arith1, 0,
                                 0, be.last_device_bools(), 1, 0, -1, -1, d_out, n, s);
  }
  if (sufhip_stream_synchronize(s)) throw std::runtime_error("route B: sync");
}

std::vector<uint64_t> trunc_inputs(std::mt19937_64& rng, size_t n, int f) {
  std::vector<uint64_t> x(n);
  const uint64_t lim = uint64_t(1) << 40;
  for (auto& v : x) v = (rng() % (2 * lim)) - lim;
  const uint64_t edge[] = {0, ~uint64_t(0), (uint64_t(1) << f) - 1, uint64_t(1) << f,
                           uint64_t(0) - (uint64_t(1) << f), lim - 1, uint64_t(0) - lim};
  for (size_t i = 0; i < sizeof(edge) / 8 && i < n; ++i) x[i] = edge[i];
  return x;
}

uint64_t trunc_want(int kind, int f, uint64_t x) {
  return kind == kTR ? x >> f : uint64_t(int64_t(x) >> f);
}
}  // namespace

static void test_trunc_addu64_route(int kind, int f, size_t n, uint64_t seed, bool rlow0) {
  HipPfssBackend::Params dp;
  dp.seed = seed;
  HipPfssBackend dealer(dp);
  std::mt19937_64 rng(seed);
  const TruncDeal d = deal_trunc(dealer, rng, kind, f, rlow0);
  const std::vector<uint64_t> x = trunc_inputs(rng, n, f);
  std::vector<uint64_t> xhat(n);
  for (size_t i = 0; i < n; ++i) xhat[i] = x[i] + d.r;
  std::vector<uint64_t> ya[2], yb[2];
  two_parties([&](int p, HipPfssBackend& be) {
    uint64_t* dx = upload_u64(xhat);
    void* dout = nullptr;
    if (sufhip_malloc(&dout, n * 8)) throw std::runtime_error("malloc out");
    trunc_route_a(be, d, p, dx, n, static_cast<uint64_t*>(dout));
    ya[p].resize(n);
    if (sufhip_memcpy_d2h(ya[p].data(), dout, n * 8, nullptr) || sufhip_stream_synchronize(nullptr))
      throw std::runtime_error("D2H route A");
    if (kind == kGapARS) {
      uint64_t* da = upload_u64(std::vector<uint64_t>{d.rout_share[p]});
      trunc_route_b(be, d, p, dx, n, da, static_cast<uint64_t*>(dout));
      yb[p].resize(n);
      if (sufhip_memcpy_d2h(yb[p].data(), dout, n * 8, nullptr) ||
          sufhip_stream_synchronize(nullptr))
        throw std::runtime_error("D2H route B");
      sufhip_free(da);
    }
    sufhip_free(dout);
    sufhip_free(dx);
  });
  for (size_t i = 0; i < n; ++i) {
    const uint64_t want = trunc_want(kind, f, x[i]);
    CHECK(ya[0][i] + ya[1][i] == want, "AddU64 route A kind=%d f=%d i=%zu x=%llx got=%llx want=%llx",
          kind, f, i, (unsigned long long)x[i], (unsigned long long)(ya[0][i] + ya[1][i]),
          (unsigned long long)want);
    if (kind == kGapARS)
      CHECK(yb[0][i] + yb[1][i] == want, "AddU64 route B f=%d i=%zu", f, i);
  }
  std::printf("AddU64 truncation route kind=%d f=%d n=%zu: %zu queries, %zu bool ports, r_low=%llu ok\n",
              kind, f, n, d.q.size(), d.ports.size(),
              (unsigned long long)(d.r & ((uint64_t(1) << f) - 1)));
}

// Times one two-party GapARS evaluation (f = 12) at n points, parties one
// after the other on one thread, median of `reps`: route A, route B, and the
// fused truncation gate of the C ABI (sufhip_trunc_eval with its own key
// format).  Prints one line per n.
static void time_trunc_routes(size_t n, int reps) {
  const int f = 12;
  HipPfssBackend::Params dp;
  dp.seed = 7;
  HipPfssBackend dealer(dp), be;
  std::mt19937_64 rng(7);
  const TruncDeal d = deal_trunc(dealer, rng, kGapARS, f, false);
  const std::vector<uint64_t> x = trunc_inputs(rng, n, f);
  std::vector<uint64_t> xhat(n);
  for (size_t i = 0; i < n; ++i) xhat[i] = x[i] + d.r;
  uint64_t* dx = upload_u64(xhat);
  uint64_t* da[2] = {upload_u64({d.rout_share[0]}), upload_u64({d.rout_share[1]})};
  void* dout = nullptr;
  if (sufhip_malloc(&dout, n * 8)) throw std::runtime_error("malloc out");
  uint64_t* out = static_cast<uint64_t*>(dout);
  // The fused gate: its own keys (same r), prepare + finish per party.
  std::vector<uint64_t> rnd(SUFHIP_TRUNC_RAND_WORDS);
  for (auto& w : rnd) w = rng();
  rnd[0] = d.r;
  const size_t kb = sufhip_trunc_key_bytes(kGapARS, f), wb = sufhip_trunc_work_bytes(f, n);
  void *dk0 = nullptr, *dk1 = nullptr, *dw = nullptr;
  const std::vector<uint8_t> prg = HipPfssBackend::prg_state();
  if (sufhip_malloc(&dk0, kb) || sufhip_malloc(&dk1, kb) || sufhip_malloc(&dw, wb ? wb : 16) ||
      sufhip_trunc_gen(kGapARS, f, prg.data(), rnd.data(), static_cast<uint8_t*>(dk0),
                       static_cast<uint8_t*>(dk1), nullptr) ||
      sufhip_stream_synchronize(nullptr))
    throw std::runtime_error("fused gate keys");
  void* dks[2] = {dk0, dk1};
  auto fused = [&] {
    for (int p = 0; p < 2; ++p)
      if (sufhip_trunc_eval(kGapARS, f, prg.data(), static_cast<const uint8_t*>(dks[p]), kb, dx,
                            n, out, dw, wb, nullptr))
        throw std::runtime_error(sufhip_last_error());
    sufhip_stream_synchronize(nullptr);
  };
  auto median_ms = [&](const std::function<void()>& fn) {
    fn();
    std::vector<double> t;
    for (int r = 0; r < reps; ++r) {
      const auto t0 = std::chrono::steady_clock::now();
      fn();
      t.push_back(std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0)
                      .count());
    }
    std::sort(t.begin(), t.end());
    return t[t.size() / 2];
  };
  const double ta = median_ms([&] {
    for (int p = 0; p < 2; ++p) trunc_route_a(be, d, p, dx, n, out);
  });
  const double tb = median_ms([&] {
    for (int p = 0; p < 2; ++p) trunc_route_b(be, d, p, dx, n, da[p], out);
  });
  const double tf = median_ms(fused);
  std::printf("trunc routes GapARS f=%d n=%zu (both parties, ms, median of %d): "
              "route_A_host_plan=%.4f route_B_device_kept=%.4f fused_gate=%.4f\n",
              f, n, reps, ta, tb, tf);
  for (void* p : {static_cast<void*>(dx), static_cast<void*>(da[0]), static_cast<void*>(da[1]),
                  dout, dk0, dk1, dw})
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
  if (argc > 1 && std::string(argv[1]) == "time-trunc") {
    uint8_t state[128];
    std::mt19937_64 g(3);
    for (auto& b : state) b = uint8_t(g() & 0xFF);
    HipPfssBackend::set_prg_state(state);
    try {
      for (size_t n : {size_t(1) << 16, size_t(1) << 20}) time_trunc_routes(n, 10);
    } catch (const std::exception& e) {
      std::fprintf(stderr, "exception: %s\n", e.what());
      return 2;
    }
    return 0;
  }
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
    for (int kind : {kTR, kARS, kGapARS}) {
      test_trunc_addu64_route(kind, 12, size_t(1) << 16, 40 + kind, false);
      test_trunc_addu64_route(kind, 7, 3000, 50 + kind, false);
      test_trunc_addu64_route(kind, 12, 777, 60 + kind, true);
    }
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
