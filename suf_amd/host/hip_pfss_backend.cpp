// HipPfssBackend over the C ABI of libsuf_hip.so.  Host code only: no HIP
// headers; device memory, streams and kernels are reached through suf_hip.h.
#include "suf_hip/hip_pfss_backend.hpp"

#include <algorithm>
#include <cctype>
#include <cstdlib>
#include <cstring>
#include <random>
#include <stdexcept>

#include "suf_hip.h"

namespace suf_hip {

struct HipRng {
  bool deterministic = false;
  std::mt19937_64 mt;
  std::random_device rd;
  uint8_t byte() { return static_cast<uint8_t>(deterministic ? (mt() & 0xFF) : (rd() & 0xFF)); }
};

namespace {

void chk(int rc, const char* what) {
  if (rc != SUFHIP_OK)
    throw std::runtime_error(std::string("HipPfssBackend: ") + what + ": " + sufhip_last_error());
}

std::mutex g_prg_mu;
bool g_prg_set = false;
uint8_t g_prg[128];

const uint8_t* prg_ptr() {
  std::lock_guard<std::mutex> lk(g_prg_mu);
  if (!g_prg_set) {
    std::random_device rd;
    for (auto& b : g_prg) b = static_cast<uint8_t>(rd() & 0xFF);
    g_prg_set = true;
  }
  return g_prg;
}

uint64_t bits_to_u64_msb(const std::vector<uint8_t>& bits, int in_bits) {
  if (static_cast<int>(bits.size()) != in_bits)
    throw std::runtime_error("HipPfssBackend: bit vector length != in_bits");
  uint64_t v = 0;
  for (int i = 0; i < in_bits; ++i) v |= uint64_t(bits[size_t(i)] & 1u) << (in_bits - 1 - i);
  return v;
}

uint64_t fnv1a(const uint8_t* p, size_t n) {
  uint64_t h = 1469598103934665603ull;
  for (size_t i = 0; i < n; ++i) {
    h ^= p[i];
    h *= 1099511628211ull;
  }
  return h;
}

// myl7 adapter header (myl7_fss_backend.hpp:159-169).
struct DcfHeader {
  int in_bits, chunks, party, payload_len;
};
DcfHeader dcf_header(const uint8_t* k, size_t key_bytes) {
  if (key_bytes < 8) throw std::runtime_error("HipPfssBackend: DCF key truncated");
  DcfHeader h{k[0], k[1], k[2],
              int(uint32_t(k[4]) | uint32_t(k[5]) << 8 | uint32_t(k[6]) << 16 |
                  uint32_t(k[7]) << 24)};
  if (h.party != 0 && h.party != 1) throw std::runtime_error("HipPfssBackend: bad party flag");
  return h;
}


void check_dcf_keys(int in_bits, size_t key_bytes, const DcfHeader& h) {
  if (h.in_bits != in_bits) throw std::runtime_error("HipPfssBackend: in_bits mismatch");
  if (sufhip_dcf_key_bytes(in_bits, h.payload_len) != key_bytes)
    throw std::runtime_error("HipPfssBackend: key_bytes does not match the DCF key header");
}

}  // namespace

int HipPfssBackend::group_for(int payload_len) const {
  return params_.xor_payloads || payload_len == 1 ? SUFHIP_GROUP_XOR : SUFHIP_GROUP_ADD;
}

void HipPfssBackend::set_prg_state(const uint8_t state[128]) {
  std::lock_guard<std::mutex> lk(g_prg_mu);
  std::memcpy(g_prg, state, 128);
  g_prg_set = true;
}

std::vector<uint8_t> HipPfssBackend::prg_state() {
  const uint8_t* p = prg_ptr();
  return std::vector<uint8_t>(p, p + 128);
}

HipPfssBackend::HipPfssBackend() : HipPfssBackend(Params{}) {}

HipPfssBackend::HipPfssBackend(Params p) : params_(p), rng_(new HipRng) {
  chk(sufhip_init(p.device), "init");
  chk(sufhip_stream_create(&stream_), "stream");
  if (p.seed) {
    rng_->deterministic = true;
    rng_->mt.seed(p.seed);
  }
}

HipPfssBackend::~HipPfssBackend() {
  if (stream_) sufhip_stream_synchronize(stream_);
  for (Buf* b : {&keys_, &xs_, &out_, &bools_, &scratch_}) sufhip_free(b->ptr);
  for (auto& kv : staged_) sufhip_free(kv.second.dev);
  sufhip_stream_destroy(stream_);
}

void HipPfssBackend::ensure(Buf& b, size_t bytes) const {
  if (bytes <= b.cap) return;
  sync();
  chk(sufhip_free(b.ptr), "free");
  b.ptr = nullptr;
  b.cap = 0;
  const size_t cap = std::max<size_t>(bytes, 256);
  chk(sufhip_malloc(&b.ptr, cap), "malloc");
  b.cap = cap;
}

void HipPfssBackend::sync() const { chk(sufhip_stream_synchronize(stream_), "sync"); }

std::vector<uint8_t> HipPfssBackend::random_bytes(size_t n) {
  std::vector<uint8_t> v(n);
  for (auto& b : v) b = rng_->byte();
  return v;
}

const uint8_t* HipPfssBackend::stage_keys(const uint8_t* host, size_t bytes) const {
  if (!host) throw std::runtime_error("HipPfssBackend: keys_flat is null");
  ensure(keys_, bytes);
  chk(sufhip_memcpy_h2d(keys_.ptr, host, bytes, stream_), "H2D keys");
  return static_cast<const uint8_t*>(keys_.ptr);
}

const uint8_t* HipPfssBackend::stage_broadcast_key(const uint8_t* host, size_t bytes) const {
  if (!host || bytes == 0) throw std::runtime_error("HipPfssBackend: broadcast key is empty");
  const uint64_t h = fnv1a(host, bytes) ^ bytes;
  auto it = staged_.find(h);
  if (it != staged_.end() && it->second.host.size() == bytes &&
      std::memcmp(it->second.host.data(), host, bytes) == 0)
    return static_cast<const uint8_t*>(it->second.dev);
  if (it != staged_.end()) {
    sync();
    sufhip_free(it->second.dev);
    staged_.erase(it);
  }
  if (staged_.size() >= 4096) {  // bound the cache
    sync();
    for (auto& kv : staged_) sufhip_free(kv.second.dev);
    staged_.clear();
  }
  Staged s;
  s.host.assign(host, host + bytes);
  chk(sufhip_malloc(&s.dev, bytes), "malloc key");
  chk(sufhip_memcpy_h2d(s.dev, s.host.data(), bytes, stream_), "H2D key");
  sync();  // s.host moves into the map; the copy must have read it
  const uint8_t* d = static_cast<const uint8_t*>(s.dev);
  staged_.emplace(h, std::move(s));
  return d;
}

const uint64_t* HipPfssBackend::stage_xs(const std::vector<uint64_t>& xs) const {
  ensure(xs_, xs.size() * 8);
  chk(sufhip_memcpy_h2d(xs_.ptr, xs.data(), xs.size() * 8, stream_), "H2D xs");
  return static_cast<const uint64_t*>(xs_.ptr);
}

std::vector<uint8_t> HipPfssBackend::u64_to_bits_msb(uint64_t x, int in_bits) const {
  std::vector<uint8_t> bits(static_cast<size_t>(in_bits));
  for (int i = 0; i < in_bits; ++i) bits[size_t(i)] = uint8_t((x >> (in_bits - 1 - i)) & 1u);
  return bits;
}

proto::DcfKeyPair HipPfssBackend::gen_dcf(int in_bits, const std::vector<uint8_t>& alpha_bits,
                                          const std::vector<uint8_t>& payload_bytes) {
  std::lock_guard<std::mutex> lk(mu_);
  if (in_bits <= 0 || in_bits > 64) throw std::runtime_error("HipPfssBackend: in_bits out of range");
  const uint64_t alpha = bits_to_u64_msb(alpha_bits, in_bits);
  const int plen = int(payload_bytes.size());
  const size_t kb = sufhip_dcf_key_bytes(in_bits, plen);
  if (kb == 0) throw std::runtime_error("HipPfssBackend: bad payload length");
  const int chunks = (plen + 15) / 16;
  std::vector<uint8_t> seeds = random_bytes(size_t(chunks) * 32);
  // scratch: [alpha 8][payload plen][seeds][key0][key1]
  const size_t off_pay = 8, off_seed = (off_pay + size_t(plen) + 15) & ~size_t(15);
  const size_t off_k0 = (off_seed + seeds.size() + 15) & ~size_t(15);
  const size_t off_k1 = (off_k0 + kb + 15) & ~size_t(15);
  ensure(scratch_, off_k1 + kb);
  uint8_t* s = static_cast<uint8_t*>(scratch_.ptr);
  chk(sufhip_memcpy_h2d(s, &alpha, 8, stream_), "H2D alpha");
  chk(sufhip_memcpy_h2d(s + off_pay, payload_bytes.data(), size_t(plen), stream_), "H2D payload");
  chk(sufhip_memcpy_h2d(s + off_seed, seeds.data(), seeds.size(), stream_), "H2D seeds");
  chk(sufhip_dcf_gen(group_for(plen), in_bits, prg_ptr(), reinterpret_cast<uint64_t*>(s),
                     s + off_pay, plen, 1, s + off_seed, 1, s + off_k0, s + off_k1, stream_),
      "dcf_gen");
  proto::DcfKeyPair kp;
  kp.k0.bytes.resize(kb);
  kp.k1.bytes.resize(kb);
  chk(sufhip_memcpy_d2h(kp.k0.bytes.data(), s + off_k0, kb, stream_), "D2H key0");
  chk(sufhip_memcpy_d2h(kp.k1.bytes.data(), s + off_k1, kb, stream_), "D2H key1");
  sync();
  return kp;
}

void HipPfssBackend::dcf_eval_dev(int in_bits, size_t key_bytes, const uint8_t* d_keys, int bcast,
                                  int payload_len, const uint64_t* d_xs, size_t n, int out_bytes,
                                  uint8_t* outs_host) const {
  const int group = group_for(payload_len);
  const bool bit = group == SUFHIP_GROUP_XOR && out_bytes == 1;
  if (!bit && (out_bytes < 1 || out_bytes > payload_len))
    throw std::runtime_error("HipPfssBackend: out_bytes must be in [1, payload_len]");
  ensure(bools_, n * size_t(out_bytes));
  chk(sufhip_dcf_eval(group, in_bits, payload_len, prg_ptr(), d_keys, key_bytes, bcast, d_xs, n,
                      bit ? SUFHIP_DCF_OUT_BIT : SUFHIP_DCF_OUT_BYTES, out_bytes, bools_.ptr,
                      stream_),
      "dcf_eval");
  if (outs_host)
    chk(sufhip_memcpy_d2h(outs_host, bools_.ptr, n * size_t(out_bytes), stream_), "D2H outs");
  sync();
}

std::vector<uint8_t> HipPfssBackend::eval_dcf(int in_bits, const proto::FssKey& kb,
                                              const std::vector<uint8_t>& x_bits) const {
  std::lock_guard<std::mutex> lk(mu_);
  const DcfHeader h = dcf_header(kb.bytes.data(), kb.bytes.size());
  check_dcf_keys(in_bits, kb.bytes.size(), h);
  const std::vector<uint64_t> xs{bits_to_u64_msb(x_bits, in_bits)};
  const uint8_t* dk = stage_keys(kb.bytes.data(), kb.bytes.size());
  std::vector<uint8_t> out(size_t(h.payload_len));
  // Full payload share (Myl7FssBackend::eval_dcf): the bytes mode for every group.
  ensure(bools_, out.size());
  chk(sufhip_dcf_eval(group_for(h.payload_len), in_bits, h.payload_len, prg_ptr(), dk,
                      kb.bytes.size(), 0, stage_xs(xs), 1, SUFHIP_DCF_OUT_BYTES, h.payload_len,
                      bools_.ptr, stream_),
      "dcf_eval");
  chk(sufhip_memcpy_d2h(out.data(), bools_.ptr, out.size(), stream_), "D2H");
  sync();
  return out;
}

void HipPfssBackend::eval_dcf_many_u64(int in_bits, size_t key_bytes, const uint8_t* keys_flat,
                                       const std::vector<uint64_t>& xs_u64, int out_bytes,
                                       uint8_t* outs_flat) const {
  std::lock_guard<std::mutex> lk(mu_);
  if (xs_u64.empty()) return;
  const DcfHeader h = dcf_header(keys_flat, key_bytes);
  check_dcf_keys(in_bits, key_bytes, h);
  const uint8_t* dk = stage_keys(keys_flat, key_bytes * xs_u64.size());
  dcf_eval_dev(in_bits, key_bytes, dk, 0, h.payload_len, stage_xs(xs_u64), xs_u64.size(),
               out_bytes, outs_flat);
}

void HipPfssBackend::eval_dcf_many_u64_device(int in_bits, size_t key_bytes,
                                              const uint8_t* keys_flat, const uint64_t* xs_device,
                                              size_t N, int out_bytes, uint8_t* outs_flat) const {
  std::lock_guard<std::mutex> lk(mu_);
  if (N == 0) return;
  if (!xs_device) throw std::runtime_error("eval_dcf_many_u64_device: xs_device is null");
  const DcfHeader h = dcf_header(keys_flat, key_bytes);
  check_dcf_keys(in_bits, key_bytes, h);
  dcf_eval_dev(in_bits, key_bytes, stage_keys(keys_flat, key_bytes * N), 0, h.payload_len,
               xs_device, N, out_bytes, outs_flat);
}

void HipPfssBackend::eval_dcf_many_u64_device_broadcast(int in_bits, size_t key_bytes,
                                                        const uint8_t* key,
                                                        const uint64_t* xs_device, size_t N,
                                                        int out_bytes, uint8_t* outs_flat) const {
  std::lock_guard<std::mutex> lk(mu_);
  if (N == 0) return;
  if (!xs_device) throw std::runtime_error("eval_dcf_many_u64_device_broadcast: xs_device is null");
  const DcfHeader h = dcf_header(key, key_bytes);
  check_dcf_keys(in_bits, key_bytes, h);
  dcf_eval_dev(in_bits, key_bytes, stage_broadcast_key(key, key_bytes), 1, h.payload_len,
               xs_device, N, out_bytes, outs_flat);
}

proto::IntervalLutKeyPair HipPfssBackend::gen_interval_lut(const proto::IntervalLutDesc& desc) {
  std::lock_guard<std::mutex> lk(mu_);
  if (desc.out_words <= 0) throw std::runtime_error("HipPfssBackend: out_words must be >0");
  if (desc.cutpoints.size() < 2) throw std::runtime_error("HipPfssBackend: need >=2 cutpoints");
  const int intervals = int(desc.cutpoints.size()) - 1;
  if (desc.payload_flat.size() != size_t(intervals) * size_t(desc.out_words))
    throw std::runtime_error("HipPfssBackend: payload size mismatch");
  const uint64_t nonce = next_id_++;
  uint8_t seed[16];
  sufhip_seed_from_id(nonce, 7, seed);
  const size_t kb = sufhip_interval_lut_key_bytes(intervals, desc.out_words);
  proto::IntervalLutKeyPair kp;
  kp.k0.bytes.resize(kb);
  kp.k1.bytes.resize(kb);
  chk(sufhip_interval_lut_build_key(0, nonce, desc.in_bits, desc.out_words, desc.cutpoints.data(),
                                    intervals, desc.payload_flat.data(), seed, kp.k0.bytes.data()),
      "lut key");
  chk(sufhip_interval_lut_build_key(1, nonce, desc.in_bits, desc.out_words, desc.cutpoints.data(),
                                    intervals, desc.payload_flat.data(), seed, kp.k1.bytes.data()),
      "lut key");
  return kp;
}

namespace {
int lut_intervals(const uint8_t* k, size_t key_bytes, int out_words) {
  if (key_bytes < 216) throw std::runtime_error("HipPfssBackend: LUT key truncated");
  uint16_t ow;
  uint32_t iv;
  std::memcpy(&ow, k + 2, 2);
  std::memcpy(&iv, k + 4, 4);
  if (int(ow) != out_words) throw std::runtime_error("HipPfssBackend: out_words mismatch");
  if (sufhip_interval_lut_key_bytes(int(iv), out_words) != key_bytes)
    throw std::runtime_error("HipPfssBackend: LUT key_bytes mismatch");
  return int(iv);
}
int packed_thresholds(const uint8_t* k, size_t key_bytes, int out_words) {
  if (key_bytes < 208) throw std::runtime_error("HipPfssBackend: packed key truncated");
  uint16_t nt;
  std::memcpy(&nt, k + 2, 2);
  if ((int(nt) + 63) / 64 != out_words)
    throw std::runtime_error("HipPfssBackend: out_words != ceil(num_thr / 64)");
  if (sufhip_packed_lt_key_bytes(int(nt)) != key_bytes)
    throw std::runtime_error("HipPfssBackend: packed key_bytes mismatch");
  return int(nt);
}
}  // namespace

void HipPfssBackend::eval_interval_lut_many_u64(size_t key_bytes, const uint8_t* keys_flat,
                                                const std::vector<uint64_t>& xs_u64, int out_words,
                                                uint64_t* outs_flat) const {
  if (xs_u64.empty()) return;
  std::lock_guard<std::mutex> lk(mu_);
  const int iv = lut_intervals(keys_flat, key_bytes, out_words);
  const size_t n = xs_u64.size();
  const uint8_t* dk = stage_keys(keys_flat, key_bytes * n);
  const uint64_t* dx = stage_xs(xs_u64);
  ensure(out_, n * size_t(out_words) * 8);
  chk(sufhip_interval_lut_eval(dk, key_bytes, 0, iv, out_words, dx, n,
                               static_cast<uint64_t*>(out_.ptr), stream_),
      "lut eval");
  chk(sufhip_memcpy_d2h(outs_flat, out_.ptr, n * size_t(out_words) * 8, stream_), "D2H");
  sync();
}

void HipPfssBackend::eval_interval_lut_many_device(size_t key_bytes, const uint8_t* keys_flat,
                                                   const uint64_t* xs_device, size_t N,
                                                   int out_words, uint64_t* outs_flat) const {
  if (N == 0) return;
  std::lock_guard<std::mutex> lk(mu_);
  const int iv = lut_intervals(keys_flat, key_bytes, out_words);
  const uint8_t* dk = stage_keys(keys_flat, key_bytes * N);
  ensure(out_, N * size_t(out_words) * 8);
  chk(sufhip_interval_lut_eval(dk, key_bytes, 0, iv, out_words, xs_device, N,
                               static_cast<uint64_t*>(out_.ptr), stream_),
      "lut eval");
  if (outs_flat)
    chk(sufhip_memcpy_d2h(outs_flat, out_.ptr, N * size_t(out_words) * 8, stream_), "D2H");
  sync();
}

void HipPfssBackend::eval_interval_lut_many_device_broadcast(size_t key_bytes, const uint8_t* key,
                                                             const uint64_t* xs_device, size_t N,
                                                             int out_words,
                                                             uint64_t* outs_flat) const {
  if (N == 0) return;
  std::lock_guard<std::mutex> lk(mu_);
  const int iv = lut_intervals(key, key_bytes, out_words);
  const uint8_t* dk = stage_broadcast_key(key, key_bytes);
  ensure(out_, N * size_t(out_words) * 8);
  chk(sufhip_interval_lut_eval(dk, key_bytes, 1, iv, out_words, xs_device, N,
                               static_cast<uint64_t*>(out_.ptr), stream_),
      "lut eval");
  if (outs_flat)
    chk(sufhip_memcpy_d2h(outs_flat, out_.ptr, N * size_t(out_words) * 8, stream_), "D2H");
  sync();
}

proto::PackedLtKeyPair HipPfssBackend::gen_packed_lt(int in_bits,
                                                     const std::vector<uint64_t>& thresholds) {
  std::lock_guard<std::mutex> lk(mu_);
  if (thresholds.empty()) throw std::runtime_error("HipPfssBackend: packed thresholds empty");
  const uint64_t nonce = next_id_++;
  uint8_t seed[16];
  sufhip_seed_from_id(nonce, 0, seed);
  const size_t kb = sufhip_packed_lt_key_bytes(int(thresholds.size()));
  proto::PackedLtKeyPair kp;
  kp.k0.bytes.resize(kb);
  kp.k1.bytes.resize(kb);
  for (int p = 0; p < 2; ++p)
    chk(sufhip_packed_lt_build_key(p, nonce, in_bits, thresholds.data(), int(thresholds.size()),
                                   seed, (p ? kp.k1 : kp.k0).bytes.data()),
        "packed key");
  return kp;
}

void HipPfssBackend::eval_packed_lt_many(size_t key_bytes, const uint8_t* keys_flat,
                                         const std::vector<uint64_t>& xs_u64, int in_bits,
                                         int out_words, uint64_t* outs_bitmask) const {
  (void)in_bits;  // the key header carries the bit width
  if (xs_u64.empty()) return;
  std::lock_guard<std::mutex> lk(mu_);
  const int nt = packed_thresholds(keys_flat, key_bytes, out_words);
  const size_t n = xs_u64.size();
  const uint8_t* dk = stage_keys(keys_flat, key_bytes * n);
  const uint64_t* dx = stage_xs(xs_u64);
  ensure(bools_, n * size_t(out_words) * 8);
  chk(sufhip_packed_lt_eval(dk, key_bytes, 0, nt, out_words, dx, n,
                            static_cast<uint64_t*>(bools_.ptr), stream_),
      "packed eval");
  chk(sufhip_memcpy_d2h(outs_bitmask, bools_.ptr, n * size_t(out_words) * 8, stream_), "D2H");
  sync();
}

void HipPfssBackend::eval_packed_lt_many_device(size_t key_bytes, const uint8_t* keys_flat,
                                                const uint64_t* xs_device, size_t N, int in_bits,
                                                int out_words, uint64_t* outs_bitmask) const {
  (void)in_bits;
  if (N == 0) return;
  std::lock_guard<std::mutex> lk(mu_);
  const int nt = packed_thresholds(keys_flat, key_bytes, out_words);
  const uint8_t* dk = stage_keys(keys_flat, key_bytes * N);
  ensure(bools_, N * size_t(out_words) * 8);
  chk(sufhip_packed_lt_eval(dk, key_bytes, 0, nt, out_words, xs_device, N,
                            static_cast<uint64_t*>(bools_.ptr), stream_),
      "packed eval");
  if (outs_bitmask)
    chk(sufhip_memcpy_d2h(outs_bitmask, bools_.ptr, N * size_t(out_words) * 8, stream_), "D2H");
  sync();
}

void HipPfssBackend::eval_packed_lt_many_device_broadcast(size_t key_bytes, const uint8_t* key,
                                                          const uint64_t* xs_device, size_t N,
                                                          int in_bits, int out_words,
                                                          uint64_t* outs_bitmask) const {
  (void)in_bits;
  if (N == 0) return;
  std::lock_guard<std::mutex> lk(mu_);
  const int nt = packed_thresholds(key, key_bytes, out_words);
  const uint8_t* dk = stage_broadcast_key(key, key_bytes);
  ensure(bools_, N * size_t(out_words) * 8);
  chk(sufhip_packed_lt_eval(dk, key_bytes, 1, nt, out_words, xs_device, N,
                            static_cast<uint64_t*>(bools_.ptr), stream_),
      "packed eval");
  if (outs_bitmask)
    chk(sufhip_memcpy_d2h(outs_bitmask, bools_.ptr, N * size_t(out_words) * 8, stream_), "D2H");
  sync();
}

const uint64_t* HipPfssBackend::last_device_output() const {
  return static_cast<const uint64_t*>(out_.ptr);
}
const uint64_t* HipPfssBackend::last_device_bools() const {
  return static_cast<const uint64_t*>(bools_.ptr);
}
void HipPfssBackend::ensure_output_buffers(size_t arith_words, size_t bool_words) const {
  std::lock_guard<std::mutex> lk(mu_);
  if (arith_words) ensure(out_, arith_words * 8);
  if (bool_words) ensure(bools_, bool_words * 8);
}

std::unique_ptr<proto::PfssBackendBatch> make_hip_backend_from_env() {
  const char* env = std::getenv("SUF_PFSS_BACKEND");
  if (!env) return nullptr;
  std::string v(env);
  std::transform(v.begin(), v.end(), v.begin(),
                 [](unsigned char c) { return static_cast<char>(std::tolower(c)); });
  if (v != "hip") return nullptr;
  return std::make_unique<HipPfssBackend>();
}

}  // namespace suf_hip
