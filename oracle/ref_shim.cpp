// Test-only shim: exposes the reference's own myl7 DCF code (compiled from
// the reference tree by oracle/build_ref.sh into oracle/_ref/) through a flat
// C ABI so the tests can pin the oracle against it.  Nothing here restates
// an algorithm; every call forwards to the reference implementation:
//   dcf_gen / dcf_eval      third_party/myl7_fss/src/dcf.c:42-193
//   prg_init                third_party/myl7_fss/src/prg/aes128_mmo.c:16-31
//   proto::Myl7FssBackend   include/proto/myl7_fss_backend.hpp:23-271
#include <cstdint>
#include <cstring>
#include <mutex>
#include <vector>

#include "proto/myl7_fss_backend.hpp"

extern "C" {
#include <fss/dcf.h>
#include <fss/prg.h>
}

namespace {
std::once_flag g_warm;
// The adapter seeds the PRG from std::random_device on its first gen_dcf
// (myl7_fss_backend.hpp:117-127).  Run that once before installing a fixed
// PRG state so later adapter calls cannot replace it.
void warm_adapter() {
  std::call_once(g_warm, [] {
    proto::Myl7FssBackend be;
    auto bits = be.u64_to_bits_msb(1, 8);
    (void)be.gen_dcf(8, bits, std::vector<uint8_t>{1});
  });
}
}  // namespace

extern "C" {

void ref_prg_init(const uint8_t* state, int len) {
  prg_init(state, len);  // the warm-up below evaluates the PRG
  warm_adapter();
  prg_init(state, len);
}

void ref_dcf_gen(int bitlen, const uint8_t* alpha_le, const uint8_t* beta, const uint8_t* s0,
                 const uint8_t* s1, uint8_t* cws, uint8_t* cw_np1) {
  std::vector<uint8_t> sbuf(10 * kLambda, 0), a(alpha_le, alpha_le + (bitlen + 7) / 8),
      b(beta, beta + kLambda);
  std::memcpy(sbuf.data(), s0, kLambda);
  std::memcpy(sbuf.data() + kLambda, s1, kLambda);
  Key k{cws, cw_np1};
  CmpFunc cf;
  cf.point.alpha = Bits{a.data(), bitlen};
  cf.point.beta = b.data();
  cf.bound = kLtAlpha;
  dcf_gen(k, cf, sbuf.data());
}

void ref_dcf_eval(int party, int bitlen, const uint8_t* x_le, const uint8_t* seed,
                  const uint8_t* cws, const uint8_t* cw_np1, uint8_t* out) {
  std::vector<uint8_t> sbuf(6 * kLambda, 0), x(x_le, x_le + (bitlen + 7) / 8);
  std::memcpy(sbuf.data(), seed, kLambda);
  Key k{const_cast<uint8_t*>(cws), const_cast<uint8_t*>(cw_np1)};
  dcf_eval(sbuf.data(), static_cast<uint8_t>(party), k, Bits{x.data(), bitlen});
  std::memcpy(out, sbuf.data(), kLambda);
}

// proto::Myl7FssBackend::eval_dcf on a u64 point; returns payload_len or -1.
int ref_adapter_eval(int in_bits, const uint8_t* key, size_t key_len, uint64_t x, uint8_t* out,
                     size_t out_cap) {
  try {
    proto::Myl7FssBackend be;
    proto::FssKey k;
    k.bytes.assign(key, key + key_len);
    auto o = be.eval_dcf(in_bits, k, be.u64_to_bits_msb(x, in_bits));
    if (o.size() > out_cap) return -1;
    std::memcpy(out, o.data(), o.size());
    return static_cast<int>(o.size());
  } catch (...) {
    return -1;
  }
}

int ref_adapter_eval_many(int in_bits, size_t key_bytes, const uint8_t* keys, const uint64_t* xs,
                          size_t n, int out_bytes, uint8_t* out) {
  try {
    proto::Myl7FssBackend be;
    std::vector<uint64_t> v(xs, xs + n);
    be.eval_dcf_many_u64(in_bits, key_bytes, keys, v, out_bytes, out);
    return 0;
  } catch (...) {
    return -1;
  }
}

// proto::Myl7FssBackend::gen_dcf (seeds drawn by the adapter from random_device).
int ref_adapter_gen(int in_bits, uint64_t alpha, const uint8_t* payload, size_t plen,
                    uint8_t* key0, uint8_t* key1, size_t cap) {
  try {
    warm_adapter();
    proto::Myl7FssBackend be;
    auto kp = be.gen_dcf(in_bits, be.u64_to_bits_msb(alpha, in_bits),
                         std::vector<uint8_t>(payload, payload + plen));
    if (kp.k0.bytes.size() > cap) return -1;
    std::memcpy(key0, kp.k0.bytes.data(), kp.k0.bytes.size());
    std::memcpy(key1, kp.k1.bytes.data(), kp.k1.bytes.size());
    return static_cast<int>(kp.k0.bytes.size());
  } catch (...) {
    return -1;
  }
}
}
