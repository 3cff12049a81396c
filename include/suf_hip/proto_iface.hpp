// The SUF PFSS backend interfaces that HipPfssBackend implements.
//
// Inside the SUF tree, define SUF_HIP_USE_REFERENCE_PROTO and the reference's
// own headers are used.  Standalone (this repository's tests), the same
// declarations are stated here with identical names, signatures and
// semantics so the backend compiles and runs without the SUF tree:
//   FssKey, DcfKeyPair, BitOrder, PfssBackend   include/proto/pfss_backend.hpp:8-54
//   PfssBackendBatch                            include/proto/pfss_backend_batch.hpp:10-29
//   IntervalLutKeyPair, IntervalLutDesc,
//   PfssIntervalLutExt                          include/proto/pfss_interval_lut_ext.hpp:8-27
//   PackedLtKeyPair, PackedLtBackend            include/proto/packed_backend.hpp:8-24
//   PfssGpuStagedEval                           include/proto/backend_gpu.hpp:15-68
#pragma once

#ifdef SUF_HIP_USE_REFERENCE_PROTO
#include "proto/backend_gpu.hpp"
#include "proto/packed_backend.hpp"
#include "proto/pfss_backend.hpp"
#include "proto/pfss_backend_batch.hpp"
#include "proto/pfss_interval_lut_ext.hpp"
#else
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <vector>

namespace proto {

using u8 = uint8_t;
using u64 = uint64_t;

struct FssKey {
  std::vector<u8> bytes;
};

struct DcfKeyPair {
  FssKey k0;
  FssKey k1;
};

enum class BitOrder : uint8_t { MSB_FIRST, LSB_FIRST };

struct PfssBackend {
  virtual ~PfssBackend() = default;
  // Key pair for f(x) = payload if x < alpha else 0.
  virtual DcfKeyPair gen_dcf(int in_bits, const std::vector<u8>& alpha_bits,
                             const std::vector<u8>& payload_bytes) = 0;
  // One party's share at one point.
  virtual std::vector<u8> eval_dcf(int in_bits, const FssKey& kb,
                                   const std::vector<u8>& x_bits) const = 0;
  virtual std::vector<u8> u64_to_bits_msb(u64 x, int in_bits) const = 0;
  virtual BitOrder bit_order() const { return BitOrder::MSB_FIRST; }
};

struct PfssBackendBatch : public PfssBackend {
  // keys_flat [N][key_bytes], outs_flat [N][out_bytes]
  virtual void eval_dcf_many_u64(int in_bits, size_t key_bytes, const uint8_t* keys_flat,
                                 const std::vector<u64>& xs_u64, int out_bytes,
                                 uint8_t* outs_flat) const {
    for (size_t i = 0; i < xs_u64.size(); i++) {
      FssKey kb;
      kb.bytes.assign(keys_flat + i * key_bytes, keys_flat + (i + 1) * key_bytes);
      auto out = eval_dcf(in_bits, kb, u64_to_bits_msb(xs_u64[i], in_bits));
      if (out.size() != static_cast<size_t>(out_bytes))
        throw std::runtime_error("eval_dcf_many_u64: output size mismatch");
      std::memcpy(outs_flat + i * out_bytes, out.data(), out_bytes);
    }
  }
};

struct IntervalLutKeyPair {
  FssKey k0, k1;
};

struct IntervalLutDesc {
  int in_bits = 64;
  int out_words = 0;               // u64 words per output
  std::vector<u64> cutpoints;      // increasing, in the masked domain
  std::vector<u64> payload_flat;   // [intervals][out_words]
};

struct PfssIntervalLutExt : public PfssBackendBatch {
  virtual IntervalLutKeyPair gen_interval_lut(const IntervalLutDesc& desc) = 0;
  virtual void eval_interval_lut_many_u64(size_t key_bytes, const uint8_t* keys_flat,
                                          const std::vector<u64>& xs_u64, int out_words,
                                          u64* outs_flat) const = 0;
};

struct PackedLtKeyPair {
  FssKey k0, k1;
};

class PackedLtBackend {
 public:
  virtual ~PackedLtBackend() = default;
  virtual PackedLtKeyPair gen_packed_lt(int in_bits, const std::vector<u64>& thresholds) = 0;
  // outs_bitmask [N][out_words]
  virtual void eval_packed_lt_many(size_t key_bytes, const uint8_t* keys_flat,
                                   const std::vector<u64>& xs_u64, int in_bits, int out_words,
                                   u64* outs_bitmask) const = 0;
};

// Device-pointer evaluation (xs already on the device).  `outs` may be null to
// keep results only in backend-owned device buffers (last_device_*()).
struct PfssGpuStagedEval {
  virtual ~PfssGpuStagedEval() = default;
  virtual void eval_dcf_many_u64_device(int in_bits, size_t key_bytes, const uint8_t* keys_flat,
                                        const uint64_t* xs_device, size_t N, int out_bytes,
                                        uint8_t* outs_flat) const = 0;
  virtual void eval_dcf_many_u64_device_broadcast(int in_bits, size_t key_bytes,
                                                  const uint8_t* key, const uint64_t* xs_device,
                                                  size_t N, int out_bytes,
                                                  uint8_t* outs_flat) const = 0;
  virtual void eval_packed_lt_many_device(size_t key_bytes, const uint8_t* keys_flat,
                                          const uint64_t* xs_device, size_t N, int in_bits,
                                          int out_words, uint64_t* outs_bitmask) const = 0;
  virtual void eval_packed_lt_many_device_broadcast(size_t key_bytes, const uint8_t* key,
                                                    const uint64_t* xs_device, size_t N,
                                                    int in_bits, int out_words,
                                                    uint64_t* outs_bitmask) const = 0;
  virtual void eval_interval_lut_many_device(size_t key_bytes, const uint8_t* keys_flat,
                                             const uint64_t* xs_device, size_t N, int out_words,
                                             uint64_t* outs_flat) const = 0;
  virtual void eval_interval_lut_many_device_broadcast(size_t key_bytes, const uint8_t* key,
                                                       const uint64_t* xs_device, size_t N,
                                                       int out_words,
                                                       uint64_t* outs_flat) const = 0;
  virtual void* device_stream() const = 0;
  virtual const uint64_t* last_device_output() const { return nullptr; }
  virtual const uint64_t* last_device_bools() const { return nullptr; }
  virtual void ensure_output_buffers(size_t /*arith_words*/, size_t /*bool_words*/) const {}
};

}  // namespace proto
#endif
