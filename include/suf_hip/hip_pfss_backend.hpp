// HipPfssBackend: SUF's PFSS backend interfaces on an MI355X, over the C ABI
// of libsuf_hip.so (include/suf_hip.h).  It takes the place of
// GpuPfssBackend (cuda/pfss_backend_gpu.cu:460-1500) as a new `hip` kind of
// make_pfss_backend (include/proto/backend_factory.hpp:95-164).
//
// DCF keys are real two-party myl7/fss v0.7.1 keys (128-bit seeds, AES-128-MMO
// PRG) in the Myl7FssBackend blob layout (include/proto/myl7_fss_backend.hpp:
// 131-213); keygen and evaluation run on the GPU.  Output group: with
// Params::xor_payloads, XOR of bytes for every payload length -- the group SUF
// links myl7 with (third_party/myl7_fss/src/group/bytes.c), so keys made by
// Myl7FssBackend evaluate as there; by default XOR for 1-byte payloads
// (XorBytes predicates) and addition mod 2^127 -- additive mod 2^64 in the
// low 8 bytes -- for longer payloads (AddU64 predicates and coefficient
// payloads).  A key blob does not record its group: keys made under one
// setting evaluate correctly only under the same setting.  Interval-LUT and
// packed compare keys use the GpuPfssBackend blob formats and kernel counters.
//
// Conventions follow the reference: one instance per party, calls serialized
// by an internal mutex, host-output calls return after the device-to-host
// copy completes, device outputs stay valid until the next call, failures
// throw std::runtime_error (no silent host fallback).  The myl7 PRG keys are
// process-wide (as prg_init makes them): both parties' instances in one
// process share them; set_prg_state() fixes them for reproducible runs.
#pragma once

#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "suf_hip/proto_iface.hpp"

namespace suf_hip {

class HipPfssBackend final : public proto::PfssIntervalLutExt,
                             public proto::PackedLtBackend,
                             public proto::PfssGpuStagedEval {
 public:
  struct Params {
    int device = 0;
    // 0: DCF seeds from std::random_device (as Myl7FssBackend); otherwise
    // std::mt19937_64(seed) for reproducible key material.
    uint64_t seed = 0;
    // true: the XOR byte group for every DCF payload length (Myl7FssBackend's
    // keys and outputs); false: XOR for 1-byte payloads, addition mod 2^127
    // for longer ones.
    bool xor_payloads = false;
  };

  HipPfssBackend();
  explicit HipPfssBackend(Params p);
  ~HipPfssBackend() override;
  HipPfssBackend(const HipPfssBackend&) = delete;
  HipPfssBackend& operator=(const HipPfssBackend&) = delete;

  // Process-wide myl7 PRG state (kBlocks x lambda = 128 bytes).  Drawn from
  // std::random_device on first use unless set first.
  static void set_prg_state(const uint8_t state[128]);
  static std::vector<uint8_t> prg_state();

  // PfssBackend
  std::vector<uint8_t> u64_to_bits_msb(uint64_t x, int in_bits) const override;
  proto::BitOrder bit_order() const override { return proto::BitOrder::MSB_FIRST; }
  proto::DcfKeyPair gen_dcf(int in_bits, const std::vector<uint8_t>& alpha_bits,
                            const std::vector<uint8_t>& payload_bytes) override;
  std::vector<uint8_t> eval_dcf(int in_bits, const proto::FssKey& kb,
                                const std::vector<uint8_t>& x_bits) const override;
  // PfssBackendBatch.  out_bytes == 1 on a 1-byte-payload key gives share
  // byte 0 & 1 per key (Myl7FssBackend::eval_dcf_many_u64); otherwise the first
  // out_bytes bytes of the payload share.
  void eval_dcf_many_u64(int in_bits, size_t key_bytes, const uint8_t* keys_flat,
                         const std::vector<uint64_t>& xs_u64, int out_bytes,
                         uint8_t* outs_flat) const override;
  // PfssIntervalLutExt
  proto::IntervalLutKeyPair gen_interval_lut(const proto::IntervalLutDesc& desc) override;
  void eval_interval_lut_many_u64(size_t key_bytes, const uint8_t* keys_flat,
                                  const std::vector<uint64_t>& xs_u64, int out_words,
                                  uint64_t* outs_flat) const override;
  // PackedLtBackend
  proto::PackedLtKeyPair gen_packed_lt(int in_bits, const std::vector<uint64_t>& thresholds) override;
  void eval_packed_lt_many(size_t key_bytes, const uint8_t* keys_flat,
                           const std::vector<uint64_t>& xs_u64, int in_bits, int out_words,
                           uint64_t* outs_bitmask) const override;
  // PfssGpuStagedEval
  void eval_dcf_many_u64_device(int in_bits, size_t key_bytes, const uint8_t* keys_flat,
                                const uint64_t* xs_device, size_t N, int out_bytes,
                                uint8_t* outs_flat) const override;
  void eval_dcf_many_u64_device_broadcast(int in_bits, size_t key_bytes, const uint8_t* key,
                                          const uint64_t* xs_device, size_t N, int out_bytes,
                                          uint8_t* outs_flat) const override;
  void eval_packed_lt_many_device(size_t key_bytes, const uint8_t* keys_flat,
                                  const uint64_t* xs_device, size_t N, int in_bits, int out_words,
                                  uint64_t* outs_bitmask) const override;
  void eval_packed_lt_many_device_broadcast(size_t key_bytes, const uint8_t* key,
                                            const uint64_t* xs_device, size_t N, int in_bits,
                                            int out_words, uint64_t* outs_bitmask) const override;
  void eval_interval_lut_many_device(size_t key_bytes, const uint8_t* keys_flat,
                                     const uint64_t* xs_device, size_t N, int out_words,
                                     uint64_t* outs_flat) const override;
  void eval_interval_lut_many_device_broadcast(size_t key_bytes, const uint8_t* key,
                                               const uint64_t* xs_device, size_t N, int out_words,
                                               uint64_t* outs_flat) const override;
  void* device_stream() const override { return stream_; }
  const uint64_t* last_device_output() const override;
  const uint64_t* last_device_bools() const override;
  void ensure_output_buffers(size_t arith_words, size_t bool_words) const override;

 private:
  struct Buf {
    void* ptr = nullptr;
    size_t cap = 0;
  };
  void ensure(Buf& b, size_t bytes) const;
  const uint8_t* stage_keys(const uint8_t* host, size_t bytes) const;
  const uint8_t* stage_broadcast_key(const uint8_t* host, size_t bytes) const;
  const uint64_t* stage_xs(const std::vector<uint64_t>& xs) const;
  void dcf_eval_dev(int in_bits, size_t key_bytes, const uint8_t* d_keys, int bcast,
                    int payload_len, const uint64_t* d_xs, size_t n, int out_bytes,
                    uint8_t* outs_host) const;
  void sync() const;
  std::vector<uint8_t> random_bytes(size_t n);
  int group_for(int payload_len) const;

  Params params_;
  void* stream_ = nullptr;
  mutable std::mutex mu_;
  mutable Buf keys_, xs_, out_, bools_, scratch_;
  // Broadcast key blobs staged on the device, keyed by content (host copy
  // kept to confirm the match), never by host address.
  struct Staged {
    std::vector<uint8_t> host;
    void* dev = nullptr;
  };
  mutable std::unordered_map<uint64_t, Staged> staged_;
  uint64_t next_id_ = 1;
  std::unique_ptr<struct HipRng> rng_;
};

// SUF_PFSS_BACKEND=hip selects this backend; returns nullptr for other values.
std::unique_ptr<proto::PfssBackendBatch> make_hip_backend_from_env();

}  // namespace suf_hip
