// Offline key material on tapes, for the HIP backend's host side.
//
// TapeWriter / TapeReader write and read SUF's tape records
// (include/proto/tape.hpp:109-232): a record is [tag u32 LE][len u32 LE]
// [payload], tags kU64 = 1, kU64Vec = 2, kBytes = 3, kTriple64 = 4 (u64
// words and {a, b, c} triples little-endian), over an in-memory buffer or a
// file; reading checks the tag and the payload size.  The byte stream is the
// reference's (tests/golden/tape_records.bin holds one written by the
// reference's own TapeWriter).
//
// CompositeTapeKey is the party key that gates::write_composite_tape /
// read_composite_tape serialise (include/gates/composite_fss.hpp:2458-2641),
// in the same field order and encoding: mask shares, wrap shares, the
// predicate / cut / coefficient key metadata and key blobs, coefficient
// shares, Beaver triples and bit triples.
//
// Per-element key arrays (N keys of key_bytes, e.g. DCF or truncation-gate
// keys for a batch) go on a tape as [kU64 N][kU64 key_bytes] and then kBytes
// blocks of whole keys; DeviceKeyArray streams them into one device buffer
// through two pinned staging buffers, so a batch's keys never need to be
// whole in host memory.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <memory>
#include <string>
#include <vector>

namespace suf_hip {

enum class TapeTag : uint32_t { kU64 = 1, kU64Vec = 2, kBytes = 3, kTriple64 = 4 };

struct Triple64 {
  uint64_t a = 0, b = 0, c = 0;
};

struct BitTriple {
  uint8_t a = 0, b = 0, c = 0;
};

class TapeSink {
 public:
  virtual ~TapeSink() = default;
  virtual void write(const uint8_t* data, size_t n) = 0;
  virtual void flush() {}
};

class TapeSource {
 public:
  virtual ~TapeSource() = default;
  virtual void read_exact(uint8_t* out, size_t n) = 0;
  virtual bool eof() = 0;
};

class BufferSink final : public TapeSink {
 public:
  std::vector<uint8_t> bytes;
  void write(const uint8_t* data, size_t n) override;
};

class BufferSource final : public TapeSource {
 public:
  BufferSource(const uint8_t* data, size_t n) : p_(data), n_(n) {}
  void read_exact(uint8_t* out, size_t n) override;
  bool eof() override { return off_ >= n_; }
  size_t offset() const { return off_; }

 private:
  const uint8_t* p_;
  size_t n_;
  size_t off_ = 0;
};

class FileSink final : public TapeSink {
 public:
  explicit FileSink(const std::string& path);
  ~FileSink() override;
  void write(const uint8_t* data, size_t n) override;
  void flush() override;

 private:
  std::FILE* f_ = nullptr;
};

class FileSource final : public TapeSource {
 public:
  explicit FileSource(const std::string& path);
  ~FileSource() override;
  void read_exact(uint8_t* out, size_t n) override;
  bool eof() override;

 private:
  std::FILE* f_ = nullptr;
};

class TapeWriter {
 public:
  explicit TapeWriter(TapeSink& sink) : sink_(&sink) {}
  void write_u64(uint64_t v);
  void write_u64_vec(const uint64_t* v, size_t n);
  void write_bytes(const uint8_t* b, size_t n);
  void write_triples(const Triple64* t, size_t n);
  void flush() { sink_->flush(); }

 private:
  TapeSink* sink_;
  void record(TapeTag tag, const uint8_t* payload, size_t len);
};

class TapeReader {
 public:
  explicit TapeReader(TapeSource& src) : src_(&src) {}
  uint64_t read_u64();
  std::vector<uint64_t> read_u64_vec();
  std::vector<uint8_t> read_bytes();
  // Reads a kBytes record into `out` (capacity `cap`); returns its length.
  size_t read_bytes_into(uint8_t* out, size_t cap);
  // A kBytes record read in pieces: begin_bytes() reads the header and
  // returns the payload length, read_raw() then takes the payload in order.
  size_t begin_bytes() { return header(TapeTag::kBytes); }
  void read_raw(uint8_t* out, size_t n) { src_->read_exact(out, n); }
  std::vector<Triple64> read_triples();
  bool eof() { return src_->eof(); }

 private:
  TapeSource* src_;
  uint32_t header(TapeTag expect);
};

// gates::CompositePartyKey's serialised fields (composite_fss.hpp:140-200).
struct CompositeTapeKey {
  uint64_t r_in_share = 0;
  std::vector<uint64_t> r_in_share_vec;
  std::vector<uint64_t> r_out_share;
  std::vector<uint64_t> wrap_share;
  uint64_t r_hi_share = 0;
  uint64_t wrap_sign_share = 0;
  std::vector<uint64_t> extra_params;
  struct Meta {
    uint8_t bit_order = 0;  // proto::BitOrder
    uint8_t sem = 0;        // proto::ShareSemantics
    uint32_t out_bytes = 0;
  };
  Meta pred_meta, cut_pred_meta;
  uint8_t coeff_bit_order = 0, coeff_sem = 0;  // proto::CoeffKeyMeta
  std::vector<std::vector<uint8_t>> pred_keys, cut_pred_keys, coeff_keys;
  std::vector<uint64_t> base_coeff_share, total_delta_share;
  std::vector<Triple64> triples;
  std::vector<BitTriple> bit_triples;
};

std::vector<uint8_t> write_composite_tape(const CompositeTapeKey& k);
// Throws std::runtime_error("composite tape truncated") on a short buffer.
CompositeTapeKey read_composite_tape(const uint8_t* data, size_t len);

// N keys of key_bytes as [kU64 N][kU64 key_bytes][kBytes block]..., blocks
// of at most keys_per_block whole keys.
void write_key_array(TapeWriter& w, const uint8_t* keys, size_t n, size_t key_bytes,
                     size_t keys_per_block);

// A device buffer filled from a key-array section of a tape.
class DeviceKeyArray {
 public:
  // Reads the section at the reader's position; allocates n * key_bytes
  // device bytes (8-byte aligned) and streams the blocks into them in pieces
  // of at most staging_bytes, through two pinned staging buffers alternating
  // on `stream`.  Returns once every copy has completed.
  DeviceKeyArray(TapeReader& r, void* stream, size_t staging_bytes = size_t(8) << 20);
  ~DeviceKeyArray();
  DeviceKeyArray(const DeviceKeyArray&) = delete;
  DeviceKeyArray& operator=(const DeviceKeyArray&) = delete;
  const uint8_t* data() const { return static_cast<const uint8_t*>(d_); }
  size_t size() const { return n_; }
  size_t key_bytes() const { return kb_; }

 private:
  void* d_ = nullptr;
  size_t n_ = 0, kb_ = 0;
};

}  // namespace suf_hip
