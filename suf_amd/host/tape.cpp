// Tape records, the composite party-key tape and key-array streaming
// (include/suf_hip/tape.hpp).  Little-endian encodings are written byte by
// byte, so the bytes do not depend on the host's byte order.
#include "suf_hip/tape.hpp"

#include <cstring>
#include <stdexcept>

#include "suf_hip.h"

namespace suf_hip {

namespace {

void put_u32(std::vector<uint8_t>& v, uint32_t x) {
  for (int i = 0; i < 4; ++i) v.push_back(uint8_t(x >> (8 * i)));
}
void put_u64(std::vector<uint8_t>& v, uint64_t x) {
  for (int i = 0; i < 8; ++i) v.push_back(uint8_t(x >> (8 * i)));
}
uint32_t get_u32(const uint8_t* p) {
  return uint32_t(p[0]) | uint32_t(p[1]) << 8 | uint32_t(p[2]) << 16 | uint32_t(p[3]) << 24;
}
uint64_t get_u64(const uint8_t* p) {
  uint64_t v = 0;
  for (int i = 0; i < 8; ++i) v |= uint64_t(p[i]) << (8 * i);
  return v;
}

void hip_ok(int rc, const char* what) {
  if (rc != SUFHIP_OK) {
    const char* m = sufhip_last_error();
    throw std::runtime_error(std::string(what) + ": " + (m ? m : "sufhip error"));
  }
}

}  // namespace

void BufferSink::write(const uint8_t* data, size_t n) { bytes.insert(bytes.end(), data, data + n); }

void BufferSource::read_exact(uint8_t* out, size_t n) {
  if (n > n_ - off_) throw std::runtime_error("tape: read past end");
  std::memcpy(out, p_ + off_, n);
  off_ += n;
}

FileSink::FileSink(const std::string& path) : f_(std::fopen(path.c_str(), "wb")) {
  if (!f_) throw std::runtime_error("tape: open output failed");
}
FileSink::~FileSink() {
  if (f_) std::fclose(f_);
}
void FileSink::write(const uint8_t* data, size_t n) {
  if (n && std::fwrite(data, 1, n, f_) != n) throw std::runtime_error("tape: file write failed");
}
void FileSink::flush() {
  if (std::fflush(f_) != 0) throw std::runtime_error("tape: file flush failed");
}

FileSource::FileSource(const std::string& path) : f_(std::fopen(path.c_str(), "rb")) {
  if (!f_) throw std::runtime_error("tape: open input failed");
}
FileSource::~FileSource() {
  if (f_) std::fclose(f_);
}
void FileSource::read_exact(uint8_t* out, size_t n) {
  if (n && std::fread(out, 1, n, f_) != n) throw std::runtime_error("tape: file read failed");
}
bool FileSource::eof() {
  const int c = std::fgetc(f_);
  if (c == EOF) return true;
  std::ungetc(c, f_);
  return false;
}

void TapeWriter::record(TapeTag tag, const uint8_t* payload, size_t len) {
  if (len > 0xffffffffu) throw std::runtime_error("tape: record longer than 2^32 - 1 bytes");
  std::vector<uint8_t> h;
  put_u32(h, uint32_t(tag));
  put_u32(h, uint32_t(len));
  sink_->write(h.data(), h.size());
  if (len) sink_->write(payload, len);
}

void TapeWriter::write_u64(uint64_t v) {
  std::vector<uint8_t> b;
  put_u64(b, v);
  record(TapeTag::kU64, b.data(), 8);
}

void TapeWriter::write_u64_vec(const uint64_t* v, size_t n) {
  std::vector<uint8_t> b;
  b.reserve(8 * n);
  for (size_t i = 0; i < n; ++i) put_u64(b, v[i]);
  record(TapeTag::kU64Vec, b.data(), b.size());
}

void TapeWriter::write_bytes(const uint8_t* p, size_t n) { record(TapeTag::kBytes, p, n); }

void TapeWriter::write_triples(const Triple64* t, size_t n) {
  std::vector<uint8_t> b;
  b.reserve(24 * n);
  for (size_t i = 0; i < n; ++i) {
    put_u64(b, t[i].a);
    put_u64(b, t[i].b);
    put_u64(b, t[i].c);
  }
  record(TapeTag::kTriple64, b.data(), b.size());
}

uint32_t TapeReader::header(TapeTag expect) {
  uint8_t h[8];
  src_->read_exact(h, 8);
  if (get_u32(h) != uint32_t(expect)) throw std::runtime_error("tape: tag mismatch");
  return get_u32(h + 4);
}

uint64_t TapeReader::read_u64() {
  if (header(TapeTag::kU64) != 8) throw std::runtime_error("tape: read_u64 size mismatch");
  uint8_t b[8];
  src_->read_exact(b, 8);
  return get_u64(b);
}

std::vector<uint64_t> TapeReader::read_u64_vec() {
  const uint32_t len = header(TapeTag::kU64Vec);
  if (len % 8) throw std::runtime_error("tape: read_u64_vec size mismatch");
  std::vector<uint8_t> b(len);
  if (len) src_->read_exact(b.data(), len);
  std::vector<uint64_t> v(len / 8);
  for (size_t i = 0; i < v.size(); ++i) v[i] = get_u64(b.data() + 8 * i);
  return v;
}

std::vector<uint8_t> TapeReader::read_bytes() {
  const uint32_t len = header(TapeTag::kBytes);
  std::vector<uint8_t> b(len);
  if (len) src_->read_exact(b.data(), len);
  return b;
}

size_t TapeReader::read_bytes_into(uint8_t* out, size_t cap) {
  const uint32_t len = header(TapeTag::kBytes);
  if (len > cap) throw std::runtime_error("tape: bytes record larger than the buffer");
  if (len) src_->read_exact(out, len);
  return len;
}

std::vector<Triple64> TapeReader::read_triples() {
  const uint32_t len = header(TapeTag::kTriple64);
  if (len % 24) throw std::runtime_error("tape: read_triple64_vec size mismatch");
  std::vector<uint8_t> b(len);
  if (len) src_->read_exact(b.data(), len);
  std::vector<Triple64> t(len / 24);
  for (size_t i = 0; i < t.size(); ++i) {
    t[i].a = get_u64(b.data() + 24 * i);
    t[i].b = get_u64(b.data() + 24 * i + 8);
    t[i].c = get_u64(b.data() + 24 * i + 16);
  }
  return t;
}

std::vector<uint8_t> write_composite_tape(const CompositeTapeKey& k) {
  std::vector<uint8_t> v;
  auto vec64 = [&](const std::vector<uint64_t>& x) {
    put_u32(v, uint32_t(x.size()));
    for (uint64_t w : x) put_u64(v, w);
  };
  auto keys = [&](const std::vector<std::vector<uint8_t>>& ks) {
    put_u32(v, uint32_t(ks.size()));
    for (const auto& b : ks) {
      put_u32(v, uint32_t(b.size()));
      v.insert(v.end(), b.begin(), b.end());
    }
  };
  auto meta = [&](const CompositeTapeKey::Meta& m) {
    v.push_back(m.bit_order);
    v.push_back(m.sem);
    put_u32(v, m.out_bytes);
  };
  put_u64(v, k.r_in_share);
  vec64(k.r_in_share_vec);
  vec64(k.r_out_share);
  vec64(k.wrap_share);
  put_u64(v, k.r_hi_share);
  put_u64(v, k.wrap_sign_share);
  vec64(k.extra_params);
  meta(k.pred_meta);
  meta(k.cut_pred_meta);
  v.push_back(k.coeff_bit_order);
  v.push_back(k.coeff_sem);
  keys(k.pred_keys);
  keys(k.cut_pred_keys);
  keys(k.coeff_keys);
  vec64(k.base_coeff_share);
  vec64(k.total_delta_share);
  put_u32(v, uint32_t(k.triples.size()));
  for (const auto& t : k.triples) {
    put_u64(v, t.a);
    put_u64(v, t.b);
    put_u64(v, t.c);
  }
  put_u32(v, uint32_t(k.bit_triples.size()));
  for (const auto& t : k.bit_triples) {
    v.push_back(t.a);
    v.push_back(t.b);
    v.push_back(t.c);
  }
  return v;
}

CompositeTapeKey read_composite_tape(const uint8_t* data, size_t len) {
  CompositeTapeKey k;
  size_t off = 0;
  auto need = [&](size_t n) {
    if (n > len - off) throw std::runtime_error("composite tape truncated");
  };
  auto u64 = [&]() {
    need(8);
    const uint64_t x = get_u64(data + off);
    off += 8;
    return x;
  };
  auto u32 = [&]() {
    need(4);
    const uint32_t x = get_u32(data + off);
    off += 4;
    return x;
  };
  auto u8 = [&]() {
    need(1);
    return data[off++];
  };
  auto vec64 = [&](std::vector<uint64_t>& x) {
    const uint32_t n = u32();
    need(size_t(n) * 8);
    x.resize(n);
    for (uint32_t i = 0; i < n; ++i) x[i] = u64();
  };
  auto keys = [&](std::vector<std::vector<uint8_t>>& ks) {
    const uint32_t n = u32();
    ks.resize(n);
    for (uint32_t i = 0; i < n; ++i) {
      const uint32_t b = u32();
      need(b);
      ks[i].assign(data + off, data + off + b);
      off += b;
    }
  };
  auto meta = [&](CompositeTapeKey::Meta& m) {
    m.bit_order = u8();
    m.sem = u8();
    m.out_bytes = u32();
  };
  k.r_in_share = u64();
  vec64(k.r_in_share_vec);
  vec64(k.r_out_share);
  vec64(k.wrap_share);
  k.r_hi_share = u64();
  k.wrap_sign_share = u64();
  vec64(k.extra_params);
  meta(k.pred_meta);
  meta(k.cut_pred_meta);
  k.coeff_bit_order = u8();
  k.coeff_sem = u8();
  keys(k.pred_keys);
  keys(k.cut_pred_keys);
  keys(k.coeff_keys);
  vec64(k.base_coeff_share);
  vec64(k.total_delta_share);
  const uint32_t nt = u32();
  need(size_t(nt) * 24);
  k.triples.resize(nt);
  for (uint32_t i = 0; i < nt; ++i) {
    k.triples[i].a = u64();
    k.triples[i].b = u64();
    k.triples[i].c = u64();
  }
  const uint32_t nb = u32();
  need(size_t(nb) * 3);
  k.bit_triples.resize(nb);
  for (uint32_t i = 0; i < nb; ++i) {
    k.bit_triples[i].a = u8();
    k.bit_triples[i].b = u8();
    k.bit_triples[i].c = u8();
  }
  return k;
}

void write_key_array(TapeWriter& w, const uint8_t* keys, size_t n, size_t key_bytes,
                     size_t keys_per_block) {
  if (key_bytes == 0 || keys_per_block == 0) throw std::runtime_error("write_key_array: empty keys");
  w.write_u64(n);
  w.write_u64(key_bytes);
  for (size_t i = 0; i < n; i += keys_per_block) {
    const size_t m = n - i < keys_per_block ? n - i : keys_per_block;
    w.write_bytes(keys + i * key_bytes, m * key_bytes);
  }
}

DeviceKeyArray::DeviceKeyArray(TapeReader& r, void* stream, size_t staging_bytes) {
  n_ = size_t(r.read_u64());
  kb_ = size_t(r.read_u64());
  if (kb_ == 0 || (n_ && kb_ > (size_t(1) << 40) / n_))
    throw std::runtime_error("DeviceKeyArray: bad key-array header");
  const size_t total = n_ * kb_;
  hip_ok(sufhip_malloc(&d_, total ? total : 8), "DeviceKeyArray: device allocation");
  if (staging_bytes == 0) staging_bytes = 1;
  void* stage[2] = {nullptr, nullptr};
  void* ev[2] = {nullptr, nullptr};
  try {
    for (int b = 0; b < 2; ++b) {
      hip_ok(sufhip_host_alloc(&stage[b], staging_bytes), "DeviceKeyArray: pinned staging");
      hip_ok(sufhip_event_create(&ev[b]), "DeviceKeyArray: event");
    }
    size_t done = 0;
    int b = 0;
    bool used[2] = {false, false};
    while (done < total) {
      size_t left = r.begin_bytes();
      if (left == 0 || left % kb_ || left > total - done)
        throw std::runtime_error("DeviceKeyArray: key block does not hold whole keys of the array");
      while (left > 0) {
        // A staging buffer is refilled only after its previous copy ended.
        if (used[b]) hip_ok(sufhip_event_synchronize(ev[b]), "DeviceKeyArray: wait");
        const size_t len = left < staging_bytes ? left : staging_bytes;
        r.read_raw(static_cast<uint8_t*>(stage[b]), len);
        hip_ok(sufhip_memcpy_h2d(static_cast<uint8_t*>(d_) + done, stage[b], len, stream),
               "DeviceKeyArray: copy");
        hip_ok(sufhip_event_record(ev[b], stream), "DeviceKeyArray: event");
        used[b] = true;
        done += len;
        left -= len;
        b ^= 1;
      }
    }
    hip_ok(sufhip_stream_synchronize(stream), "DeviceKeyArray: sync");
  } catch (...) {
    sufhip_stream_synchronize(stream);
    for (int q = 0; q < 2; ++q) {
      if (stage[q]) sufhip_host_free(stage[q]);
      if (ev[q]) sufhip_event_destroy(ev[q]);
    }
    sufhip_free(d_);
    d_ = nullptr;
    throw;
  }
  for (int q = 0; q < 2; ++q) {
    sufhip_host_free(stage[q]);
    sufhip_event_destroy(ev[q]);
  }
}

DeviceKeyArray::~DeviceKeyArray() {
  if (d_) sufhip_free(d_);
}

}  // namespace suf_hip
