// Runtime plumbing behind the C ABI: error reporting, device, streams,
// memory, events; the AES-128-CTR and myl7 PRG kernels; seeded host inputs.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstring>
#include <random>
#include <string>

#include "aes_bitsliced.hpp"
#include "aes_lds.hpp"
#include "sufhip_internal.hpp"

namespace sufhip {

namespace {
thread_local std::string t_last_error;
std::atomic<bool> g_keystream_per_party{false};
}

void set_error(const std::string& msg) { t_last_error = msg; }

bool keystream_per_party() { return g_keystream_per_party.load(); }
void clear_error() { t_last_error.clear(); }

int hip_status(hipError_t st, const char* what) {
  set_error(std::string(what) + ": " + hipGetErrorString(st));
  return st == hipErrorOutOfMemory ? SUFHIP_ERR_NOMEM : SUFHIP_ERR_HIP;
}

int check_launch(const char* what) {
  hipError_t st = hipGetLastError();
  if (st != hipSuccess) return hip_status(st, what);
  return SUFHIP_OK;
}

// One AES block per thread; T table replicated 32 ways in LDS.
constexpr int kCtrCopies = 32;

__global__ void __launch_bounds__(256) aes128_ctr_kernel(uint8_t* __restrict__ out,
                                                         RoundKeys rk, uint64_t ctr_lo,
                                                         uint64_t ctr_hi, size_t blocks) {
  __shared__ __align__(16) uint32_t lds[256 * kCtrCopies];
  __shared__ uint4 rkl[11];
  fill_ttable<kCtrCopies>(lds, kTDev.v);
  fill_round_keys(rkl, &rk.w, 1);
  __syncthreads();
  AesLds<kCtrCopies> aes{lds, threadIdx.x % kCtrCopies};
  for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < blocks;
       i += size_t(gridDim.x) * blockDim.x) {
    uint64_t c = ctr_lo + i;
    uint32_t s0 = uint32_t(c), s1 = uint32_t(c >> 32), s2 = uint32_t(ctr_hi),
             s3 = uint32_t(ctr_hi >> 32);
    aes.encrypt(s0, s1, s2, s3, rkl);
    uint4 v = make_uint4(s0, s1, s2, s3);
    *reinterpret_cast<uint4*>(out + 16 * i) = v;
  }
}

// The same keystream bitsliced (aes_bitsliced.hpp): lane g encrypts the 32
// counter blocks 32 g .. 32 g + 31 held as 128 slices, no tables.  Block k's
// counter is c0 + k, c0 = ctr_lo + 32 g: its low 5 bits, (c0 + k) mod 32,
// are rotations of fixed patterns (c0 mod 32 = ctr_lo mod 32 for every
// lane), and its bits above come from c0 - c0 mod 32 for the blocks before
// the carry out of bit 4 and from 32 more after it.
__global__ void __launch_bounds__(256) aes128_ctr_bs_kernel(uint8_t* __restrict__ out,
                                                            RoundKeys rk, uint64_t ctr_lo,
                                                            uint64_t ctr_hi, size_t blocks) {
  const size_t groups = (blocks + 31) / 32;
  const uint32_t low = uint32_t(ctr_lo) & 31u;
  const uint32_t first = low == 0 ? 0xffffffffu : (1u << (32 - low)) - 1u;  // k < 32 - low
  constexpr uint32_t kPat[5] = {0xaaaaaaaau, 0xccccccccu, 0xf0f0f0f0u, 0xff00ff00u, 0xffff0000u};
  for (size_t g = blockIdx.x * size_t(blockDim.x) + threadIdx.x; g < groups;
       g += size_t(gridDim.x) * blockDim.x) {
    const uint64_t h0 = (ctr_lo + 32 * uint64_t(g)) & ~uint64_t(31), h1 = h0 + 32;
    uint32_t s[128];
#pragma unroll
    for (int b = 0; b < 5; ++b)
      s[b] = low == 0 ? kPat[b] : ((kPat[b] >> low) | (kPat[b] << (32 - low)));
#pragma unroll
    for (int i = 5; i < 64; ++i)
      s[i] = (((h0 >> i) & 1u) ? first : 0u) | (((h1 >> i) & 1u) ? ~first : 0u);
#pragma unroll
    for (int i = 0; i < 64; ++i) s[64 + i] = 0u - uint32_t((ctr_hi >> i) & 1u);
    aes_bs::encrypt(s, rk.w);
    // Quarter w of the slices transposed holds word w of each block.
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t a[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) a[i] = s[32 * w + i];
      aes_bs::transpose32(a);
#pragma unroll
      for (int i = 0; i < 32; ++i) s[32 * w + i] = a[i];
    }
    const size_t b0 = 32 * g;
#pragma unroll
    for (int k = 0; k < 32; ++k)
      if (b0 + k < blocks)
        *reinterpret_cast<uint4*>(out + 16 * (b0 + k)) =
            make_uint4(s[k], s[32 + k], s[64 + k], s[96 + k]);
  }
}

__global__ void __launch_bounds__(256) prg_mmo_kernel(PrgKeys keys, int out_blocks,
                                                      const uint8_t* __restrict__ seeds,
                                                      uint8_t* __restrict__ out, size_t n) {
  __shared__ __align__(16) uint32_t lds[256 * kCtrCopies];
  __shared__ uint4 rkl[kPrgMaxBlocks * 11];
  fill_ttable<kCtrCopies>(lds, kTDev.v);
  fill_round_keys(rkl, keys.rk, kPrgMaxBlocks);
  __syncthreads();
  AesLds<kCtrCopies> aes{lds, threadIdx.x % kCtrCopies};
  for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x) {
    const uint32_t* sp = reinterpret_cast<const uint32_t*>(seeds + 16 * i);
    uint32_t a = sp[0], b = sp[1], c = sp[2], d = sp[3];
    for (int j = 0; j < out_blocks; ++j) {
      uint32_t s0 = a, s1 = b, s2 = c, s3 = d;
      aes.encrypt(s0, s1, s2, s3, rkl + 11 * j);
      uint4 v = make_uint4(s0 ^ a, s1 ^ b, s2 ^ c, s3 ^ d);
      *reinterpret_cast<uint4*>(out + 16 * (size_t(out_blocks) * i + j)) = v;
    }
  }
}

unsigned int capped_grid(size_t n, unsigned int block) {
  size_t g = (n + block - 1) / block;
  if (g > 65536 * 4) g = 65536 * 4;
  return static_cast<unsigned int>(g);
}

}  // namespace sufhip

using namespace sufhip;

extern "C" {

int sufhip_abi_version(void) { return SUFHIP_ABI_VERSION; }

int sufhip_set_keystream_per_party(int per_party) {
  g_keystream_per_party.store(per_party != 0);
  return SUFHIP_OK;
}

int sufhip_keystream_per_party(void) { return g_keystream_per_party.load() ? 1 : 0; }

const char* sufhip_last_error(void) { return t_last_error.c_str(); }

int sufhip_init(int device) {
  int count = 0;
  SUFHIP_CHECK(hipGetDeviceCount(&count), "hipGetDeviceCount");
  SUFHIP_REQUIRE(device >= 0 && device < count, "sufhip_init: device index out of range");
  SUFHIP_CHECK(hipSetDevice(device), "hipSetDevice");
  hipDeviceProp_t prop;
  SUFHIP_CHECK(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    set_error(std::string("sufhip_init: built for gfx950, device is ") + prop.gcnArchName);
    return SUFHIP_ERR_INVALID;
  }
  return SUFHIP_OK;
}

int sufhip_device_count(int* count) {
  SUFHIP_REQUIRE(count, "sufhip_device_count: null");
  SUFHIP_CHECK(hipGetDeviceCount(count), "hipGetDeviceCount");
  return SUFHIP_OK;
}

int sufhip_stream_create(void** stream) {
  SUFHIP_REQUIRE(stream, "sufhip_stream_create: null");
  hipStream_t s = nullptr;
  SUFHIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
  *stream = s;
  return SUFHIP_OK;
}

int sufhip_stream_destroy(void* stream) {
  if (!stream) return SUFHIP_OK;
  SUFHIP_CHECK(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy");
  return SUFHIP_OK;
}

int sufhip_stream_synchronize(void* stream) {
  SUFHIP_CHECK(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
  return SUFHIP_OK;
}

int sufhip_malloc(void** d_ptr, size_t bytes) {
  SUFHIP_REQUIRE(d_ptr, "sufhip_malloc: null");
  *d_ptr = nullptr;
  if (bytes == 0) return SUFHIP_OK;
  SUFHIP_CHECK(hipMalloc(d_ptr, bytes), "hipMalloc");
  return SUFHIP_OK;
}

int sufhip_free(void* d_ptr) {
  if (!d_ptr) return SUFHIP_OK;
  SUFHIP_CHECK(hipFree(d_ptr), "hipFree");
  return SUFHIP_OK;
}

int sufhip_host_alloc(void** h_ptr, size_t bytes) {
  SUFHIP_REQUIRE(h_ptr, "sufhip_host_alloc: null");
  *h_ptr = nullptr;
  if (bytes == 0) return SUFHIP_OK;
  SUFHIP_CHECK(hipHostMalloc(h_ptr, bytes, hipHostMallocDefault), "hipHostMalloc");
  return SUFHIP_OK;
}

int sufhip_host_free(void* h_ptr) {
  if (!h_ptr) return SUFHIP_OK;
  SUFHIP_CHECK(hipHostFree(h_ptr), "hipHostFree");
  return SUFHIP_OK;
}

int sufhip_memcpy_h2d(void* d_dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_dst && src, "sufhip_memcpy_h2d: null");
  SUFHIP_CHECK(hipMemcpyAsync(d_dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)),
               "hipMemcpyAsync H2D");
  return SUFHIP_OK;
}

int sufhip_memcpy_d2h(void* dst, const void* d_src, size_t bytes, void* stream) {
  if (bytes == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(dst && d_src, "sufhip_memcpy_d2h: null");
  SUFHIP_CHECK(hipMemcpyAsync(dst, d_src, bytes, hipMemcpyDeviceToHost, as_stream(stream)),
               "hipMemcpyAsync D2H");
  return SUFHIP_OK;
}

int sufhip_memcpy_d2d(void* d_dst, const void* d_src, size_t bytes, void* stream) {
  if (bytes == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_dst && d_src, "sufhip_memcpy_d2d: null");
  SUFHIP_CHECK(hipMemcpyAsync(d_dst, d_src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)),
               "hipMemcpyAsync D2D");
  return SUFHIP_OK;
}

int sufhip_event_create(void** ev) {
  SUFHIP_REQUIRE(ev, "sufhip_event_create: null");
  hipEvent_t e = nullptr;
  SUFHIP_CHECK(hipEventCreate(&e), "hipEventCreate");
  *ev = e;
  return SUFHIP_OK;
}

int sufhip_event_destroy(void* ev) {
  if (!ev) return SUFHIP_OK;
  SUFHIP_CHECK(hipEventDestroy(reinterpret_cast<hipEvent_t>(ev)), "hipEventDestroy");
  return SUFHIP_OK;
}

int sufhip_event_record(void* ev, void* stream) {
  SUFHIP_REQUIRE(ev, "sufhip_event_record: null");
  SUFHIP_CHECK(hipEventRecord(reinterpret_cast<hipEvent_t>(ev), as_stream(stream)),
               "hipEventRecord");
  return SUFHIP_OK;
}

int sufhip_event_synchronize(void* ev) {
  SUFHIP_REQUIRE(ev, "sufhip_event_synchronize: null event");
  SUFHIP_CHECK(hipEventSynchronize(reinterpret_cast<hipEvent_t>(ev)), "hipEventSynchronize");
  return SUFHIP_OK;
}

int sufhip_event_elapsed_ms(void* start, void* stop, float* ms) {
  SUFHIP_REQUIRE(start && stop && ms, "sufhip_event_elapsed_ms: null");
  SUFHIP_CHECK(hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop)), "hipEventSynchronize");
  SUFHIP_CHECK(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                   reinterpret_cast<hipEvent_t>(stop)),
               "hipEventElapsedTime");
  return SUFHIP_OK;
}

int sufhip_aes128_ctr(uint8_t* d_out, const uint8_t* round_keys, uint64_t ctr_lo,
                      uint64_t ctr_hi, size_t blocks, void* stream) {
  if (blocks == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_out && round_keys, "sufhip_aes128_ctr: null pointer");
  RoundKeys rk;
  std::memcpy(rk.w, round_keys, 176);
  hipLaunchKernelGGL(aes128_ctr_kernel, dim3(capped_grid(blocks, 256)), dim3(256), 0,
                     as_stream(stream), d_out, rk, ctr_lo, ctr_hi, blocks);
  return check_launch("aes128_ctr_kernel");
}

int sufhip_aes128_ctr_bitsliced(uint8_t* d_out, const uint8_t* round_keys, uint64_t ctr_lo,
                                uint64_t ctr_hi, size_t blocks, void* stream) {
  if (blocks == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_out && round_keys, "sufhip_aes128_ctr_bitsliced: null pointer");
  SUFHIP_REQUIRE((reinterpret_cast<uintptr_t>(d_out) & 15) == 0,
                 "sufhip_aes128_ctr_bitsliced: d_out must be 16-byte aligned");
  RoundKeys rk;
  std::memcpy(rk.w, round_keys, 176);
  hipLaunchKernelGGL(aes128_ctr_bs_kernel, dim3(capped_grid((blocks + 31) / 32, 256)), dim3(256),
                     0, as_stream(stream), d_out, rk, ctr_lo, ctr_hi, blocks);
  return check_launch("aes128_ctr_bs_kernel");
}

int sufhip_prg_mmo(const uint8_t* prg_state, const uint8_t* d_seeds, size_t n, int out_blocks,
                   uint8_t* d_out, void* stream) {
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(prg_state && d_seeds && d_out, "sufhip_prg_mmo: null pointer");
  SUFHIP_REQUIRE(out_blocks >= 1 && out_blocks <= kPrgMaxBlocks,
                 "sufhip_prg_mmo: out_blocks must be in [1, 8]");
  SUFHIP_REQUIRE((reinterpret_cast<uintptr_t>(d_seeds) & 3) == 0 &&
                     (reinterpret_cast<uintptr_t>(d_out) & 15) == 0,
                 "sufhip_prg_mmo: seeds must be 4-byte and out 16-byte aligned");
  PrgKeys keys;
  expand_prg_keys(prg_state, out_blocks, &keys);
  hipLaunchKernelGGL(prg_mmo_kernel, dim3(capped_grid(n, 256)), dim3(256), 0, as_stream(stream),
                     keys, out_blocks, d_seeds, d_out, n);
  return check_launch("prg_mmo_kernel");
}

int sufhip_host_mt19937_64(uint64_t seed, uint64_t* out, size_t n) {
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(out, "sufhip_host_mt19937_64: null");
  std::mt19937_64 g(seed);
  for (size_t i = 0; i < n; ++i) out[i] = g();
  return SUFHIP_OK;
}

int sufhip_host_normal_fixed(uint64_t seed, double sigma, double clip, int frac_bits,
                             uint64_t* out, size_t n) {
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(out, "sufhip_host_normal_fixed: null");
  SUFHIP_REQUIRE(frac_bits >= 0 && frac_bits <= 40, "sufhip_host_normal_fixed: frac_bits");
  std::mt19937_64 g(seed);
  const double scale = std::ldexp(1.0, frac_bits);
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t i = 0; i < n; i += 2) {
    // Box-Muller on two 53-bit uniforms in (0, 1].
    double u1 = (double((g() >> 11) + 1)) * 0x1.0p-53;
    double u2 = (double(g() >> 11)) * 0x1.0p-53;
    double r = std::sqrt(-2.0 * std::log(u1));
    double z[2] = {r * std::cos(two_pi * u2), r * std::sin(two_pi * u2)};
    for (int k = 0; k < 2 && i + k < n; ++k) {
      double v = sigma * z[k];
      if (clip > 0) v = v < -clip ? -clip : (v > clip ? clip : v);
      out[i + k] = static_cast<uint64_t>(static_cast<int64_t>(std::llround(v * scale)));
    }
  }
  return SUFHIP_OK;
}

}  // extern "C"
