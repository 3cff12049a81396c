// Truncation gate on one GPU: dealer keygen and the online evaluation that
// SUF splits over composite_eval_batch_backend's AddU64 branch
// (include/gates/composite_fss.hpp:1385-1638) and the trunc postproc hook
// (include/gates/postproc_hooks.hpp:172-373), fused into one pass per party.
//
// Keygen follows composite_gen_trunc_gate (composite_fss.hpp:645-833): the
// gate's predicates after the mask rewrite (include/suf/mask_rewrite.hpp,
// src/compiler/suf_to_pfss.cpp:443-455), for x^ = x + r public and
// r_low = r mod 2^f, are
//   carry = 1[x^_low < r_low]           one f-bit DCF (none if r_low == 0)
//   wrap  = 1[x^ < r]                   TR, ARS: one 64-bit DCF
//   sign  = (wrap - 1[x^ < r + 2^63]) + 1[r < 2^63]           ARS
// with 8-byte additive payloads (SUF's AddU64 semantics).  The rewrite's
// second carry query, 1[x^_low < 0], is identically 0 and is not keyed.
//
// Evaluation of the carry DCF uses a prefix frontier: the walk state after
// the first d levels depends only on the top d bits of x^_low, so for a
// broadcast key and a large batch the 2^d frontier states are computed once
// and every element continues from its prefix.  The first k0 = min(d, 12)
// levels are walked one node per lane; deeper levels are expanded
// breadth-first, one child per lane (2 AES per node).  For f <= 14, d = f:
// the frontier holds the final share of every point of the domain and an
// element's carry is a single table read (the key-only work, 2^f walks, is
// off the critical path: it needs no input).  Above, d = min(f, max(floor(
// log2 N) - 1, 12), 22) balances the 2^(d+1) expansions against the N (f - d)
// per-element levels, never leaving more than f - 12 levels per element.  The
// results are the same bytes a full walk produces.  sufhip_trunc_prepare_batch
// runs the key-only halves of many gates in one walk launch plus one launch
// per expanded level; sufhip_trunc_finish2 evaluates both parties' keys in
// one launch.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "dcf_device.hpp"
#include "suf_hip.h"
#include "trunc_device.hpp"
#include "walk_device.hpp"

namespace sufhip {
namespace {

constexpr uint32_t kTag = kTruncTag;
constexpr int kHdrBytes = kTruncHdrBytes;
constexpr int kMaxFrontierBits = 22;
constexpr int kWalkFrontierBits = 12;

__host__ __device__ constexpr size_t pad8(size_t v) { return (v + 7) & ~size_t(7); }

size_t dcf_bytes(int in_bits) { return sufhip_dcf_key_bytes(in_bits, 8); }

int frontier_bits(int f, size_t n) {
  if (n == 0) return 0;
  if (f <= kTruncTableBits) return f;
  int lg = 0;
  while (lg < 63 && (size_t(1) << (lg + 1)) <= n) ++lg;
  int d = lg - 1 > kWalkFrontierBits ? lg - 1 : kWalkFrontierBits;
  if (d > kMaxFrontierBits) d = kMaxFrontierBits;
  return d < f ? d : f;
}

// Nodes of the walked level (k0) and of the final level (d) in the workspace:
// level d always lands in the first 2^d slots, the level before it in the
// 2^(d-1) slots after them.
int walk_bits(int d) { return d < kWalkFrontierBits ? d : kWalkFrontierBits; }

// The batched prepare walks a table gate's whole domain (d = f <= 14) in one
// launch: a lane per table entry, no expansion launches after it.
int batch_walk_bits(int d, int f) { return d == f && f <= kTruncTableBits ? d : walk_bits(d); }

size_t frontier_nodes(int d) {
  if (d == 0) return 0;
  return (size_t(1) << d) + (d > walk_bits(d) ? size_t(1) << (d - 1) : 0);
}

struct TruncGenArgs {
  Prg4 prg;
  uint8_t* key0;
  uint8_t* key1;
  uint64_t hdr[2][8];
  uint64_t alpha[3];
  uint64_t seeds[3][4];
  uint32_t off[3];
  int bits[3];
  int flags;
  uint32_t total;
};

// One workgroup: zero both blobs, write the headers, then lanes 0..2 each
// generate one DCF key pair.
__global__ void __launch_bounds__(kDcfBlock) trunc_gen_kernel(TruncGenArgs a) {
  SUFHIP_DCF_LDS_SETUP(a.prg);
  __shared__ uint8_t one8[8];
  __shared__ uint8_t seeds[3][32];
  if (threadIdx.x < 8) one8[threadIdx.x] = threadIdx.x == 0 ? 1 : 0;
  if (threadIdx.x < 96) {
    const int j = threadIdx.x / 32, b = threadIdx.x % 32;
    seeds[j][b] = uint8_t(a.seeds[j][b / 8] >> (8 * (b % 8)));
  }
  for (uint32_t i = threadIdx.x; i < a.total / 8; i += blockDim.x) {
    const uint64_t v0 = i < 8 ? a.hdr[0][i] : 0;
    const uint64_t v1 = i < 8 ? a.hdr[1][i] : 0;
    reinterpret_cast<uint64_t*>(a.key0)[i] = v0;
    reinterpret_cast<uint64_t*>(a.key1)[i] = v1;
  }
  __syncthreads();
  const int j = threadIdx.x;
  if (j < 3 && (a.flags >> j) & 1)
    gen_key<SUFHIP_GROUP_ADD>(aes, rkl, a.bits[j], 1, 8, a.alpha[j], one8, seeds[j],
                              a.key0 + a.off[j], a.key1 + a.off[j]);
}

// Frontier node v: {s0, s1, s2, s3} and {v_lo, v_hi, t, 0}.  With d == f the
// node's value word holds the final share at point v.
struct FrontierArgs {
  Prg4 prg;
  const uint8_t* key;
  uint4* nodes;
  int f;
  int d;
};

__global__ void __launch_bounds__(kDcfBlock) trunc_frontier_kernel(FrontierArgs a) {
  SUFHIP_DCF_LDS_SETUP(a.prg);
  const uint32_t v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v >= (1u << a.d) || !(a.key[7] & 1)) return;
  const uint32_t party = a.key[6] & 1u;
  const uint8_t* chunk = a.key + kHdrBytes + 8;
  const uint64_t x = uint64_t(v) << (a.f - a.d);
  Add64State st = add64_root(chunk, party);
  add64_walk(aes, rkl, chunk, a.f, 0, a.d, x, party, st);
  if (a.d == a.f) {
    const uint64_t out = add64_finish(chunk, a.f, party, st);
    a.nodes[2 * v + 1] = make_uint4(uint32_t(out), uint32_t(out >> 32), 0, 0);
  } else {
    a.nodes[2 * v] = make_uint4(st.s0, st.s1, st.s2, st.s3);
    a.nodes[2 * v + 1] = make_uint4(uint32_t(st.v), uint32_t(st.v >> 32), st.t, 0);
  }
}

// One breadth-first level: nodes at depth `level` (in) -> depth level + 1
// (out), one child per lane.  When level + 1 == f the children are final
// shares.
struct ExpandArgs {
  Prg4 prg;
  const uint8_t* key;
  const uint4* in;
  uint4* out;
  int f;
  int level;
};

__global__ void __launch_bounds__(kDcfBlock) trunc_expand_kernel(ExpandArgs a) {
  SUFHIP_DCF_LDS_SETUP(a.prg);
  if (!(a.key[7] & 1)) return;
  const uint32_t party = a.key[6] & 1u;
  const uint8_t* chunk = a.key + kHdrBytes + 8;
  const uint32_t count = 2u << a.level;
  for (uint32_t c = blockIdx.x * blockDim.x + threadIdx.x; c < count;
       c += gridDim.x * blockDim.x) {
    const uint4 s = a.in[2 * (c >> 1)], q = a.in[2 * (c >> 1) + 1];
    Add64State st{s.x, s.y, s.z, s.w, q.z, uint64_t(q.x) | uint64_t(q.y) << 32};
    const uint64_t x = uint64_t(c & 1u) << (a.f - 1 - a.level);
    add64_walk(aes, rkl, chunk, a.f, a.level, a.level + 1, x, party, st);
    if (a.level + 1 == a.f) {
      const uint64_t out = add64_finish(chunk, a.f, party, st);
      a.out[2 * c + 1] = make_uint4(uint32_t(out), uint32_t(out >> 32), 0, 0);
    } else {
      a.out[2 * c] = make_uint4(st.s0, st.s1, st.s2, st.s3);
      a.out[2 * c + 1] = make_uint4(uint32_t(st.v), uint32_t(st.v >> 32), st.t, 0);
    }
  }
}

// One launch evaluates one or both parties: grid.y selects the party slot.
struct TruncEvalArgs {
  Prg4 prg;
  const uint8_t* keys[2];
  const uint64_t* xhat;
  uint64_t* ys[2];
  const uint4* tables[2];
  size_t n;
  int f;
  int d;
};

using Hdr = TruncHdr;

__device__ __forceinline__ Hdr read_hdr(const uint8_t* key) { return read_trunc_hdr(key); }

template <int kKind>
__device__ __forceinline__ uint64_t postproc(const Hdr& h, int f, uint64_t x, uint64_t carry,
                                             uint64_t wrap, uint64_t sign) {
  return trunc_postproc<kKind>(h, f, x, carry, wrap, sign);
}

__device__ __forceinline__ uint64_t carry_from(const Hdr& h, uint64_t a) {
  return trunc_carry_from(h, a);
}

// Every DCF walk the element needs runs here (frontier continuation, 64-bit
// wrap / sign keys).
template <int kKind>
__global__ void __launch_bounds__(kDcfBlock) trunc_eval_aes_kernel(TruncEvalArgs a) {
  SUFHIP_DCF_LDS_SETUP(a.prg);
  const uint8_t* key = a.keys[blockIdx.y];
  const uint4* nodes = a.tables[blockIdx.y];
  uint64_t* y = a.ys[blockIdx.y];
  const Hdr h = read_hdr(key);
  const uint8_t* carry_chunk = key + kHdrBytes + 8;
  const uint8_t* wrap_chunk = key + kHdrBytes + pad8(h.ckb) + 8;
  const uint8_t* sign_chunk = wrap_chunk + pad8(h.ukb);
  const uint64_t low = (uint64_t(1) << a.f) - 1;
  const size_t stride = size_t(gridDim.x) * kDcfBlock;
  for (size_t e = size_t(blockIdx.x) * kDcfBlock + threadIdx.x; e < a.n; e += stride) {
    const uint64_t x = a.xhat[e];
    uint64_t carry = 0, wrap = 0, sign = 0;
    if (h.flags & 1) {
      const uint64_t xl = x & low;
      uint64_t share;
      if (a.d == a.f) {
        const uint4 q = nodes[2 * xl + 1];
        share = uint64_t(q.x) | uint64_t(q.y) << 32;
      } else {
        Add64State st;
        if (a.d > 0) {
          const size_t v = size_t(xl >> (a.f - a.d));
          const uint4 s = nodes[2 * v], q = nodes[2 * v + 1];
          st = Add64State{s.x, s.y, s.z, s.w, q.z, uint64_t(q.x) | uint64_t(q.y) << 32};
        } else {
          st = add64_root(carry_chunk, h.party);
        }
        add64_walk(aes, rkl, carry_chunk, a.f, a.d, a.f, xl, h.party, st);
        share = add64_finish(carry_chunk, a.f, h.party, st);
      }
      carry = carry_from(h, share);
    }
    if constexpr (kKind != SUFHIP_TRUNC_GAPARS) {
      Add64State st = add64_root(wrap_chunk, h.party);
      add64_walk(aes, rkl, wrap_chunk, 64, 0, 64, x, h.party, st);
      wrap = add64_finish(wrap_chunk, 64, h.party, st);
    }
    if constexpr (kKind == SUFHIP_TRUNC_ARS) {
      Add64State st = add64_root(sign_chunk, h.party);
      add64_walk(aes, rkl, sign_chunk, 64, 0, 64, x, h.party, st);
      sign = (wrap - add64_finish(sign_chunk, 64, h.party, st)) + h.sw;
    }
    y[e] = postproc<kKind>(h, a.f, x, carry, wrap, sign);
  }
}

// GapARS with the full-domain table (or no carry key): one table read per
// element, HBM-bound.
__global__ void __launch_bounds__(256) trunc_eval_table_kernel(TruncEvalArgs a) {
  const uint8_t* key = a.keys[blockIdx.y];
  const uint4* nodes = a.tables[blockIdx.y];
  uint64_t* y = a.ys[blockIdx.y];
  const Hdr h = read_hdr(key);
  const uint64_t low = (uint64_t(1) << a.f) - 1;
  const size_t stride = size_t(gridDim.x) * 256;
  for (size_t e = size_t(blockIdx.x) * 256 + threadIdx.x; e < a.n; e += stride) {
    const uint64_t x = a.xhat[e];
    uint64_t carry = 0;
    if (h.flags & 1) {
      const uint4 q = nodes[2 * (x & low) + 1];
      carry = carry_from(h, uint64_t(q.x) | uint64_t(q.y) << 32);
    }
    y[e] = postproc<SUFHIP_TRUNC_GAPARS>(h, a.f, x, carry, 0, 0);
  }
}

// Key-only halves of several gates at once: the walk to depth min(d, 12) of
// up to kWalkJobs jobs in one launch (walk_device.hpp), then per level one
// launch expanding up to kBatchJobs jobs that go deeper.  Both argument
// blocks stay under 4 KB.
constexpr int kWalkJobs = 96;
constexpr int kBatchJobs = 32;
// Up to 1024 lanes per workgroup: the walk's 8 lanes per node and one
// workgroup per CU (128 KB of AES tables) must cover a batch in one round.
constexpr int kWalkBlock = 1024;

using WalkArgs = WalkJobs<kWalkJobs>;

struct BatchLevelArgs {
  Prg4 prg;
  int count;
  int level;  // the common input depth
  uint32_t begin[kBatchJobs + 1];
  const uint8_t* key[kBatchJobs];
  const uint4* in[kBatchJobs];
  uint4* out[kBatchJobs];
  int f[kBatchJobs];
};

static_assert(sizeof(WalkArgs) <= 4096 && sizeof(BatchLevelArgs) <= 4096,
              "kernel argument blocks must fit in 4 KB");

__global__ void __launch_bounds__(kWalkBlock) trunc_batch_walk_kernel(WalkArgs a) {
  SUFHIP_DCF_LDS_SETUP(a.prg);
  const uint32_t gl = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t g = gl >> 3;  // walk; whole 8-lane groups leave together
  if (g >= a.begin[a.count]) return;
  const int j = batch_job<kWalkJobs>(a.begin, a.count, g);
  const uint8_t* key = a.key[j];
  const uint32_t v = g - a.begin[j];
  if (!(key[7] & 1)) return;
  const uint32_t geo = a.geo[j];
  const int f = int(geo & 0xff), d = int((geo >> 8) & 0xff), e = int(geo >> 16);
  const uint8_t* chunk = key + kHdrBytes + 8;
  // The body stays in the kernel: passed through a helper function, the same
  // steps spill at the 1024-lane register limit.
  const Walk8Ctx<DcfAes> c{aes, rkl, chunk, a.out[j], f, uint32_t(key[6] & 1u),
                           (gl >> 2) & 1u, gl & 3u};
  const int dw = d - e;  // depth walked before the local expansion
  const uint64_t x = uint64_t(v) << (f - dw);
  Walk8 w;
  w.s = word_at(chunk, int(c.q));
  if (c.q == 3) w.s &= 0x7fffffffu;
  w.t = c.party;
  w.v = 0;
  const uint8_t* cw = chunk + 16;
  for (int i = 0; i < dw; ++i, cw += 33) {
    Walk8 n[1];
    walk8_step_n<1>(c, cw, uint32_t(x >> (f - 1 - i)) & 1u, &w, n);
    w = n[0];
  }
  if (e > 0) {
    const Walk8 root[1] = {w};
    if (e == 1)
      walk8_expand<0, 1>(c, cw, root, v);
    else if (e == 2)
      walk8_expand<0, 2>(c, cw, root, v);
    else if (e == 3)
      walk8_expand<0, 3>(c, cw, root, v);
    else  // e == 4: the host picks e <= kWalkLocal <= 4 (static_assert above)
      walk8_expand<0, 4>(c, cw, root, v);
  } else if (d == f) {
    walk8_leaf(c, w, v);
  } else {
    // Frontier node for the expansion launches: {s0..s3}, {v_lo, v_hi, t, 0}.
    const uint4 sn = make_uint4(quad_bcast<0>(w.s), quad_bcast<1>(w.s), quad_bcast<2>(w.s),
                                quad_bcast<3>(w.s));
    if (c.h == 1 && c.q == 0) {
      c.nodes[2 * v] = sn;
      c.nodes[2 * v + 1] = make_uint4(uint32_t(w.v), uint32_t(w.v >> 32), w.t, 0);
    }
  }
}

__global__ void __launch_bounds__(kDcfBlock) trunc_batch_expand_kernel(BatchLevelArgs a) {
  SUFHIP_DCF_LDS_SETUP(a.prg);
  const uint32_t total = a.begin[a.count];
  for (uint32_t g = blockIdx.x * blockDim.x + threadIdx.x; g < total;
       g += gridDim.x * blockDim.x) {
    const int j = batch_job<kBatchJobs>(a.begin, a.count, g);
    const uint8_t* key = a.key[j];
    if (!(key[7] & 1)) continue;
    const uint32_t party = key[6] & 1u;
    const uint8_t* chunk = key + kHdrBytes + 8;
    const int f = a.f[j], level = a.level;
    const uint32_t c = g - a.begin[j];
    const uint4 s = a.in[j][2 * (c >> 1)], q = a.in[j][2 * (c >> 1) + 1];
    Add64State st{s.x, s.y, s.z, s.w, q.z, uint64_t(q.x) | uint64_t(q.y) << 32};
    const uint64_t x = uint64_t(c & 1u) << (f - 1 - level);
    add64_walk(aes, rkl, chunk, f, level, level + 1, x, party, st);
    if (level + 1 == f) {
      const uint64_t out = add64_finish(chunk, f, party, st);
      a.out[j][2 * c + 1] = make_uint4(uint32_t(out), uint32_t(out >> 32), 0, 0);
    } else {
      a.out[j][2 * c] = make_uint4(st.s0, st.s1, st.s2, st.s3);
      a.out[j][2 * c + 1] = make_uint4(uint32_t(st.v), uint32_t(st.v >> 32), st.t, 0);
    }
  }
}

int cu_count(int* cus) {
  int dev = 0;
  SUFHIP_CHECK(hipGetDevice(&dev), "hipGetDevice");
  SUFHIP_CHECK(hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev),
               "hipDeviceGetAttribute(CU count)");
  return SUFHIP_OK;
}

// Launch shape for the frontier kernels: spread `count` lanes over all CUs
// (one workgroup per CU, the AES tables fill its LDS), 256..512 lanes each.
int spread_grid(size_t count, unsigned int* grid, unsigned int* block) {
  int cus = 0;
  if (int rc = cu_count(&cus)) return rc;
  // At least 256 lanes per workgroup: every lane helps fill the LDS tables,
  // which dominates small launches.
  size_t per = (count + size_t(cus) - 1) / size_t(cus);
  per = (per + 63) / 64 * 64;
  const size_t b = per < 256 ? 256 : (per > size_t(kDcfBlock) ? size_t(kDcfBlock) : per);
  const size_t g = (count + b - 1) / b;
  *block = unsigned(b);
  *grid = unsigned(g < size_t(cus) ? g : size_t(cus));
  return SUFHIP_OK;
}

// Launch shape for the batched walk (8 lanes per walk, no grid stride): the
// lanes spread over every CU, 128..kWalkBlock per workgroup.
int walk_grid(size_t count, unsigned int* grid, unsigned int* block) {
  int cus = 0;
  if (int rc = cu_count(&cus)) return rc;
  size_t per = (count + size_t(cus) - 1) / size_t(cus);
  per = (per + 63) / 64 * 64;
  const size_t b = per < 128 ? 128 : (per > size_t(kWalkBlock) ? size_t(kWalkBlock) : per);
  *block = unsigned(b);
  *grid = unsigned((count + b - 1) / b);
  return SUFHIP_OK;
}

bool valid_kind(int kind) {
  return kind == SUFHIP_TRUNC_TR || kind == SUFHIP_TRUNC_ARS || kind == SUFHIP_TRUNC_GAPARS;
}

constexpr size_t kMaxElems = size_t(1) << 38;

// Finish for `parties` (1 or 2) key slots: the table kernel for GapARS with
// a full-domain table, else the DCF-walk kernel.
int launch_finish(int kind, const TruncEvalArgs& a, int parties, hipStream_t s) {
  if (kind == SUFHIP_TRUNC_GAPARS && a.d == a.f) {
    size_t blocks = (a.n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(trunc_eval_table_kernel, dim3(unsigned(blocks), parties), dim3(256), 0, s,
                       a);
    return check_launch("trunc_eval_table_kernel");
  }
  unsigned int g = 0;
  if (int rc = dcf_grid(a.n, &g)) return rc;
  const dim3 grid(g, parties);
  if (kind == SUFHIP_TRUNC_GAPARS)
    hipLaunchKernelGGL(trunc_eval_aes_kernel<SUFHIP_TRUNC_GAPARS>, grid, dim3(kDcfBlock), 0, s,
                       a);
  else if (kind == SUFHIP_TRUNC_TR)
    hipLaunchKernelGGL(trunc_eval_aes_kernel<SUFHIP_TRUNC_TR>, grid, dim3(kDcfBlock), 0, s, a);
  else
    hipLaunchKernelGGL(trunc_eval_aes_kernel<SUFHIP_TRUNC_ARS>, grid, dim3(kDcfBlock), 0, s, a);
  return check_launch("trunc_eval_aes_kernel");
}

// Shared argument checks of the evaluation entry points.
int trunc_check(const char* fn, int kind, int frac_bits, const uint8_t* prg_state,
                const uint8_t* d_key, size_t key_bytes, size_t n, const void* d_work,
                size_t work_bytes) {
  SUFHIP_REQUIRE(valid_kind(kind), std::string(fn) + ": unknown kind");
  SUFHIP_REQUIRE(frac_bits >= 1 && frac_bits <= 62, std::string(fn) + ": frac_bits out of [1, 62]");
  SUFHIP_REQUIRE(key_bytes == sufhip_trunc_key_bytes(kind, frac_bits),
                 std::string(fn) + ": key_bytes does not match (kind, frac_bits)");
  SUFHIP_REQUIRE(n < kMaxElems, std::string(fn) + ": n too large");
  SUFHIP_REQUIRE(prg_state && d_key, std::string(fn) + ": null pointer");
  SUFHIP_REQUIRE((reinterpret_cast<uintptr_t>(d_key) & 7) == 0,
                 std::string(fn) + ": key must be 8-byte aligned");
  const size_t need = sufhip_trunc_work_bytes(frac_bits, n);
  SUFHIP_REQUIRE(work_bytes >= need && (need == 0 || d_work),
                 std::string(fn) + ": workspace smaller than sufhip_trunc_work_bytes()");
  SUFHIP_REQUIRE(need == 0 || (reinterpret_cast<uintptr_t>(d_work) & 15) == 0,
                 std::string(fn) + ": workspace must be 16-byte aligned");
  return SUFHIP_OK;
}

// The walk launch of m <= kWalkJobs prepare jobs: per job its depth d, walked
// depth k0 and the two workspace regions, alternated so that depth d ends in
// the first (as sufhip_trunc_prepare), and the local levels el of the
// full-domain walks.
struct WalkPlan {
  int d[kWalkJobs], k0s[kWalkJobs], cur[kWalkJobs];
  uint4* lvl[kWalkJobs][2];
  int maxd, el;
};

int plan_walk(const uint8_t* prg_state, const sufhip_trunc_job* jobs, int m, const char* what,
              WalkPlan& p, size_t lanes_cap = 0) {
  p.maxd = 0;
  for (int i = 0; i < m; ++i) {
    const sufhip_trunc_job& jb = jobs[i];
    if (int rc = trunc_check(what, jb.kind, jb.frac_bits, prg_state, jb.d_key, jb.key_bytes,
                             jb.n, jb.d_work, jb.work_bytes))
      return rc;
    p.d[i] = frontier_bits(jb.frac_bits, jb.n);
    p.k0s[i] = batch_walk_bits(p.d[i], jb.frac_bits);
    p.lvl[i][0] = static_cast<uint4*>(jb.d_work);
    p.lvl[i][1] = p.d[i] > 0 ? p.lvl[i][0] + 2 * (size_t(1) << p.d[i]) : nullptr;
    p.cur[i] = (p.d[i] - p.k0s[i]) & 1;
    if (p.d[i] > p.maxd) p.maxd = p.d[i];
  }
  // Local levels of the full-domain walks: a walk level costs about as
  // much as one lockstep group of the expansion, so the walks go as deep as
  // the lanes allow -- the fewest local levels whose walks take less than
  // three quarters of one full workgroup per CU (at most kWalkLocal; past
  // that the extra waves per SIMD slow every level more than a local level
  // costs).  A hosted walk (lanes_cap > 0) takes the fewest whose walks fit
  // in the host's room.
  int cus = 0;
  if (int rc = cu_count(&cus)) return rc;
  const size_t cap = lanes_cap > 0 ? lanes_cap + 1 : 3 * size_t(cus) * kWalkBlock / 4;
  p.el = 0;
  for (; p.el < kWalkLocal; ++p.el) {
    size_t lanes = 0;
    for (int i = 0; i < m; ++i) {
      const int k0 = p.k0s[i];
      const int e = k0 == jobs[i].frac_bits && k0 >= p.el ? p.el : 0;
      lanes += p.d[i] > 0 ? 8 * (size_t(1) << (k0 - e)) : 0;
    }
    if (lanes < cap) break;
  }
  return SUFHIP_OK;
}

// WalkJobs' fields for the plan: walks per job, keys, outputs, geometry.
void fill_walk(const WalkPlan& p, const sufhip_trunc_job* jobs, int m, uint32_t* begin,
               const uint8_t** key, uint4** out, uint32_t* geo) {
  begin[0] = 0;
  for (int i = 0; i < m; ++i) {
    const sufhip_trunc_job& jb = jobs[i];
    const int k0 = p.k0s[i];
    const int e = k0 == jb.frac_bits && k0 >= p.el ? p.el : 0;
    key[i] = jb.d_key;
    out[i] = p.lvl[i][p.cur[i]];
    geo[i] = uint32_t(jb.frac_bits) | uint32_t(k0) << 8 | uint32_t(e) << 16;
    begin[i + 1] = begin[i] + (p.d[i] > 0 ? (1u << (k0 - e)) : 0u);
  }
}

}  // namespace

int trunc_walk_plan(const uint8_t* prg_state, const sufhip_trunc_job* jobs, int count,
                    int max_jobs, uint32_t* begin, const uint8_t** key, uint4** out,
                    uint32_t* geo, bool* one) {
  *one = false;
  SUFHIP_REQUIRE(count >= 0 && (count == 0 || jobs), "sufhip_kb_open_split_prepare: bad jobs");
  SUFHIP_REQUIRE(prg_state, "sufhip_kb_open_split_prepare: null prg_state");
  if (count > max_jobs || count > kWalkJobs) return SUFHIP_OK;
  WalkPlan p;
  if (int rc = plan_walk(prg_state, jobs, count, "sufhip_kb_open_split_prepare", p)) return rc;
  // Table gates only (every walk ends in a table entry), no local levels and
  // no expansion launches.
  bool ok = p.el == 0;
  for (int i = 0; i < count; ++i)
    ok = ok && (p.d[i] == 0 || (p.k0s[i] == p.d[i] && p.d[i] == jobs[i].frac_bits));
  if (!ok) return SUFHIP_OK;
  fill_walk(p, jobs, count, begin, key, out, geo);
  *one = true;
  return SUFHIP_OK;
}

int trunc_walk_plan_fit(const uint8_t* prg_state, const sufhip_trunc_job* jobs, int count,
                        int max_jobs, size_t lanes_cap, uint32_t* begin, const uint8_t** key,
                        uint4** out, uint32_t* geo, bool* one, const char* what) {
  *one = false;
  SUFHIP_REQUIRE(count >= 0 && (count == 0 || jobs), "trunc walk: bad jobs");
  SUFHIP_REQUIRE(prg_state, "trunc walk: null prg_state");
  if (count > max_jobs || count > kWalkJobs) return SUFHIP_OK;
  WalkPlan p;
  if (int rc = plan_walk(prg_state, jobs, count, what, p, lanes_cap > 0 ? lanes_cap : 1))
    return rc;
  // Table gates only: every walk ends in table entries, nothing is left for
  // the expansion launches.
  bool ok = true;
  for (int i = 0; i < count; ++i)
    ok = ok && (p.d[i] == 0 || (p.k0s[i] == p.d[i] && p.d[i] == jobs[i].frac_bits));
  if (!ok) return SUFHIP_OK;
  fill_walk(p, jobs, count, begin, key, out, geo);
  *one = true;
  return SUFHIP_OK;
}

}  // namespace sufhip

using namespace sufhip;

// Workspace of sufhip_trunc_eval_noalloc: a file-scope device array, so that
// the entry point needs no allocation.  Each GPU the library runs on holds its
// own copy for the life of the process.  In host code `scratch` names a host
// stand-in, not device memory: the array's device address on each GPU comes
// from hipGetSymbolAddress (noalloc_scratch below) and only that address is
// passed to kernels.  1 MiB holds the carry frontier of any batch for
// frac_bits <= 14 (the full-domain table, 786,432 bytes at f = 14) and of
// batches below 2^16 points for larger frac_bits.
static constexpr size_t kNoAllocScratchBytes = size_t(1) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

constexpr int kNoAllocMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kNoAllocMaxDevices];

// The current device's address of `scratch`, looked up once per device (with
// that device current) and kept.
int noalloc_scratch(void** out) {
  int dev = 0;
  SUFHIP_CHECK(hipGetDevice(&dev), "hipGetDevice");
  SUFHIP_REQUIRE(dev >= 0 && dev < kNoAllocMaxDevices,
                 "sufhip_trunc_eval_noalloc: device index beyond 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    SUFHIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    SUFHIP_REQUIRE(p != nullptr, "hipGetSymbolAddress(scratch) returned null");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SUFHIP_OK;
}

}  // namespace

extern "C" {

size_t sufhip_trunc_noalloc_max_work_bytes(void) { return kNoAllocScratchBytes; }

int sufhip_trunc_eval_noalloc(int kind, int frac_bits, const uint8_t* prg_state,
                              const uint8_t* d_key, size_t key_bytes, const uint64_t* d_xhat,
                              size_t n, uint64_t* d_y, void* stream) {
  const size_t need = sufhip_trunc_work_bytes(frac_bits, n);
  SUFHIP_REQUIRE(need <= kNoAllocScratchBytes,
                 "sufhip_trunc_eval_noalloc: the carry frontier for this (frac_bits, n) needs " +
                     std::to_string(need) + " bytes, above the " +
                     std::to_string(kNoAllocScratchBytes) +
                     "-byte static workspace (use sufhip_trunc_eval with a workspace)");
  void* work = nullptr;
  if (need > 0) {
    if (int rc = noalloc_scratch(&work)) return rc;
  }
  return sufhip_trunc_eval(kind, frac_bits, prg_state, d_key, key_bytes, d_xhat, n, d_y, work,
                           need > 0 ? kNoAllocScratchBytes : 0, stream);
}

size_t sufhip_trunc_key_bytes(int kind, int frac_bits) {
  if (!valid_kind(kind) || frac_bits < 1 || frac_bits > 62) return 0;
  size_t b = kHdrBytes + pad8(dcf_bytes(frac_bits));
  if (kind != SUFHIP_TRUNC_GAPARS) b += pad8(dcf_bytes(64));
  if (kind == SUFHIP_TRUNC_ARS) b += pad8(dcf_bytes(64));
  return b;
}

int sufhip_trunc_gen(int kind, int frac_bits, const uint8_t* prg_state, const uint64_t* rnd,
                     uint8_t* d_key0, uint8_t* d_key1, void* stream) {
  SUFHIP_REQUIRE(valid_kind(kind), "sufhip_trunc_gen: unknown kind");
  SUFHIP_REQUIRE(frac_bits >= 1 && frac_bits <= 62, "sufhip_trunc_gen: frac_bits out of [1, 62]");
  SUFHIP_REQUIRE(prg_state && rnd && d_key0 && d_key1, "sufhip_trunc_gen: null pointer");
  SUFHIP_REQUIRE((reinterpret_cast<uintptr_t>(d_key0) & 7) == 0 &&
                     (reinterpret_cast<uintptr_t>(d_key1) & 7) == 0,
                 "sufhip_trunc_gen: keys must be 8-byte aligned");
  const int f = frac_bits;
  const uint64_t r = rnd[0];
  const uint64_t r_low = r & ((uint64_t(1) << f) - 1);
  const uint64_t r_hi = r >> f;
  const uint64_t m = (kind == SUFHIP_TRUNC_GAPARS && (r >> 63)) ? uint64_t(1) << (64 - f) : 0;
  const uint64_t sign_w = r < (uint64_t(1) << 63) ? 1 : 0;
  const int has_carry = r_low != 0;
  const int has_wrap = kind != SUFHIP_TRUNC_GAPARS;
  const int has_sign = kind == SUFHIP_TRUNC_ARS;
  const uint32_t ckb = uint32_t(dcf_bytes(f)), ukb = uint32_t(dcf_bytes(64));
  TruncGenArgs a{};
  fill_prg4(prg_state, &a.prg);
  a.key0 = d_key0;
  a.key1 = d_key1;
  a.flags = has_carry | has_wrap << 1 | has_sign << 2;
  for (int p = 0; p < 2; ++p) {
    auto split = [&](uint64_t v, uint64_t s) { return p == 0 ? s : v - s; };
    a.hdr[p][0] = uint64_t(kTag) | uint64_t(kind) << 32 | uint64_t(f) << 40 |
                  uint64_t(p) << 48 | uint64_t(a.flags) << 56;
    a.hdr[p][1] = split(r, rnd[1]);
    a.hdr[p][2] = split(r_hi, rnd[5]);
    a.hdr[p][3] = split(0, rnd[2]);
    a.hdr[p][4] = has_carry ? split(1, rnd[3]) : 0;
    a.hdr[p][5] = has_sign ? split(sign_w, rnd[4]) : 0;
    a.hdr[p][6] = kind == SUFHIP_TRUNC_GAPARS ? split(m, rnd[6]) : 0;
    a.hdr[p][7] = uint64_t(ckb) | uint64_t(ukb) << 32;
  }
  a.alpha[0] = r_low;
  a.alpha[1] = r;
  a.alpha[2] = r + (uint64_t(1) << 63);
  a.bits[0] = f;
  a.bits[1] = 64;
  a.bits[2] = 64;
  a.off[0] = kHdrBytes;
  a.off[1] = uint32_t(kHdrBytes + pad8(ckb));
  a.off[2] = uint32_t(a.off[1] + pad8(ukb));
  for (int j = 0; j < 3; ++j)
    for (int w = 0; w < 4; ++w) a.seeds[j][w] = rnd[7 + 4 * j + w];
  a.total = uint32_t(sufhip_trunc_key_bytes(kind, f));
  hipLaunchKernelGGL(trunc_gen_kernel, dim3(1), dim3(kDcfBlock), 0, as_stream(stream), a);
  return check_launch("trunc_gen_kernel");
}

size_t sufhip_trunc_work_bytes(int frac_bits, size_t n) {
  if (frac_bits < 1 || frac_bits > 62) return 0;
  return frontier_nodes(frontier_bits(frac_bits, n)) * 32;
}

int sufhip_trunc_prepare(int kind, int frac_bits, const uint8_t* prg_state, const uint8_t* d_key,
                         size_t key_bytes, size_t n, void* d_work, size_t work_bytes,
                         void* stream) {
  if (int rc = trunc_check("sufhip_trunc_prepare", kind, frac_bits, prg_state, d_key, key_bytes,
                           n, d_work, work_bytes))
    return rc;
  const int d = frontier_bits(frac_bits, n);
  if (n == 0 || d == 0) return SUFHIP_OK;
  hipStream_t s = as_stream(stream);
  Prg4 prg;
  fill_prg4(prg_state, &prg);
  // Walk to depth k0, then expand level by level, alternating between the
  // two workspace regions so that depth d ends in the first one.
  uint4* lvl[2] = {static_cast<uint4*>(d_work), static_cast<uint4*>(d_work) + 2 * (size_t(1) << d)};
  const int k0 = walk_bits(d);
  int cur = (d - k0) & 1;
  FrontierArgs fa{prg, d_key, lvl[cur], frac_bits, k0};
  unsigned int g = 0, b = 0;
  if (int rc = spread_grid(size_t(1) << k0, &g, &b)) return rc;
  // The walk kernel is one lane per node (no stride loop): cover all nodes.
  g = unsigned(((size_t(1) << k0) + b - 1) / b);
  hipLaunchKernelGGL(trunc_frontier_kernel, dim3(g), dim3(b), 0, s, fa);
  if (int rc = check_launch("trunc_frontier_kernel")) return rc;
  for (int level = k0; level < d; ++level) {
    ExpandArgs ea{prg, d_key, lvl[cur], lvl[cur ^ 1], frac_bits, level};
    unsigned int eg = 0, eb = 0;
    if (int rc = spread_grid(size_t(2) << level, &eg, &eb)) return rc;
    hipLaunchKernelGGL(trunc_expand_kernel, dim3(eg), dim3(eb), 0, s, ea);
    if (int rc = check_launch("trunc_expand_kernel")) return rc;
    cur ^= 1;
  }
  return SUFHIP_OK;
}

int sufhip_trunc_finish(int kind, int frac_bits, const uint8_t* prg_state, const uint8_t* d_key,
                        size_t key_bytes, const uint64_t* d_xhat, size_t n, uint64_t* d_y,
                        const void* d_work, size_t work_bytes, void* stream) {
  if (int rc = trunc_check("sufhip_trunc_finish", kind, frac_bits, prg_state, d_key, key_bytes,
                           n, d_work, work_bytes))
    return rc;
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_xhat && d_y, "sufhip_trunc_finish: null pointer");
  const int d = frontier_bits(frac_bits, n);
  hipStream_t s = as_stream(stream);
  Prg4 prg;
  fill_prg4(prg_state, &prg);
  const uint4* tab = static_cast<const uint4*>(d_work);
  TruncEvalArgs a{prg, {d_key, d_key}, d_xhat, {d_y, d_y}, {tab, tab}, n, frac_bits, d};
  return launch_finish(kind, a, 1, s);
}

int sufhip_trunc_finish2(int kind, int frac_bits, const uint8_t* prg_state, const uint8_t* d_key0,
                         const uint8_t* d_key1, size_t key_bytes, const uint64_t* d_xhat, size_t n,
                         uint64_t* d_y0, uint64_t* d_y1, const void* d_work0,
                         const void* d_work1, size_t work_bytes, void* stream) {
  if (int rc = trunc_check("sufhip_trunc_finish2", kind, frac_bits, prg_state, d_key0, key_bytes,
                           n, d_work0, work_bytes))
    return rc;
  if (int rc = trunc_check("sufhip_trunc_finish2", kind, frac_bits, prg_state, d_key1, key_bytes,
                           n, d_work1, work_bytes))
    return rc;
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_xhat && d_y0 && d_y1, "sufhip_trunc_finish2: null pointer");
  Prg4 prg;
  fill_prg4(prg_state, &prg);
  TruncEvalArgs a{prg,
                  {d_key0, d_key1},
                  d_xhat,
                  {d_y0, d_y1},
                  {static_cast<const uint4*>(d_work0), static_cast<const uint4*>(d_work1)},
                  n,
                  frac_bits,
                  frontier_bits(frac_bits, n)};
  return launch_finish(kind, a, 2, as_stream(stream));
}

int sufhip_trunc_prepare_batch(const uint8_t* prg_state, const sufhip_trunc_job* jobs, int count,
                               void* stream) {
  SUFHIP_REQUIRE(count >= 0 && (count == 0 || jobs), "sufhip_trunc_prepare_batch: bad jobs");
  SUFHIP_REQUIRE(prg_state, "sufhip_trunc_prepare_batch: null prg_state");
  hipStream_t s = as_stream(stream);
  Prg4 prg;
  fill_prg4(prg_state, &prg);
  for (int base = 0; base < count; base += kWalkJobs) {
    const int m = count - base < kWalkJobs ? count - base : kWalkJobs;
    WalkPlan p;
    if (int rc = plan_walk(prg_state, jobs + base, m, "sufhip_trunc_prepare_batch", p)) return rc;
    int(&d)[kWalkJobs] = p.d;
    int(&k0s)[kWalkJobs] = p.k0s;
    int(&cur)[kWalkJobs] = p.cur;
    uint4*(&lvl)[kWalkJobs][2] = p.lvl;
    const int maxd = p.maxd;
    WalkArgs wa{};
    wa.prg = prg;
    fill_walk(p, jobs + base, m, wa.begin, wa.key, wa.out, wa.geo);
    wa.count = m;
    if (wa.begin[m] > 0) {
      unsigned int g = 0, b = 0;
      if (int rc = walk_grid(8 * size_t(wa.begin[m]), &g, &b)) return rc;
      hipLaunchKernelGGL(trunc_batch_walk_kernel, dim3(g), dim3(b), 0, s, wa);
      if (int rc = check_launch("trunc_batch_walk_kernel")) return rc;
    }
    for (int level = kWalkFrontierBits; level < maxd; ++level) {
      // Jobs still expanding at this level, kBatchJobs per launch.
      int deep[kWalkJobs], nd = 0;
      for (int i = 0; i < m; ++i)
        if (d[i] > level && k0s[i] <= level) deep[nd++] = i;
      for (int q0 = 0; q0 < nd; q0 += kBatchJobs) {
        BatchLevelArgs ea{};
        ea.prg = prg;
        ea.level = level;
        ea.begin[0] = 0;
        for (int q = q0; q < nd && q < q0 + kBatchJobs; ++q) {
          const int i = deep[q];
          ea.key[ea.count] = jobs[base + i].d_key;
          ea.in[ea.count] = lvl[i][cur[i]];
          ea.out[ea.count] = lvl[i][cur[i] ^ 1];
          ea.f[ea.count] = jobs[base + i].frac_bits;
          ea.begin[ea.count + 1] = ea.begin[ea.count] + (2u << level);
          ++ea.count;
          cur[i] ^= 1;
        }
        unsigned int eg = 0, eb = 0;
        if (int rc = spread_grid(ea.begin[ea.count], &eg, &eb)) return rc;
        hipLaunchKernelGGL(trunc_batch_expand_kernel, dim3(eg), dim3(eb), 0, s, ea);
        if (int rc = check_launch("trunc_batch_expand_kernel")) return rc;
      }
    }
  }
  return SUFHIP_OK;
}

int sufhip_trunc_eval(int kind, int frac_bits, const uint8_t* prg_state, const uint8_t* d_key,
                      size_t key_bytes, const uint64_t* d_xhat, size_t n, uint64_t* d_y,
                      void* d_work, size_t work_bytes, void* stream) {
  if (int rc = trunc_check("sufhip_trunc_eval", kind, frac_bits, prg_state, d_key, key_bytes, n,
                           d_work, work_bytes))
    return rc;
  if (n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_xhat && d_y, "sufhip_trunc_eval: null pointer");
  if (int rc = sufhip_trunc_prepare(kind, frac_bits, prg_state, d_key, key_bytes, n, d_work,
                                    work_bytes, stream))
    return rc;
  return sufhip_trunc_finish(kind, frac_bits, prg_state, d_key, key_bytes, d_xhat, n, d_y, d_work,
                             work_bytes, stream);
}

}  // extern "C"
