// Composite gates with boolean outputs (SUF l_out > 0), both parties on one
// GPU, and the bucket staging of the masked inputs that precedes them.
//
// Boolean network: composite_eval_batch_backend's path for ell > 0
// (include/gates/composite_fss.hpp:2132-2456).  The PFSS evaluation gives
// XOR-shared bits: predicate query q at element i, pred[q][i], and the
// piece cuts, cut[k][i] = 1[xhat_i < cut_k] over the x^-domain segments of
// the gate (the x pieces rotated by r_in, split at the wrap, sorted).  Then
//   * b2a of each cut bit (one Beaver product of the parties' bits,
//     a + b - 2ab; gates::b2a_bit, include/gates/bool_dag_xor.hpp:120-127);
//   * one-hot selectors sel_0 = cut_0, sel_k = (1 - cut_{k-1}) cut_k,
//     sel_C = 1 - cut_{C-1} (selectors_from_cutbits_block,
//     composite_fss.hpp:893-974);
//   * each segment's boolean outputs: the rewritten BoolExpr of the piece
//     the segment comes from, over XOR-shared bits (eval_bool_xor_view,
//     bool_dag_xor.hpp:13-104): NOT flips party 0's share, XOR is local, AND
//     and OR = x ^ y ^ (x AND y) take one bit triple each, a wrap variable is
//     the low bit of its additive share;
//   * b2a of each output bit and out_j = sum_s sel_s * bool_{s,j} (one
//     Beaver product each).
// With both parties in one process every open is a sum of the two parties'
// masked values, computed in the lane that needs it: one launch runs the
// whole network for both parties.  Segment s's bit b2a and selector
// products may run in any order because every product has its own triple.
//
// Staging: PfssSuperBatch::flush_eval concatenates a bucket's jobs' x^ into
// one device buffer, unpacking eff_bits-packed uploads
// (src/runtime/pfss_superbatch.cpp:740-930); sufhip_stage_hatx does all of a
// bucket's segments in one launch.
#include <hip/hip_runtime.h>

#include <string>

#include "suf_hip.h"
#include "sufhip_internal.hpp"

namespace sufhip {
namespace {

struct StageArgs {
  sufhip_stage_seg seg[SUFHIP_STAGE_MAX_SEGS];
  uint64_t* bucket;
};

__global__ void __launch_bounds__(256) stage_hatx_kernel(StageArgs a) {
  const sufhip_stage_seg s = a.seg[blockIdx.y];
  uint64_t* dst = a.bucket + s.dst;
  const size_t stride = size_t(gridDim.x) * 256;
  if (s.eff_bits >= 64) {
    const uint64_t* src = static_cast<const uint64_t*>(s.src);
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < s.len; i += stride) dst[i] = src[i];
    return;
  }
  // LSB-first bitstream of eff_bits-wide values in u64 words
  // (pack_eff_bits_host / launch_unpack_eff_bits_kernel layout).
  const uint64_t* w = static_cast<const uint64_t*>(s.src);
  const int eb = s.eff_bits;
  const uint64_t m = (uint64_t(1) << eb) - 1;
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < s.len; i += stride) {
    const size_t bit = i * size_t(eb);
    const size_t q = bit >> 6;
    const int off = int(bit & 63);
    uint64_t v = w[q] >> off;
    if (off + eb > 64) v |= w[q + 1] << (64 - off);  // the value's high bits are in word q + 1
    dst[i] = v & m;
  }
}

// One Beaver product for both parties: shares x, y; triple (a, b, c) of
// step t at element i.
struct Tri2 {
  const uint64_t* p[2];
  size_t n;
  __device__ __forceinline__ void mul(size_t t, size_t i, const uint64_t (&x)[2],
                                      const uint64_t (&y)[2], uint64_t (&z)[2]) const {
    const size_t base = 3 * t * n + i;
    const uint64_t a0 = p[0][base], b0 = p[0][base + n], c0 = p[0][base + 2 * n];
    const uint64_t a1 = p[1][base], b1 = p[1][base + n], c1 = p[1][base + 2 * n];
    const uint64_t d = (x[0] - a0) + (x[1] - a1);
    const uint64_t e = (y[0] - b0) + (y[1] - b1);
    z[0] = c0 + d * b0 + e * a0 + d * e;
    z[1] = c1 + d * b1 + e * a1;
  }
  // XOR-shared bit (bx0, bx1) -> additive shares of the same bit.
  __device__ __forceinline__ void b2a(size_t t, size_t i, uint32_t bx0, uint32_t bx1,
                                      uint64_t (&out)[2]) const {
    const uint64_t x[2] = {bx0, 0}, y[2] = {0, bx1};
    uint64_t z[2];
    mul(t, i, x, y, z);
    out[0] = uint64_t(bx0) - 2 * z[0];
    out[1] = uint64_t(bx1) - 2 * z[1];
  }
};

struct BoolArgs {
  sufhip_composite_bool_args g;
};

// A stack entry is a bit pair: party 0's XOR share in bit 0, party 1's in
// bit 1; the stack is 16 such pairs in one word (the top in bits 0-1).
__device__ __forceinline__ uint32_t eval_program(const sufhip_composite_bool_args& g, int begin,
                                                 int end, size_t i, size_t& and_idx) {
  uint32_t stk = 0;
  for (int pc = begin; pc < end; ++pc) {
    const int32_t ins = g.prog[pc];
    const int op = ins & 0xf;
    const int arg = ins >> 4;
    if (op == SUFHIP_BOOL_VAR) {
      const uint32_t b0 = g.pred[0][size_t(arg) * g.n + i] & 1u;
      const uint32_t b1 = g.pred[1][size_t(arg) * g.n + i] & 1u;
      stk = (stk << 2) | b0 | b1 << 1;
    } else if (op == SUFHIP_BOOL_WRAP) {
      const uint32_t b0 = uint32_t(g.wrap[0][arg]) & 1u;  // low bit of the additive share
      const uint32_t b1 = uint32_t(g.wrap[1][arg]) & 1u;
      stk = (stk << 2) | b0 | b1 << 1;
    } else if (op == SUFHIP_BOOL_CONST) {
      stk = (stk << 2) | uint32_t(arg & 1);  // party 0 holds the constant
    } else if (op == SUFHIP_BOOL_NOT) {
      stk ^= 1u;
    } else {
      const uint32_t y = stk & 3u, x = (stk >> 2) & 3u;
      stk >>= 4;
      uint32_t r = x ^ y;
      if (op == SUFHIP_BOOL_AND || op == SUFHIP_BOOL_OR) {
        const uint8_t t0 = g.bit_tri[0][and_idx * g.n + i], t1 = g.bit_tri[1][and_idx * g.n + i];
        ++and_idx;
        // e = x ^ a, f = y ^ b opened; z_p = c_p ^ (e & b_p) ^ (f & a_p) ^ [p0](e & f).
        const uint32_t a0 = t0 & 1u, b0 = (t0 >> 1) & 1u, c0 = (t0 >> 2) & 1u;
        const uint32_t a1 = t1 & 1u, b1 = (t1 >> 1) & 1u, c1 = (t1 >> 2) & 1u;
        const uint32_t e = (x ^ (x >> 1) ^ a0 ^ a1) & 1u;
        const uint32_t f = (y ^ (y >> 1) ^ b0 ^ b1) & 1u;
        const uint32_t z0 = c0 ^ (e & b0) ^ (f & a0) ^ (e & f);
        const uint32_t z1 = c1 ^ (e & b1) ^ (f & a1);
        const uint32_t z = z0 | z1 << 1;
        r = op == SUFHIP_BOOL_AND ? z : (r ^ z);
      }
      stk = (stk << 2) | r;
    }
  }
  return stk & 3u;
}

// kEll: the number of boolean outputs (a template parameter, so that the
// accumulators stay in registers).
template <int kEll>
__global__ void __launch_bounds__(256) composite_bool2_kernel(BoolArgs A) {
  const sufhip_composite_bool_args& g = A.g;
  const Tri2 tri{{g.tri[0], g.tri[1]}, g.n};
  const int C = g.cuts, S = C + 1, ell = kEll;
  const size_t t_bits = size_t(C > 0 ? 2 * C - 1 : 0);  // first triple of the bits' b2a
  const size_t t_sel = t_bits + size_t(S) * size_t(ell);  // first selector product
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < g.n;
       i += size_t(gridDim.x) * 256) {
    uint64_t acc[kEll][2];
#pragma unroll
    for (int j = 0; j < kEll; ++j) acc[j][0] = acc[j][1] = 0;
    uint64_t prev[2] = {0, 0};  // additive cut_{s-1}
    size_t and_idx = 0;
    for (int s = 0; s < S; ++s) {
      uint64_t sel[2];
      uint64_t cur[2] = {0, 0};
      if (s < C) {
        const uint32_t c0 = g.cut[0][size_t(s) * g.n + i] & 1u;
        const uint32_t c1 = g.cut[1][size_t(s) * g.n + i] & 1u;
        tri.b2a(size_t(s), i, c0, c1, cur);
      }
      if (C == 0) {
        sel[0] = 1;
        sel[1] = 0;
      } else if (s == 0) {
        sel[0] = cur[0];
        sel[1] = cur[1];
      } else if (s == C) {
        sel[0] = 1 - prev[0];
        sel[1] = uint64_t(0) - prev[1];
      } else {
        const uint64_t np[2] = {1 - prev[0], uint64_t(0) - prev[1]};
        tri.mul(size_t(C) + size_t(s - 1), i, np, cur, sel);
      }
      prev[0] = cur[0];
      prev[1] = cur[1];
#pragma unroll
      for (int j = 0; j < kEll; ++j) {
        const int k = s * ell + j;
        const uint32_t bx = eval_program(g, g.prog_off[k], g.prog_off[k + 1], i, and_idx);
        uint64_t badd[2], z[2];
        tri.b2a(t_bits + size_t(k), i, bx & 1u, bx >> 1, badd);
        tri.mul(t_sel + size_t(k), i, sel, badd, z);
        acc[j][0] += z[0];
        acc[j][1] += z[1];
      }
    }
#pragma unroll
    for (int j = 0; j < kEll; ++j) {
      g.out[0][i * size_t(ell) + j] = acc[j][0];
      g.out[1][i * size_t(ell) + j] = acc[j][1];
    }
  }
}

// Host check of a boolean program: known opcodes, operands in range, the
// stack within SUFHIP_BOOL_MAX_STACK and one value left; counts AND/OR.
bool program_ok(const int32_t* prog, int begin, int end, int queries, int wraps, int* ands) {
  int depth = 0;
  for (int pc = begin; pc < end; ++pc) {
    const int op = prog[pc] & 0xf, arg = prog[pc] >> 4;
    switch (op) {
      case SUFHIP_BOOL_VAR:
        if (arg < 0 || arg >= queries) return false;
        ++depth;
        break;
      case SUFHIP_BOOL_WRAP:
        if (arg < 0 || arg >= wraps) return false;
        ++depth;
        break;
      case SUFHIP_BOOL_CONST:
        if (arg != 0 && arg != 1) return false;
        ++depth;
        break;
      case SUFHIP_BOOL_NOT:
        if (depth < 1) return false;
        break;
      case SUFHIP_BOOL_XOR:
      case SUFHIP_BOOL_AND:
      case SUFHIP_BOOL_OR:
        if (depth < 2) return false;
        --depth;
        if (op != SUFHIP_BOOL_XOR) ++*ands;
        break;
      default:
        return false;
    }
    if (depth > SUFHIP_BOOL_MAX_STACK) return false;
  }
  return depth == 1;
}

}  // namespace
}  // namespace sufhip

using namespace sufhip;

extern "C" {

int sufhip_stage_hatx(const sufhip_stage_seg* segs, int count, uint64_t* d_bucket,
                      size_t bucket_len, void* stream) {
  SUFHIP_REQUIRE(count >= 0 && count <= SUFHIP_STAGE_MAX_SEGS && (count == 0 || segs),
                 "sufhip_stage_hatx: 0..SUFHIP_STAGE_MAX_SEGS segments");
  if (count == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(d_bucket != nullptr, "sufhip_stage_hatx: null bucket");
  StageArgs a{};
  a.bucket = d_bucket;
  size_t longest = 0;
  for (int k = 0; k < count; ++k) {
    const sufhip_stage_seg& s = segs[k];
    SUFHIP_REQUIRE(s.eff_bits >= 1 && s.eff_bits <= 64, "sufhip_stage_hatx: eff_bits in [1, 64]");
    SUFHIP_REQUIRE(s.len == 0 || s.src, "sufhip_stage_hatx: null source");
    SUFHIP_REQUIRE(s.dst <= bucket_len && s.len <= bucket_len - s.dst,
                   "sufhip_stage_hatx: segment " + std::to_string(k) + " ends past the bucket");
    for (int q = 0; q < k; ++q) {
      const sufhip_stage_seg& o = segs[q];
      SUFHIP_REQUIRE(s.len == 0 || o.len == 0 || s.dst + s.len <= o.dst || o.dst + o.len <= s.dst,
                     "sufhip_stage_hatx: segments overlap in the bucket");
    }
    a.seg[k] = s;
    if (s.len > longest) longest = s.len;
  }
  for (int k = count; k < SUFHIP_STAGE_MAX_SEGS; ++k) a.seg[k] = sufhip_stage_seg{nullptr, 0, 0, 64};
  if (longest == 0) return SUFHIP_OK;
  size_t gx = (longest + 255) / 256;
  if (gx > 2048) gx = 2048;
  hipLaunchKernelGGL(stage_hatx_kernel, dim3(unsigned(gx), unsigned(count)), dim3(256), 0,
                     as_stream(stream), a);
  return check_launch("stage_hatx_kernel");
}

size_t sufhip_composite_bool_triples(int cuts, int ell) {
  if (cuts < 0 || ell < 1 || ell > SUFHIP_COMPOSITE_MAX_ELL) return 0;
  return size_t(cuts > 0 ? 2 * cuts - 1 : 0) + 2 * size_t(cuts + 1) * size_t(ell);
}

int sufhip_composite_bool2(const sufhip_composite_bool_args* args, void* stream) {
  SUFHIP_REQUIRE(args != nullptr, "sufhip_composite_bool2: null args");
  const sufhip_composite_bool_args& g = *args;
  SUFHIP_REQUIRE(g.ell >= 1 && g.ell <= SUFHIP_COMPOSITE_MAX_ELL,
                 "sufhip_composite_bool2: ell in [1, SUFHIP_COMPOSITE_MAX_ELL]");
  SUFHIP_REQUIRE(g.cuts >= 0 && g.cuts <= SUFHIP_COMPOSITE_MAX_CUTS,
                 "sufhip_composite_bool2: cuts in [0, SUFHIP_COMPOSITE_MAX_CUTS]");
  SUFHIP_REQUIRE(g.queries >= 0 && g.wraps >= 0 && g.wraps <= SUFHIP_COMPOSITE_MAX_WRAP &&
                     g.prog_len >= 0 && g.prog_len <= SUFHIP_COMPOSITE_MAX_PROG,
                 "sufhip_composite_bool2: queries, wraps or program length out of range");
  if (g.n == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(g.out[0] && g.out[1] && g.tri[0] && g.tri[1],
                 "sufhip_composite_bool2: null output or triples");
  SUFHIP_REQUIRE(g.cuts == 0 || (g.cut[0] && g.cut[1]), "sufhip_composite_bool2: null cut bits");
  SUFHIP_REQUIRE(g.queries == 0 || (g.pred[0] && g.pred[1]),
                 "sufhip_composite_bool2: null predicate bits");
  const int progs = (g.cuts + 1) * g.ell;
  SUFHIP_REQUIRE(g.prog_off[0] == 0, "sufhip_composite_bool2: program offsets must start at 0");
  int ands = 0;
  for (int k = 0; k < progs; ++k) {
    SUFHIP_REQUIRE(g.prog_off[k + 1] > g.prog_off[k] && g.prog_off[k + 1] <= g.prog_len,
                   "sufhip_composite_bool2: bad program offsets");
    SUFHIP_REQUIRE(program_ok(g.prog, g.prog_off[k], g.prog_off[k + 1], g.queries, g.wraps, &ands),
                   "sufhip_composite_bool2: program " + std::to_string(k) +
                       " is malformed (opcode, operand or stack depth)");
  }
  SUFHIP_REQUIRE(ands == g.and_count,
                 "sufhip_composite_bool2: and_count differs from the programs' AND/OR count");
  SUFHIP_REQUIRE(ands == 0 || (g.bit_tri[0] && g.bit_tri[1]),
                 "sufhip_composite_bool2: null bit triples");
  BoolArgs a{g};
  size_t blocks = (g.n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  const hipStream_t st = as_stream(stream);
  switch (g.ell) {
#define SUFHIP_ELL_CASE(E)                                                                  \
  case E:                                                                                   \
    hipLaunchKernelGGL(composite_bool2_kernel<E>, dim3(unsigned(blocks)), dim3(256), 0, st, a); \
    break;
    SUFHIP_ELL_CASE(1)
    SUFHIP_ELL_CASE(2)
    SUFHIP_ELL_CASE(3)
    SUFHIP_ELL_CASE(4)
    SUFHIP_ELL_CASE(5)
    SUFHIP_ELL_CASE(6)
    SUFHIP_ELL_CASE(7)
    SUFHIP_ELL_CASE(8)
#undef SUFHIP_ELL_CASE
    default:
      break;
  }
  return check_launch("composite_bool2_kernel");
}

}  // extern "C"
