// Key-only walks of truncation gates' carry DCFs (the myl7/fss v0.7.1 DCF of
// third_party/myl7_fss/src/dcf.c:146-193, 8-byte additive payloads): a table
// gate's full domain walked one node per 8 lanes.  Shared by the prepare
// launches (trunc_gate.hip) and the launch that runs the walks beside the
// opens' digit-plane split (beaver_mfma2.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "dcf_device.hpp"
#include "suf_hip.h"
#include "trunc_device.hpp"

namespace sufhip {

// Plans the key-only halves of `count` truncation jobs (at most max_jobs) as
// one walk launch with every level walked by its own 8 lanes: *one is set
// when that launch alone prepares every job (table gates, few enough walks
// that sufhip_trunc_prepare_batch would expand no level locally either), and
// then begin[0..count], key, out and geo hold WalkJobs' fields.  Otherwise
// the jobs need sufhip_trunc_prepare_batch's own launches.  Validates every
// job as that entry point does (defined in trunc_gate.hip).
int trunc_walk_plan(const uint8_t* prg_state, const sufhip_trunc_job* jobs, int count,
                    int max_jobs, uint32_t* begin, const uint8_t** key, uint4** out,
                    uint32_t* geo, bool* one);

// Plans `count` table-gate jobs (at most max_jobs) as the walks of a launch
// that another kernel hosts, with room for lanes_cap walk lanes at once: the
// fewest local levels (at most kWalkLocal) whose walks fit in lanes_cap, so
// that the walks take one pass of the room when they can.  *one is set when
// every job is a table gate (f <= 14, no expansion launches) and there are at
// most max_jobs of them; then begin[0..count], key, out and geo hold
// WalkJobs' fields for walk_table.  Validates every job as
// sufhip_trunc_prepare_batch does (defined in trunc_gate.hip).
int trunc_walk_plan_fit(const uint8_t* prg_state, const sufhip_trunc_job* jobs, int count,
                        int max_jobs, size_t lanes_cap, uint32_t* begin, const uint8_t** key,
                        uint4** out, uint32_t* geo, bool* one, const char* what);

namespace {

// A table job's walks go to depth f - kWalkLocal and expand the last
// kWalkLocal levels themselves (both children of each node), so a walk writes
// 2^kWalkLocal entries: 2 (f - kWalkLocal) + 4 (2^kWalkLocal - 1) AES blocks
// per 2^kWalkLocal entries instead of 2 f per entry.
#ifndef SUFHIP_WALK_LOCAL
#define SUFHIP_WALK_LOCAL 4
#endif
constexpr int kWalkLocal = SUFHIP_WALK_LOCAL;
static_assert(kWalkLocal >= 1 && kWalkLocal <= 4, "kWalkLocal: 1..4");
#ifndef SUFHIP_WALK_GROUP
#define SUFHIP_WALK_GROUP 4
#endif
constexpr int kWalkGroup = SUFHIP_WALK_GROUP;  // lockstep width of the expansion

// Up to kJobs jobs of one walk launch: lanes [8 begin[j], 8 begin[j+1]) walk
// job j's nodes.
template <int kJobs>
struct WalkJobs {
  Prg4 prg;
  int count;
  uint32_t begin[kJobs + 1];
  const uint8_t* key[kJobs];
  uint4* out[kJobs];
  uint32_t geo[kJobs];  // f | d << 8 | e << 16: bits, depth written, local levels
};

// The job of lane g: the last j < count with begin[j] <= g (jobs with no
// lanes share their begin with the next job, so the last such j owns g).
template <int kJobs>
__device__ __forceinline__ int batch_job(const uint32_t (&begin)[kJobs + 1], int count,
                                         uint32_t g) {
  int lo = 0, hi = count - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (begin[mid] <= g)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

// One walk per 8 lanes.  Lanes 0-3 of the group compute the next-seed block
// AES_{K_{2b}}(s) and lanes 4-7 the value block AES_{K_{2b+1}}(s), column-
// parallel (encrypt_quad_n of the AES table type): lane q of either half
// holds word q of the seed.  A level is then about a quarter of the dependent
// issue time of the one-lane walk (add64_walk), which bounds these
// latency-bound launches.
struct Walk8 {
  uint32_t s;  // seed word q (both halves)
  uint32_t t;  // control bit (both halves)
  uint64_t v;  // accumulated value, low 64 bits (value half)
};

// Little-endian word at byte address p + 4 idx (any alignment; reads the
// aligned words idx and idx + 1 around it).
__device__ __forceinline__ uint32_t word_at(const uint8_t* p, int idx) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t* w = reinterpret_cast<const uint32_t*>(a & ~uintptr_t(3));
  return __builtin_amdgcn_alignbyte(w[idx + 1], w[idx], uint32_t(a & 3));
}

__device__ __forceinline__ uint32_t row_shr4(uint32_t v) {
  return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x114, 0xf, 0xf, false));
}

template <class Aes>
struct Walk8Ctx {
  const Aes& aes;
  const uint4* rkl;
  const uint8_t* chunk;
  uint4* nodes;
  int f;
  uint32_t party, h, q;
};

// One level (record cw) of N independent walks in lockstep: walk n goes
// from state par[(b0 + n) >> 1] towards child bit (b0 + n) & 1 (the walk
// loop passes N = 1 and its own bit as b0).  add64_walk's level on 8 lanes.
template <int N, class Ctx>
__device__ __forceinline__ void walk8_step_n(const Ctx& c, const uint8_t* cw, uint32_t b0,
                                             const Walk8* par, Walk8* kid) {
  const uint32_t csq = word_at(cw, int(c.q));
  const uint64_t cv = uint64_t(word_at(cw, 4)) | uint64_t(word_at(cw, 5)) << 32;
  const uint32_t tb = cw[32];
  uint32_t o[N];
  const uint32_t* rkq[N];
#pragma unroll
  for (int n = 0; n < N; ++n) {
    const uint32_t b = N == 1 ? b0 : ((b0 + n) & 1u);
    o[n] = par[N == 1 ? 0 : (b0 + n) >> 1].s;
    rkq[n] = reinterpret_cast<const uint32_t*>(c.rkl + 11 * (2 * b + c.h)) + c.q;
  }
  c.aes.template encrypt_quad_n<N>(o, rkq);
#pragma unroll
  for (int n = 0; n < N; ++n) {
    const Walk8& w = par[N == 1 ? 0 : (b0 + n) >> 1];
    const uint32_t b = N == 1 ? b0 : ((b0 + n) & 1u);
    uint32_t on = o[n] ^ w.s;
    // Value half: the low 64 bits of its block; seed half: bit 127 of its block.
    const uint64_t vd0 = uint64_t(quad_bcast<0>(on)) | uint64_t(quad_bcast<1>(on)) << 32;
    uint32_t tn = quad_bcast<3>(on) >> 31;
    if (c.q == 3) on &= 0x7fffffffu;
    on ^= csq & (0u - w.t);
    tn ^= ((b ? tb : (tb >> 1)) & 1u) & w.t;
    const uint64_t vd = vd0 + (w.t ? cv : 0);
    Walk8 r;
    r.v = w.v + (c.party ? 0 - vd : vd);
    // The seed half's next seed and t move to the value half (lane - 4).
    const uint32_t os = row_shr4(on), ts = row_shr4(tn);
    r.s = c.h ? os : on;
    r.t = c.h ? ts : tn;
    kid[n] = r;
  }
}

// Table entry `leaf` from a depth-f state (add64_finish), written by lane 0
// of the value half, which holds the seed, t and v.
template <class Ctx>
__device__ __forceinline__ void walk8_leaf(const Ctx& c, const Walk8& w, uint32_t leaf) {
  const uint8_t* np1 = c.chunk + 16 + 33 * c.f;
  const uint64_t s64 = uint64_t(quad_bcast<0>(w.s)) | uint64_t(quad_bcast<1>(w.s)) << 32;
  const uint64_t n64 = uint64_t(word_at(np1, 0)) | uint64_t(word_at(np1, 1)) << 32;
  const uint64_t sv = s64 + (w.t ? n64 : 0);
  const uint64_t out = w.v + (c.party ? 0 - sv : sv);
  if (c.h == 1 && c.q == 0)
    c.nodes[2 * leaf + 1] = make_uint4(uint32_t(out), uint32_t(out >> 32), 0, 0);
}

// Breadth-first expansion of the subtree below a depth-(f - E) node: the
// 2^(L+1) children of level L in lockstep groups of kWalkGroup, then the
// table entries (v << E) | i in order.
template <int L, int E, class Ctx>
__device__ __forceinline__ void walk8_expand(const Ctx& c, const uint8_t* cw,
                                             const Walk8 (&par)[1 << L], uint32_t v) {
  if constexpr (L == E) {
    walk8_leaf(c, par[0], v);  // E = 0
  } else if constexpr (L + 1 == E) {
    // The last level: each group's children are written as soon as they exist.
    constexpr int kKids = 2 << L;
    constexpr int kGroup = kKids < kWalkGroup ? kKids : kWalkGroup;
#pragma unroll
    for (int b0 = 0; b0 < kKids; b0 += kGroup) {
      Walk8 kid[kGroup];
      walk8_step_n<kGroup>(c, cw, b0, par, kid);
#pragma unroll
      for (int i = 0; i < kGroup; ++i) walk8_leaf(c, kid[i], (v << E) | uint32_t(b0 + i));
    }
  } else {
    constexpr int kKids = 2 << L;
    constexpr int kGroup = kKids < kWalkGroup ? kKids : kWalkGroup;
    Walk8 kid[kKids];
#pragma unroll
    for (int b0 = 0; b0 < kKids; b0 += kGroup) walk8_step_n<kGroup>(c, cw, b0, par, kid + b0);
    walk8_expand<L + 1, E>(c, cw + 33, kid, v);
  }
}

// Lane gl's walk of every level: table entry v of the job with key `key`,
// table `out` and geometry `geo` (WalkJobs::geo, d = f and no local levels,
// as trunc_walk_plan gives).  The caller finds the job of lane gl (batch_job)
// and leaves past the launch's last walk; whole 8-lane groups leave together.
// (trunc_batch_walk_kernel runs the same steps with local levels and
// frontier nodes.)
template <class Aes>
__device__ __forceinline__ void walk_leaf_path(const Aes& aes, const uint4* rkl,
                                               const uint8_t* key, uint4* out, uint32_t geo,
                                               uint32_t v, uint32_t gl) {
  if (!(key[7] & 1)) return;
  const int f = int(geo & 0xff);
  const uint8_t* chunk = key + kTruncHdrBytes + 8;
  const Walk8Ctx<Aes> c{aes, rkl, chunk, out, f, uint32_t(key[6] & 1u), (gl >> 2) & 1u, gl & 3u};
  Walk8 w;
  w.s = word_at(chunk, int(c.q));
  if (c.q == 3) w.s &= 0x7fffffffu;
  w.t = c.party;
  w.v = 0;
  const uint8_t* cw = chunk + 16;
  for (int i = 0; i < f; ++i, cw += 33) {
    Walk8 n[1];
    walk8_step_n<1>(c, cw, (v >> (f - 1 - i)) & 1u, &w, n);
    w = n[0];
  }
  walk8_leaf(c, w, v);
}

// Lane gl's walk of a table job with e = geo >> 16 local levels (0..4): the
// depth-(f - e) node v, then its subtree's 2^e table entries (v << e) + i,
// as trunc_batch_walk_kernel walks table jobs.  For kernels that run these
// walks as a role beside their own work, at 512 lanes per workgroup or
// fewer (the expansion's lockstep groups need more than the 128 registers
// of a 1024-lane workgroup when passed through this function).
template <class Aes>
__device__ __forceinline__ void walk_table(const Aes& aes, const uint4* rkl, const uint8_t* key,
                                           uint4* out, uint32_t geo, uint32_t v, uint32_t gl) {
  if (!(key[7] & 1)) return;
  const int f = int(geo & 0xff), e = int(geo >> 16);
  const uint8_t* chunk = key + kTruncHdrBytes + 8;
  const Walk8Ctx<Aes> c{aes, rkl, chunk, out, f, uint32_t(key[6] & 1u), (gl >> 2) & 1u, gl & 3u};
  Walk8 w;
  w.s = word_at(chunk, int(c.q));
  if (c.q == 3) w.s &= 0x7fffffffu;
  w.t = c.party;
  w.v = 0;
  const int dw = f - e;
  const uint8_t* cw = chunk + 16;
  for (int i = 0; i < dw; ++i, cw += 33) {
    Walk8 n[1];
    walk8_step_n<1>(c, cw, (v >> (dw - 1 - i)) & 1u, &w, n);
    w = n[0];
  }
  const Walk8 root[1] = {w};
  if (e == 0)
    walk8_leaf(c, w, v);
  else if (e == 1)
    walk8_expand<0, 1>(c, cw, root, v);
  else if (e == 2)
    walk8_expand<0, 2>(c, cw, root, v);
  else if (e == 3)
    walk8_expand<0, 3>(c, cw, root, v);
  else  // e == 4 = kWalkLocal at most (static_assert above)
    walk8_expand<0, 4>(c, cw, root, v);
}

// The walk role of a host kernel's spare workgroups (table jobs planned by
// trunc_walk_plan_fit): lane gl of the launch's walk lanes, on the role's own
// AES tables and round keys in LDS -- the walk launch's four-table span
// (kFour: 128 KB, for hosts with one workgroup per CU and the LDS to spare)
// or a 16-copy single table (16 KB).  Called by whole workgroups (it has
// barriers); whole 8-lane groups leave together.
constexpr int kHostedWalkCopies = 16;

template <int kJobs, bool kFour>
__device__ __forceinline__ void hosted_walk_role(const WalkJobs<kJobs>& w, uint32_t gl) {
  using Aes = std::conditional_t<kFour, DcfAes, AesLds<kHostedWalkCopies>>;
  __shared__ __align__(16) uint32_t wtab[Aes::kWords];
  __shared__ uint4 rkl[4 * 11];
  if constexpr (kFour) {
    __shared__ uint32_t stage[256];
    DcfAes::fill(wtab, stage, kTDev.v);
  } else {
    fill_ttable<kHostedWalkCopies>(wtab, kTDev.v);
  }
  fill_round_keys(rkl, w.prg.rk, 4);
  __syncthreads();
  const Aes aes = [&] {
    if constexpr (kFour)
      return DcfAes::make(wtab);
    else
      return Aes{wtab, uint32_t(threadIdx.x % kHostedWalkCopies)};
  }();
  const uint32_t g = gl >> 3;
  if (g >= w.begin[w.count]) return;
  const int j = batch_job<kJobs>(w.begin, w.count, g);
  walk_table(aes, rkl, w.key[j], w.out[j], w.geo[j], g - w.begin[j], gl);
}

// Host side of a hosted walk: w for `count` jobs walked by a launch with
// room for lanes_cap walk lanes in one pass, and *lanes = the walk lanes the
// launch must add (0 for no jobs).  Job sets a hosted walk cannot take (more
// than kJobs jobs, gates other than table gates) go through
// sufhip_trunc_prepare_batch on `stream` here instead, with *lanes = 0.
template <int kJobs>
int plan_hosted_walk(const uint8_t* prg_state, const sufhip_trunc_job* jobs, int count,
                     size_t lanes_cap, void* stream, const char* what, WalkJobs<kJobs>& w,
                     size_t* lanes) {
  *lanes = 0;
  w.count = 0;
  if (count <= 0) return SUFHIP_OK;
  bool one = false;
  if (int rc = trunc_walk_plan_fit(prg_state, jobs, count, kJobs, lanes_cap, w.begin, w.key,
                                   w.out, w.geo, &one, what))
    return rc;
  if (!one) return sufhip_trunc_prepare_batch(prg_state, jobs, count, stream);
  fill_prg4(prg_state, &w.prg);
  w.count = count;
  *lanes = 8 * size_t(w.begin[count]);
  return SUFHIP_OK;
}

}  // namespace
}  // namespace sufhip
