// Row-local task blocks for two parties on one GPU, each in one launch.
//
// With both parties in one process every open is a local sum, so a task
// chain whose rounds only combine values of one row needs no grid-wide
// synchronisation: one workgroup runs all rounds of its row, holding the row
// in registers, with workgroup sums for the row reductions and one lane for
// the per-row scalar gates.  Element indices, triples and keys are those of
// the launch-per-step evaluation, so the shares are bit-identical to it.
//
//   layernorm2_kernel  LayerNormTask (include/runtime/phase_tasks.hpp:
//                      2186-2668) with RsqrtTask (:1383-1700)
//   softmax2_kernel    SoftmaxBlockTask (include/nn/softmax_block_task.hpp:
//                      97-450) with RowMaxDiffTask, nExp, row sum, Recip
#include <hip/hip_runtime.h>

#include <type_traits>

#include "chain_device.hpp"
#include "digit_planes.hpp"
#include "reduce_device.hpp"
#include "relu_tree_device.hpp"
#include "walk_device.hpp"

namespace sufhip {
namespace {

// Rows of up to 1024 elements: 512 threads, up to two elements each (half
// the per-thread element work of 256 threads; the first LayerNorm of the
// layer 22.6 -> 21.4 us).  Longer rows (up to 2048): 256 threads, up to eight
// elements each (at 512 threads eight elements spill).
constexpr int kLnBlock = 512;
constexpr int kLnWideBlock = 256;
constexpr int kLnMaxPer = 2;      // elements per thread at kLnBlock: cols <= 1024
constexpr int kLnWidePer = 8;     // at kLnWideBlock: cols <= 2048
constexpr int kLnCopies = 4;  // the T table serves one lane per workgroup
using LnAes = AesLds<kLnCopies>;  // one lane's chain: the small table fills fastest
// Key-only walks of later gates' tables, run by the workgroups past the rows'
// (hosted_walk_role): up to kLnWalkJobs jobs.
constexpr int kLnWalkJobs = 24;

struct LnArgs {
  const uint64_t* x[2];
  int rows, cols;
  uint64_t inv_len, eps;
  TruncEpi tr[5];  // mean, var0, var1, norm, and the input's (with in_slices)
  uint64_t mask[5];
  sufhip_triple2 sq, norm;
  ChainArgs rs;
  uint64_t* out[2];
  sufhip_x_planes xp;
  const uint64_t* in_slices;  // optional: [slices][2][rows cols] partial products
  int in_count;
  int row_groups;              // workgroups [0, row_groups) run the rows
  WalkJobs<kLnWalkJobs> w;     // the others walk these jobs' tables
};
static_assert(sizeof(LnArgs) <= 4096, "kernel argument blocks must fit in 4 KB");

enum { kTrMean = 0, kTrVar0 = 1, kTrVar1 = 2, kTrNorm = 3, kTrIn = 4 };
constexpr int kLnMaxSlices = 8;
constexpr int kLnMaxInPer = kLnMaxPer;  // in_slices rows of up to 1024 elements

// Every load that does not depend on an open is issued when the row starts:
// x, both triples' shares, and (lane 0) the rsqrt chain's triples; the key
// headers of all truncation gates sit in LDS.  What remains serial per row
// is one table read per truncation gate and the rsqrt LUT's AES.
// kWalk: the workgroups past the rows' walk A.w's jobs (a separate
// instantiation, so that launches without walks keep the rows' own register
// allocation and LDS).
template <int kPer, bool kIn, int kBlock, bool kWalk>
__global__ void __launch_bounds__(kBlock) layernorm2_kernel(LnArgs A) {
  constexpr int kLnWaves = kBlock / 64;
  if constexpr (kWalk) {
    if (int(blockIdx.x) >= A.row_groups) {
      hosted_walk_role<kLnWalkJobs, true>(A.w,
                                          (blockIdx.x - A.row_groups) * kBlock + threadIdx.x);
      return;
    }
  }
  __shared__ __align__(16) uint32_t tab[256 * kLnCopies];
  __shared__ ChainLds L;
  constexpr int kRsProds = chain_products<SUFHIP_CHAIN_RSQRT>();
  __shared__ TruncHdr th[5][2];
  __shared__ TruncHdr rth[kRsProds][2];  // the rsqrt chain's truncation key headers
  __shared__ uint64_t red[2][kLnWaves];
  __shared__ uint64_t bc[2];
  __shared__ ChainPre pre;
  fill_ttable<kLnCopies>(tab, kTDev.v);
  chain_stage(A.rs, 2, L);
  if (threadIdx.x < (kIn ? 10 : 8))
    th[threadIdx.x >> 1][threadIdx.x & 1] =
        read_trunc_hdr(A.tr[threadIdx.x >> 1].key[threadIdx.x & 1]);
  {
    TruncHdrStager<kRsProds> hs;
    hs.load(A.rs, 64);
    hs.store(rth);
  }
  __syncthreads();
  chain_compare(A.rs, L);
  __syncthreads();
  const LnAes aes{tab, threadIdx.x % kLnCopies};
  const ChainKeyInfo K = chain_key_info(A.rs, L);
  auto gate = [&](int j, uint64_t v) {
    return Two{{trunc_table_eval_h(th[j][0], A.tr[j].table[0], A.tr[j].f, v),
                trunc_table_eval_h(th[j][1], A.tr[j].table[1], A.tr[j].f, v)}};
  };
  const int cols = A.cols;
  for (int r = blockIdx.x; r < A.rows; r += A.row_groups) {
    const size_t base = size_t(r) * size_t(cols);
    // The row's rsqrt triples, one word per lane (visible to lane 0 after
    // the row sum's barriers).
    if (threadIdx.x < 24) pre.word(threadIdx.x) = chain_triple_word(A.rs, threadIdx.x, size_t(r));
    // Loads in the order of use (x, the square's triple, the norm triple):
    // each step then waits only for its own words, and the norm triple's
    // arrive while lane 0 runs the rsqrt chain.
    uint64_t d[kPer][2], sa[kPer][2], sb[kPer][2], sc[kPer][2], na[kPer][2], nc[kPer][2];
    if (kIn) {
      // x = tr_in(the open of the product's slice sums) + addend, written
      // out as the product's output.  All slice and addend loads first.
      const size_t mn = size_t(A.rows) * size_t(cols);
      const TruncEpi& ti = A.tr[kTrIn];
      uint64_t ad[kPer][2];
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const int c = threadIdx.x + k * kBlock;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          d[k][p] = 0;
          ad[k][p] = c < cols && ti.add[0] ? ti.add[p][base + c] : 0;
        }
      }
      // Slices in groups of four, then one by one: every load of a group is
      // unconditional (a lane past the row end reads the row's first
      // element and drops the sum), so a group is one round trip.  A load
      // whose value a select or branch might drop would be sunk into the
      // branch and wait for the loads before it.
      const int ns = A.in_count;
      auto add_slices = [&](int z0, auto nz) {
        constexpr int kN = decltype(nz)::value;
        uint64_t t[kPer][2][kN];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
          const int c = threadIdx.x + k * kBlock;
          const size_t e = c < cols ? base + c : base;
#pragma unroll
          for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int dz = 0; dz < kN; ++dz)
              t[k][p][dz] = A.in_slices[(size_t(z0 + dz) * 2 + p) * mn + e];
        }
        // Every load of the group before any add (the scheduler otherwise
        // waits for each element's loads before issuing the next one's).
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < kPer; ++k)
#pragma unroll
          for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int dz = 0; dz < kN; ++dz) d[k][p] += t[k][p][dz];
      };
      int z0 = 0;
      for (; z0 + 4 <= ns; z0 += 4) add_slices(z0, std::integral_constant<int, 4>{});
      for (; z0 < ns; ++z0) add_slices(z0, std::integral_constant<int, 1>{});
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        if (threadIdx.x + k * kBlock >= cols) d[k][0] = d[k][1] = 0;
      }
      uint64_t zh[kPer], w[kPer][2];
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        zh[k] = d[k][0] + d[k][1] + A.mask[kTrIn];
        w[k][0] = trunc_table_word(th[kTrIn][0], ti.table[0], ti.f, zh[k]);
        w[k][1] = trunc_table_word(th[kTrIn][1], ti.table[1], ti.f, zh[k]);
      }
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const int c = threadIdx.x + k * kBlock;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          d[k][p] = c < cols ? trunc_table_out(th[kTrIn][p], ti.f, zh[k], w[k][p]) + ad[k][p] : 0;
          if (c < cols) ti.y[p][base + c] = d[k][p];
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const int c = threadIdx.x + k * kBlock;
#pragma unroll
        for (int p = 0; p < 2; ++p) d[k][p] = c < cols ? A.x[p][base + c] : 0;
      }
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int c = threadIdx.x + k * kBlock;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        sa[k][p] = c < cols ? A.sq.a[p][base + c] : 0;
        sb[k][p] = c < cols ? A.sq.b[p][base + c] : 0;
        sc[k][p] = c < cols ? A.sq.c[p][base + c] : 0;
      }
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int c = threadIdx.x + k * kBlock;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        na[k][p] = c < cols ? A.norm.a[p][base + c] : 0;
        nc[k][p] = c < cols ? A.norm.c[p][base + c] : 0;
      }
    }
    const uint64_t nb0 = A.norm.b[0][r], nb1 = A.norm.b[1][r];
    uint64_t s0 = 0, s1 = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      s0 += d[k][0];
      s1 += d[k][1];
    }
    // mu = tr_mean(inv_len * row sum).
    block_sum2_u64<kLnWaves>(s0, s1, red);
    const Two mu = gate(kTrMean, s0 * A.inv_len + s1 * A.inv_len + A.mask[kTrMean]);
    // d = x - mu; q = d * d (Beaver), summed over the row.
    uint64_t q0 = 0, q1 = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int c = threadIdx.x + k * kBlock;
      if (c < cols) {
        d[k][0] -= mu.v[0];
        d[k][1] -= mu.v[1];
        const uint64_t dd = (d[k][0] - sa[k][0]) + (d[k][1] - sa[k][1]);
        const uint64_t ee = (d[k][0] - sb[k][0]) + (d[k][1] - sb[k][1]);
        q0 += sc[k][0] + dd * sb[k][0] + ee * sa[k][0] + dd * ee;
        q1 += sc[k][1] + dd * sb[k][1] + ee * sa[k][1];
      }
    }
    block_sum2_u64<kLnWaves>(q0, q1, red);
    const Two va = gate(kTrVar0, q0 * A.inv_len + q1 * A.inv_len + A.mask[kTrVar0]);
    const Two var = gate(kTrVar1, va.v[0] + va.v[1] + A.mask[kTrVar1]);
    // rsqrt of the row's variance on the first wave (its keystream blocks
    // column-parallel on eight lanes, the rest of the chain on every lane).
    if (threadIdx.x < 64) {
      const Two v{{var.v[0] + A.eps, var.v[1]}};
      const Two rs =
          chain_eval_quad<SUFHIP_CHAIN_RSQRT, LnAes>(A.rs, L, K, aes, size_t(r), v, pre, rth);
      if (threadIdx.x == 0) {
        bc[0] = rs.v[0];
        bc[1] = rs.v[1];
      }
    }
    __syncthreads();
    // out = tr_norm(d * rs[row]) (row-broadcast Beaver).
    const uint64_t ee = (bc[0] - nb0) + (bc[1] - nb1);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int c = threadIdx.x + k * kBlock;
      if (c < cols) {
        const size_t i = base + c;
        const uint64_t dd = (d[k][0] - na[k][0]) + (d[k][1] - na[k][1]);
        const uint64_t z0 = nc[k][0] + dd * nb0 + ee * na[k][0] + dd * ee;
        const uint64_t z1 = nc[k][1] + dd * nb1 + ee * na[k][1];
        const Two o = gate(kTrNorm, z0 + z1 + A.mask[kTrNorm]);
        if (A.out[0]) {
          A.out[0][i] = o.v[0];
          A.out[1][i] = o.v[1];
        }
        if (A.xp.planes) {
          put_x_digits(A.xp, size_t(A.rows), i, 0, o.v[0]);
          put_x_digits(A.xp, size_t(A.rows), i, 1, o.v[1]);
        }
      }
    }
    __syncthreads();  // bc is rewritten for the next row
  }
}

// Softmax rows: one wavefront per row, groups of `waves` rows per workgroup.
// The row's scores go to registers and to level 0 of the max tree in LDS;
// after the tree every step is wave-local (the row sum is a wave reduction,
// the reciprocal runs on lane 0 and is broadcast by a lane shuffle).
constexpr int kSmRounds = 10;
constexpr int kSmMaxRow = 512;
// Six rows per workgroup, one workgroup per CU: the 64 KB two-table AES
// span, the staged keys and six rows of up to 512 elements fit the CU's
// 160 KB of LDS, and the config's 1536 rows are one workgroup on each of
// 256 CUs.
constexpr int kSmWaves = 6;
constexpr int kSmThreads = 64 * kSmWaves;
using SmAes = AesLds2<32>;
constexpr size_t kSmLdsCap = 160 * 1024;
constexpr int kSmLock = 2;  // nExp chains per lane evaluated in lockstep

struct SmArgs {
  sufhip_operand2 x;
  int pre;
  TruncEpi pre_tr[2];
  uint64_t pre_mask[2];
  const int32_t* offs;
  const int32_t* round_off;
  TreeKeys<kSmRounds> keys;
  int rows, max_row, waves;
  ChainArgs nexp, recip;
  sufhip_triple2 norm;
  TruncEpi tr_norm;
  uint64_t norm_mask;
  uint64_t* out[2];
  uint64_t* dense;
  const uint64_t* dense_a[2];
  int dense_cols;
  sufhip_kb_planes dkb;  // the dense open also as digit planes
};

struct SmStatic {
  uint32_t tab[SmAes::kSpanWords];
  TreeLds<kSmRounds> t;
  ChainLds nexp, recip;
  TruncHdr thn[3][2], thr[3][2];  // the chains' truncation key headers
  ChainPreN<3> rpre[kSmWaves];  // each row's reciprocal triples
  uint32_t j0[kSmWaves][kSmRounds];  // each row's tree slot offsets
};

__device__ __forceinline__ uint64_t bcast_lane0(uint64_t v) {
  const uint32_t lo = __shfl(uint32_t(v), 0, 64);
  const uint32_t hi = __shfl(uint32_t(v >> 32), 0, 64);
  return uint64_t(lo) | uint64_t(hi) << 32;
}

// Everything the block keeps in LDS for the whole launch -- the AES span,
// every tree round's keys, both chains' keys -- in one staging pass: a
// thread issues all of its global loads (about a dozen table words, up to
// two tree items and a few chain items, spread over the workgroup by a flat
// item index) before its first LDS store, so staging costs about one memory
// round trip.  load() and store() split the pass so that the first rows'
// loads go in between; the caller syncs after store().
template <int kThreads>
struct SmStagerT {
  static constexpr int kChainPer = (3 * kSmThreads + kThreads - 1) / kThreads;
  typename SmAes::template Filler<kThreads> tf;
  TreeStager<kSmRounds, 2> ts;
  TruncHdrStager<3> hn, hr;
  uint4 cv[kChainPer];
  int c0, nn, nc;
  __device__ __forceinline__ void load(const SmArgs& a) {
    static_assert(kSmRounds * kTreeItems <= 2 * kThreads, "SmStager: tree items in one pass");
    tf.load(kTDev.v);
    ts.load(kernarg_tree_keys<kSmRounds>(offsetof(SmArgs, keys)), int(threadIdx.x));
    hn.load(a.nexp, 0);
    hr.load(a.recip, 64);
    // Chain items continue the tree's flat item space.
    nn = chain_items(a.nexp, 4);
    nc = nn + chain_items(a.recip, 2);
    const int shift = (a.keys.rounds * kTreeItems) % kThreads;
    c0 = (int(threadIdx.x) + kThreads - shift) % kThreads;
#pragma unroll
    for (int u = 0; u < kChainPer; ++u) {
      // Unconditional loads on a clamped item (see TreeStager::load).
      const int c = c0 + u * kThreads < nc ? c0 + u * kThreads : 0;
      bool rn, rr;
      const uint64_t* an = chain_item_addr(a.nexp, 4, c < nn ? c : 0, &rn);
      const uint64_t* ar = chain_item_addr(a.recip, 2, c < nn ? 0 : c - nn, &rr);
      cv[u] = chain_item_fetch(c < nn ? an : ar, c < nn ? rn : rr);
    }
  }
  __device__ __forceinline__ void store(const SmArgs& a, SmStatic& st) const {
#pragma unroll
    for (int u = 0; u < kChainPer; ++u) {
      const int c = c0 + u * kThreads;
      if (c < nn)
        chain_item_store(a.nexp, 4, st.nexp, c, cv[u]);
      else if (c < nc)
        chain_item_store(a.recip, 2, st.recip, c - nn, cv[u]);
    }
    // Chains with more items than one pass covers (wide LUTs): the rest
    // item by item.
    for (int c = c0 + kChainPer * kThreads; c < nc; c += kThreads) {
      if (c < nn)
        chain_item_store(a.nexp, 4, st.nexp, c, chain_item_load(a.nexp, 4, c));
      else
        chain_item_store(a.recip, 2, st.recip, c - nn, chain_item_load(a.recip, 2, c - nn));
    }
    ts.store(st.t);
    tf.store(st.tab);
    hn.store(st.thn);
    hr.store(st.thr);
    if (threadIdx.x == 0) {
      st.t.diff = a.keys.own_ks;
      st.nexp.diff = a.nexp.own_ks;
      st.recip.diff = a.recip.own_ks;
    }
  }
};
using SmStager = SmStagerT<kSmThreads>;

template <int kPer>
__global__ void __launch_bounds__(kSmThreads) softmax2_kernel(SmArgs a) {
  __shared__ __align__(16) SmStatic st;
  extern __shared__ uint64_t rowbuf[];
  const int mr = a.max_row;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  uint64_t* even = rowbuf + size_t(wave) * tree_row_words(mr);
  uint64_t* odd = even + 2 * size_t(mr);
  constexpr bool kPre = kPer <= 2;
  int b = 0, len = 0;
  uint64_t na[kPre ? kPer : 1][2], nc[kPre ? kPer : 1][2];
  uint64_t s[kPer][2];
  // Group g's row loads: offsets, the loads that need no open (issued now
  // to land while the tree runs: the reciprocal's triples, one word per
  // lane, to LDS, and for short rows every element's normalisation triple),
  // and the scores through the optional truncations of their open, into
  // registers and level 0 of the tree.  They touch no staged LDS, so for
  // rows of up to 128 elements the first group's run before the staging and
  // overlap its loads (longer rows keep too many scores in registers).
  auto load_rows = [&](int g) {
    const int r = g * a.waves + wave;
    b = 0;
    len = 0;
    if (r < a.rows) {
      b = a.offs[r];
      len = a.offs[r + 1] - b;
      if (len < 1 || len > mr) len = 0;  // refused on the host
    }
    if (len > 0 && lane < 18) st.rpre[wave].word(lane) = chain_triple_word(a.recip, lane, size_t(r));
    tree_row_offsets(a.keys, a.round_off, a.rows, r, len, st.j0[wave]);
    if constexpr (kPre) {
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const int j = lane + 64 * k;
        const size_t i = size_t(b) + size_t(j < len ? j : 0);
        na[k][0] = j < len ? a.norm.a[0][i] : 0;
        na[k][1] = j < len ? a.norm.a[1][i] : 0;
        nc[k][0] = j < len ? a.norm.c[0][i] : 0;
        nc[k][1] = j < len ? a.norm.c[1][i] : 0;
      }
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int j = lane + 64 * k;
      s[k][0] = s[k][1] = 0;
      if (j < len) {
        const size_t i = size_t(b) + size_t(j);
        uint64_t v0 = operand_at(a.x, 0, i), v1 = operand_at(a.x, 1, i);
        // Compile-time gate indices: a runtime index into the by-value
        // argument block would copy it to private scratch memory.
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          if (q >= a.pre) break;
          const uint64_t o = v0 + v1 + a.pre_mask[q];
          v0 = trunc_table_eval(a.pre_tr[q].key[0], a.pre_tr[q].table[0], a.pre_tr[q].f, o);
          v1 = trunc_table_eval(a.pre_tr[q].key[1], a.pre_tr[q].table[1], a.pre_tr[q].f, o);
        }
        s[k][0] = v0;
        s[k][1] = v1;
        even[j] = v0;
        even[mr + j] = v1;
      }
    }
  };
  {
    SmStager stager;
    stager.load(a);
    if constexpr (kPre) load_rows(blockIdx.x);
    stager.store(a, st);
  }
  __syncthreads();
  tree_compare(a.keys, st.t);
  chain_compare(a.nexp, st.nexp);
  chain_compare(a.recip, st.recip);
  __syncthreads();
  const SmAes aes = SmAes::make(st.tab);
  const ChainKeyInfo Kn = chain_key_info(a.nexp, st.nexp);
  const ChainKeyInfo Kr = chain_key_info(a.recip, st.recip);
  const uint32_t shared = ~st.t.diff;
  for (int g = blockIdx.x; g * a.waves < a.rows; g += gridDim.x) {
    if (!kPre || g != int(blockIdx.x)) {
      load_rows(g);
      __syncthreads();
    }
    const int r = g * a.waves + wave;
    const int level =
        tree_row<kSmRounds, SmAes>(a.keys, st.t, aes, even, odd, mr, len, st.j0[wave], shared);
    const uint64_t* fin = (level & 1) ? odd : even;
    const int fw = (level & 1) ? (mr + 1) / 2 : mr;
    const uint64_t m0 = len > 0 ? fin[0] : 0, m1 = len > 0 ? fin[fw] : 0;
    // e = nExp(max - s), summed over the row; the lane's elements kSmLock at
    // a time, their chains in lockstep (elements past the row end compute on
    // clamped indices and are dropped).
    uint64_t e[kPer][2];
    uint64_t es0 = 0, es1 = 0;
#pragma unroll
    for (int k0 = 0; k0 < kPer; k0 += kSmLock) {
      size_t ii[kSmLock];
      Two dl[kSmLock], ev[kSmLock];
      plain_loader<SUFHIP_CHAIN_CUBIC> pl[kSmLock] = {};
#pragma unroll
      for (int u = 0; u < kSmLock; ++u) {
        const int j = lane + 64 * (k0 + u);
        ii[u] = size_t(b) + size_t(j < len ? j : 0);
        dl[u] = Two{{m0 - s[k0 + u][0], m1 - s[k0 + u][1]}};
        pl[u] = plain_loader<SUFHIP_CHAIN_CUBIC>{&a.nexp, ii[u]};
      }
      chain_eval_m<SUFHIP_CHAIN_CUBIC, SmAes, kSmLock>(a.nexp, st.nexp, Kn, aes, ii, dl, pl,
                                                        ev, st.thn);
#pragma unroll
      for (int u = 0; u < kSmLock; ++u) {
        const bool ok = lane + 64 * (k0 + u) < len;
        e[k0 + u][0] = ok ? ev[u].v[0] : 0;
        e[k0 + u][1] = ok ? ev[u].v[1] : 0;
        es0 += e[k0 + u][0];
        es1 += e[k0 + u][1];
      }
    }
    es0 = wave_sum_u64(es0);
    es1 = wave_sum_u64(es1);
    // inv = Recip(row sum) on the whole wave (its keystream blocks
    // column-parallel on eight lanes, every lane ends with the result).
    uint64_t inv0 = 0, inv1 = 0;
    if (len > 0) {
      const Two iv = chain_eval_quad<SUFHIP_CHAIN_RECIP, SmAes, ChainPreN<3>>(
          a.recip, st.recip, Kr, aes, size_t(r), Two{{es0, es1}}, st.rpre[wave], st.thr);
      inv0 = iv.v[0];
      inv1 = iv.v[1];
    }
    // prob = tr_norm(e * inv[row]) (row-broadcast Beaver), and the next
    // product's open over the dense row.
    if (len > 0) {
      const uint64_t nb0 = a.norm.b[0][r], nb1 = a.norm.b[1][r];
      const uint64_t ee = (inv0 - nb0) + (inv1 - nb1);
      const size_t drow = size_t(r) * size_t(a.dense_cols);
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const int j = lane + 64 * k;
        if (j < len) {
          const size_t i = size_t(b) + size_t(j);
          uint64_t a0, a1, c0, c1;
          if constexpr (kPre) {
            a0 = na[k][0];
            a1 = na[k][1];
            c0 = nc[k][0];
            c1 = nc[k][1];
          } else {
            a0 = a.norm.a[0][i];
            a1 = a.norm.a[1][i];
            c0 = a.norm.c[0][i];
            c1 = a.norm.c[1][i];
          }
          const uint64_t dd = (e[k][0] - a0) + (e[k][1] - a1);
          const uint64_t z0 = c0 + dd * nb0 + ee * a0 + dd * ee;
          const uint64_t z1 = c1 + dd * nb1 + ee * a1;
          const uint64_t o = z0 + z1 + a.norm_mask;
          const uint64_t p0 =
              trunc_table_eval(a.tr_norm.key[0], a.tr_norm.table[0], a.tr_norm.f, o);
          const uint64_t p1 =
              trunc_table_eval(a.tr_norm.key[1], a.tr_norm.table[1], a.tr_norm.f, o);
          if (a.out[0]) {
            a.out[0][i] = p0;
            a.out[1][i] = p1;
          }
          if (a.dense) {
            const size_t di = drow + size_t(j);
            const uint64_t dv = (p0 - a.dense_a[0][di]) + (p1 - a.dense_a[1][di]);
            a.dense[di] = dv;
            if (a.dkb.planes) put_kb_digits(a.dkb, di, dv);
          }
        }
      }
      if (a.dense)
        for (int j = len + lane; j < a.dense_cols; j += 64) {
          const size_t di = drow + size_t(j);
          const uint64_t dv = (uint64_t(0) - a.dense_a[0][di]) + (uint64_t(0) - a.dense_a[1][di]);
          a.dense[di] = dv;
          if (a.dkb.planes) put_kb_digits(a.dkb, di, dv);
        }
    }
    __syncthreads();  // the row buffers are rewritten by the next group
  }
}

// ---------------------------------------------------------------------------
// Rows of up to 128 elements on a team of two waves: six rows per
// workgroup of 768 lanes (twelve waves, three per SIMD; the LDS is the
// six-row kernel's).  Wave t of a row's team holds element lane + 64 t.
// The max tree's first two levels (up to 64 and 32 pairs) are split between
// the team's waves, with a workgroup barrier after each; the shorter levels
// run on the team's first wave.  Each lane then runs one element's nExp
// chain with both parties' keystream blocks in one lockstep group, the
// row sum adds the two waves' partial sums through LDS, the reciprocal runs
// on the first wave's lane 0, and each wave normalises its elements.  The
// per-wave work of the tree's wide levels, of the nExp chain and of the
// normalisation halves; every output equals the one-wave-per-row kernel's.
constexpr int kSmTeam = 2;
constexpr int kSmTeamThreads = 64 * kSmWaves * kSmTeam;
constexpr int kSmTeamMaxRow = 128;

// Levels 0 and 1 split over the team (pairs [32 t, 32 t + 32) and
// [16 t, 16 t + 16)), a workgroup barrier after each; later levels on wave
// t = 0 only (its wave-local ordering as in tree_row).  Every thread of the
// workgroup runs the same number of barriers.  Returns the level count (the
// same in both waves).
template <class Aes>
__device__ __forceinline__ int tree_row_team(const TreeKeys<kSmRounds>& K,
                                             const TreeLds<kSmRounds>& L, const Aes& aes,
                                             uint64_t* even, uint64_t* odd, int mr, int len,
                                             const uint32_t* j0s, uint32_t shared, int tw) {
  const int lane = threadIdx.x & 63, half = (mr + 1) / 2;
  int level = 0;
  for (int k = 0; k < K.rounds; ++k) {
    const bool split = k < 2;
    if (len > 1) {
      const uint64_t* src = (level & 1) ? odd : even;
      const int sw = (level & 1) ? half : mr;
      uint64_t* dst = (level & 1) ? even : odd;
      const int dw = (level & 1) ? mr : half;
      const int pairs = len >> 1;
      const uint32_t j0 = j0s[k];
      const bool one_ks = (shared >> k) & 1u;
      if (split) {
        const int per = k == 0 ? 32 : 16;
        const int t0 = per * tw;
        const int nb = pairs - t0 < per ? pairs - t0 : per;
        if (nb > 16)
          tree_chunk<2>(K, L, aes, k, src, sw, dst, dw, j0, t0, nb, one_ks);
        else if (nb > 0)
          tree_chunk<1>(K, L, aes, k, src, sw, dst, dw, j0, t0, nb, one_ks);
      } else if (tw == 0) {
        for (int t0 = 0; t0 < pairs; t0 += 64) {
          const int nb = pairs - t0 < 64 ? pairs - t0 : 64;
          if (nb > 48)
            tree_chunk<4>(K, L, aes, k, src, sw, dst, dw, j0, t0, nb, one_ks);
          else if (nb > 32)
            tree_chunk<3>(K, L, aes, k, src, sw, dst, dw, j0, t0, nb, one_ks);
          else if (nb > 16)
            tree_chunk<2>(K, L, aes, k, src, sw, dst, dw, j0, t0, nb, one_ks);
          else
            tree_chunk<1>(K, L, aes, k, src, sw, dst, dw, j0, t0, nb, one_ks);
        }
      }
      if ((len & 1) && lane == 0 && tw == 0) {
        dst[pairs] = src[2 * pairs];
        dst[dw + pairs] = src[sw + 2 * pairs];
      }
      len = (len + 1) >> 1;
      ++level;
    }
    if (split) {
      __syncthreads();
    } else if (tw == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
  return level;
}

__global__ void __launch_bounds__(kSmTeamThreads) softmax2_team_kernel(SmArgs a) {
  __shared__ __align__(16) SmStatic st;
  __shared__ uint64_t part[kSmWaves][kSmTeam][2];  // the team's partial row sums
  __shared__ uint64_t invs[kSmWaves][2];           // the row's reciprocal shares
  extern __shared__ uint64_t rowbuf[];
  const int mr = a.max_row;
  // Wave-uniform (a scalar register): the row offsets then load through the
  // scalar cache and the team's branches are scalar branches.
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int slot = wave >> 1, tw = wave & 1;  // row slot in the group, wave in the team
  const int j = lane + 64 * tw;               // this lane's element of the row
  uint64_t* even = rowbuf + size_t(slot) * tree_row_words(mr);
  uint64_t* odd = even + 2 * size_t(mr);
  int b = 0, len = 0;
  uint64_t na0 = 0, na1 = 0, nc0 = 0, nc1 = 0, s0 = 0, s1 = 0;
  // The row group's loads, as in softmax2_kernel (one element per lane).
  auto load_rows = [&](int g) {
    const int r = g * a.waves + slot;
    b = 0;
    len = 0;
    if (r < a.rows) {
      b = a.offs[r];
      len = a.offs[r + 1] - b;
      if (len < 1 || len > mr) len = 0;  // refused on the host
    }
    if (tw == 0) {
      if (len > 0 && lane < 18)
        st.rpre[slot].word(lane) = chain_triple_word(a.recip, lane, size_t(r));
      tree_row_offsets(a.keys, a.round_off, a.rows, r, len, st.j0[slot]);
    }
    const size_t i = size_t(b) + size_t(j < len ? j : 0);
    na0 = j < len ? a.norm.a[0][i] : 0;
    na1 = j < len ? a.norm.a[1][i] : 0;
    nc0 = j < len ? a.norm.c[0][i] : 0;
    nc1 = j < len ? a.norm.c[1][i] : 0;
    s0 = s1 = 0;
    if (j < len) {
      uint64_t v0 = operand_at(a.x, 0, i), v1 = operand_at(a.x, 1, i);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        if (q >= a.pre) break;
        const uint64_t o = v0 + v1 + a.pre_mask[q];
        v0 = trunc_table_eval(a.pre_tr[q].key[0], a.pre_tr[q].table[0], a.pre_tr[q].f, o);
        v1 = trunc_table_eval(a.pre_tr[q].key[1], a.pre_tr[q].table[1], a.pre_tr[q].f, o);
      }
      s0 = v0;
      s1 = v1;
      even[j] = v0;
      even[mr + j] = v1;
    }
  };
  {
    SmStagerT<kSmTeamThreads> stager;
    stager.load(a);
    load_rows(blockIdx.x);
    stager.store(a, st);
  }
  __syncthreads();
  tree_compare(a.keys, st.t);
  chain_compare(a.nexp, st.nexp);
  chain_compare(a.recip, st.recip);
  __syncthreads();
  const SmAes aes = SmAes::make(st.tab);
  const ChainKeyInfo Kn = chain_key_info(a.nexp, st.nexp);
  const ChainKeyInfo Kr = chain_key_info(a.recip, st.recip);
  const uint32_t shared = ~st.t.diff;
  for (int g = blockIdx.x; g * a.waves < a.rows; g += gridDim.x) {
    if (g != int(blockIdx.x)) {
      load_rows(g);
      __syncthreads();
    }
    const int r = g * a.waves + slot;
    const int level = tree_row_team<SmAes>(a.keys, st.t, aes, even, odd, mr, len, st.j0[slot],
                                           shared, tw);
    __syncthreads();  // the first wave's later levels, for the second wave
    const uint64_t* fin = (level & 1) ? odd : even;
    const int fw = (level & 1) ? (mr + 1) / 2 : mr;
    const uint64_t m0 = len > 0 ? fin[0] : 0, m1 = len > 0 ? fin[fw] : 0;
    // e = nExp(max - s) for this lane's element, both parties' keystream
    // blocks in one lockstep group (elements past the row end compute on a
    // clamped index and are dropped).
    const bool ok = j < len;
    const size_t ii = size_t(b) + size_t(ok ? j : 0);
    const Two ev = chain_eval<SUFHIP_CHAIN_CUBIC, SmAes, plain_loader<SUFHIP_CHAIN_CUBIC>, true>(
        a.nexp, st.nexp, Kn, aes, ii, Two{{m0 - s0, m1 - s1}},
        plain_loader<SUFHIP_CHAIN_CUBIC>{&a.nexp, ii}, st.thn);
    const uint64_t e0 = ok ? ev.v[0] : 0, e1 = ok ? ev.v[1] : 0;
    const uint64_t ps0 = wave_sum_u64(e0), ps1 = wave_sum_u64(e1);
    if (lane == 0) {
      part[slot][tw][0] = ps0;
      part[slot][tw][1] = ps1;
    }
    __syncthreads();
    // inv = Recip(row sum) on the first wave (its keystream blocks
    // column-parallel on eight lanes).
    if (tw == 0 && len > 0) {
      const Two es{{part[slot][0][0] + part[slot][1][0], part[slot][0][1] + part[slot][1][1]}};
      const Two iv = chain_eval_quad<SUFHIP_CHAIN_RECIP, SmAes, ChainPreN<3>>(
          a.recip, st.recip, Kr, aes, size_t(r), es, st.rpre[slot], st.thr);
      if (lane == 0) {
        invs[slot][0] = iv.v[0];
        invs[slot][1] = iv.v[1];
      }
    }
    __syncthreads();
    // prob = tr_norm(e * inv[row]) (row-broadcast Beaver), and the next
    // product's open over the dense row.
    if (len > 0) {
      const uint64_t inv0 = invs[slot][0], inv1 = invs[slot][1];
      const uint64_t nb0 = a.norm.b[0][r], nb1 = a.norm.b[1][r];
      const uint64_t ee = (inv0 - nb0) + (inv1 - nb1);
      const size_t drow = size_t(r) * size_t(a.dense_cols);
      if (ok) {
        const size_t i = size_t(b) + size_t(j);
        const uint64_t dd = (e0 - na0) + (e1 - na1);
        const uint64_t z0 = nc0 + dd * nb0 + ee * na0 + dd * ee;
        const uint64_t z1 = nc1 + dd * nb1 + ee * na1;
        const uint64_t o = z0 + z1 + a.norm_mask;
        const uint64_t p0 = trunc_table_eval(a.tr_norm.key[0], a.tr_norm.table[0], a.tr_norm.f, o);
        const uint64_t p1 = trunc_table_eval(a.tr_norm.key[1], a.tr_norm.table[1], a.tr_norm.f, o);
        if (a.out[0]) {
          a.out[0][i] = p0;
          a.out[1][i] = p1;
        }
        if (a.dense) {
          const size_t di = drow + size_t(j);
          const uint64_t dv = (p0 - a.dense_a[0][di]) + (p1 - a.dense_a[1][di]);
          a.dense[di] = dv;
          if (a.dkb.planes) put_kb_digits(a.dkb, di, dv);
        }
      }
      if (a.dense)
        for (int jj = len + j; jj < a.dense_cols; jj += 64 * kSmTeam) {
          const size_t di = drow + size_t(jj);
          const uint64_t dv = (uint64_t(0) - a.dense_a[0][di]) + (uint64_t(0) - a.dense_a[1][di]);
          a.dense[di] = dv;
          if (a.dkb.planes) put_kb_digits(a.dkb, di, dv);
        }
    }
    __syncthreads();  // the row buffers are rewritten by the next group
  }
}

// The dynamic LDS of a softmax launch goes past 64 KB; allowed once per
// kernel.
template <int kPer>
bool sm_lds_allowed() {
  static const bool ok =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&softmax2_kernel<kPer>),
                          hipFuncAttributeMaxDynamicSharedMemorySize,
                          int(kSmLdsCap - sizeof(SmStatic))) == hipSuccess;
  return ok;
}

constexpr size_t kSmTeamStatic = sizeof(SmStatic) + sizeof(uint64_t) * kSmWaves * (2 * kSmTeam + 2);

bool sm_team_lds_allowed() {
  static const bool ok =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&softmax2_team_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize,
                          int(kSmLdsCap - kSmTeamStatic)) == hipSuccess;
  return ok;
}

int triple_ok(const sufhip_triple2& t) {
  return t.a[0] && t.a[1] && t.b[0] && t.b[1] && t.c[0] && t.c[1];
}

int table_epi(const sufhip_trunc_epilogue& t, size_t n, const char* what, TruncEpi* e) {
  sufhip_trunc_epilogue c = t;
  if (c.add[0] || c.add[1]) {
    set_error(std::string(what) + ": the block's truncations take no addend");
    return SUFHIP_ERR_INVALID;
  }
  uint64_t dummy = 0;
  c.y[0] = c.y[1] = &dummy;  // the block writes its own outputs
  return make_epi(&c, n, what, e);
}

}  // namespace
}  // namespace sufhip

using namespace sufhip;

extern "C" {

int sufhip_layernorm2(const sufhip_layernorm2_args* args, void* stream) {
  SUFHIP_REQUIRE(args != nullptr, "sufhip_layernorm2: null args");
  const sufhip_layernorm2_args& g = *args;
  SUFHIP_REQUIRE(g.rows >= 0 && g.cols >= 1 && g.cols <= kLnWideBlock * kLnWidePer,
                 "sufhip_layernorm2: cols in [1, 2048]");
  SUFHIP_REQUIRE(g.walk_count >= 0 && (g.walk_count == 0 || (g.walk_jobs && g.walk_prg_state)),
                 "sufhip_layernorm2: walk_count >= 0, walk jobs and PRG state given");
  if (g.rows == 0)
    return g.walk_count > 0
               ? sufhip_trunc_prepare_batch(g.walk_prg_state, g.walk_jobs, g.walk_count, stream)
               : SUFHIP_OK;
  SUFHIP_REQUIRE((g.in_slices || (g.x[0] && g.x[1])) &&
                     (g.out[0] == nullptr) == (g.out[1] == nullptr) &&
                     (g.out[0] || g.out_planes.planes),
                 "sufhip_layernorm2: null input or output");
  SUFHIP_REQUIRE(!g.in_slices || (g.in_slice_count >= 2 && g.in_slice_count <= kLnMaxSlices),
                 "sufhip_layernorm2: in_slice_count in [2, 8]");
  SUFHIP_REQUIRE(!g.in_slices || g.cols <= kLnBlock * kLnMaxInPer,
                 "sufhip_layernorm2: in_slices need cols <= 1024");
  SUFHIP_REQUIRE(x_planes_ok(g.out_planes, size_t(g.rows) * size_t(g.cols)) &&
                     (!g.out_planes.planes || g.out_planes.cols == g.cols),
                 "sufhip_layernorm2: out_planes needs cols == the row length, rows and cols "
                 "multiples of 32, 16-byte alignment");
  SUFHIP_REQUIRE(triple_ok(g.sq) && triple_ok(g.norm), "sufhip_layernorm2: a triple is missing");
  SUFHIP_REQUIRE(g.rsqrt.kind == SUFHIP_CHAIN_RSQRT && g.rsqrt.n == size_t(g.rows),
                 "sufhip_layernorm2: the rsqrt chain must be RSQRT over rows elements");
  const size_t n = size_t(g.rows) * size_t(g.cols);
  LnArgs A{};
  if (int rc = make_chain_args(g.rsqrt, false, "sufhip_layernorm2 rsqrt", &A.rs)) return rc;
  if (int rc = table_epi(g.tr_mean, size_t(g.rows), "sufhip_layernorm2 tr_mean", &A.tr[kTrMean]))
    return rc;
  if (int rc = table_epi(g.tr_var[0], size_t(g.rows), "sufhip_layernorm2 tr_var", &A.tr[kTrVar0]))
    return rc;
  if (int rc = table_epi(g.tr_var[1], size_t(g.rows), "sufhip_layernorm2 tr_var", &A.tr[kTrVar1]))
    return rc;
  if (int rc = table_epi(g.tr_norm, n, "sufhip_layernorm2 tr_norm", &A.tr[kTrNorm])) return rc;
  if (g.in_slices) {
    if (int rc = make_epi(&g.tr_in, n, "sufhip_layernorm2 tr_in", &A.tr[kTrIn])) return rc;
    A.in_slices = g.in_slices;
    A.in_count = g.in_slice_count;
    A.mask[kTrIn] = g.in_mask;
  }
  A.x[0] = g.x[0];
  A.x[1] = g.x[1];
  A.rows = g.rows;
  A.cols = g.cols;
  A.inv_len = g.inv_len;
  A.eps = g.eps;
  A.mask[kTrMean] = g.mean_mask;
  A.mask[kTrVar0] = g.var_mask[0];
  A.mask[kTrVar1] = g.var_mask[1];
  A.mask[kTrNorm] = g.norm_mask;
  A.sq = g.sq;
  A.norm = g.norm;
  A.xp = g.out_planes;
  A.out[0] = g.out[0];
  A.out[1] = g.out[1];
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const int grid = g.rows < cus * 8 ? g.rows : cus * 8;
  const int per = (g.cols + kLnBlock - 1) / kLnBlock;
  const int block = per <= kLnMaxPer || A.in_slices ? kLnBlock : kLnWideBlock;
  A.row_groups = grid;
  // The walks: one workgroup per CU fits beside the rows' (the kernel's
  // registers allow one), so the CUs without a row hold one pass of them.
  // The 256-lane form for rows past 1024 elements walks nothing itself.
  size_t walk_lanes = 0;
  if (block == kLnBlock) {
    if (int rc = plan_hosted_walk(g.walk_prg_state, g.walk_jobs, g.walk_count,
                                  size_t(cus > grid ? cus - grid : 0) * size_t(block), stream,
                                  "sufhip_layernorm2 walk", A.w, &walk_lanes))
      return rc;
  } else if (g.walk_count > 0) {
    if (int rc = sufhip_trunc_prepare_batch(g.walk_prg_state, g.walk_jobs, g.walk_count, stream))
      return rc;
  }
  const size_t walk_groups = (walk_lanes + block - 1) / size_t(block);
  SUFHIP_REQUIRE(size_t(grid) + walk_groups <= 0x7fffffffu, "sufhip_layernorm2: grid too large");
  const dim3 launch(unsigned(size_t(grid) + walk_groups));
  hipStream_t s = as_stream(stream);
  auto rows512 = [&](auto per_c, auto in_c) {
    constexpr int kP = decltype(per_c)::value;
    constexpr bool kI = decltype(in_c)::value;
    if (walk_groups > 0)
      hipLaunchKernelGGL((layernorm2_kernel<kP, kI, kLnBlock, true>), launch, dim3(kLnBlock), 0,
                         s, A);
    else
      hipLaunchKernelGGL((layernorm2_kernel<kP, kI, kLnBlock, false>), launch, dim3(kLnBlock), 0,
                         s, A);
  };
  using PerOne = std::integral_constant<int, 1>;
  if (A.in_slices) {
    if (per <= 1)
      rows512(PerOne{}, std::true_type{});
    else
      rows512(std::integral_constant<int, kLnMaxInPer>{}, std::true_type{});
  } else if (per <= 1) {
    rows512(PerOne{}, std::false_type{});
  } else if (per <= kLnMaxPer) {
    rows512(std::integral_constant<int, kLnMaxPer>{}, std::false_type{});
  } else {
    hipLaunchKernelGGL((layernorm2_kernel<kLnWidePer, false, kLnWideBlock, false>), launch,
                       dim3(kLnWideBlock), 0, s, A);
  }
  return check_launch("layernorm2_kernel");
}


int sufhip_softmax2(const sufhip_softmax2_args* args, void* stream) {
  SUFHIP_REQUIRE(args != nullptr, "sufhip_softmax2: null args");
  const sufhip_softmax2_args& g = *args;
  SUFHIP_REQUIRE(g.rows >= 0, "sufhip_softmax2: rows < 0");
  SUFHIP_REQUIRE(g.max_row >= 1 && g.max_row <= kSmMaxRow,
                 "sufhip_softmax2: rows of 1..512 elements");
  SUFHIP_REQUIRE(g.pre_truncs >= 0 && g.pre_truncs <= 2, "sufhip_softmax2: pre_truncs in [0, 2]");
  SmArgs A{};
  if (int rc = make_tree_keys<kSmRounds>(g.keys, g.rounds, g.max_row, "sufhip_softmax2", &A.keys))
    return rc;
  if (g.rows == 0) return SUFHIP_OK;
  SUFHIP_REQUIRE(g.d_row_offsets && (g.rounds == 0 || g.d_round_offsets),
                 "sufhip_softmax2: null offsets");
  SUFHIP_REQUIRE(g.nexp.kind == SUFHIP_CHAIN_CUBIC && g.recip.kind == SUFHIP_CHAIN_RECIP &&
                     g.recip.n == size_t(g.rows),
                 "sufhip_softmax2: nexp must be CUBIC and recip RECIP over rows elements");
  const size_t n = g.nexp.n;
  if (int rc = make_chain_args(g.nexp, false, "sufhip_softmax2 nexp", &A.nexp)) return rc;
  SUFHIP_REQUIRE(A.nexp.plain,
                 "sufhip_softmax2: the nExp chain's triples must be plain arrays (no index, "
                 "multiplier, shift or negation; stride 1 or 3)");
  if (int rc = make_chain_args(g.recip, false, "sufhip_softmax2 recip", &A.recip)) return rc;
  if (int rc = check_operand(g.x, n, "sufhip_softmax2 x")) return rc;
  SUFHIP_REQUIRE(g.x.t[0].p[0] != nullptr, "sufhip_softmax2: empty input operand");
  for (int q = 0; q < g.pre_truncs; ++q)
    if (int rc = table_epi(g.pre[q], n, "sufhip_softmax2 pre", &A.pre_tr[q])) return rc;
  SUFHIP_REQUIRE(triple_ok(g.norm), "sufhip_softmax2: the norm triple is missing");
  if (int rc = table_epi(g.tr_norm, n, "sufhip_softmax2 tr_norm", &A.tr_norm)) return rc;
  SUFHIP_REQUIRE((g.out[0] == nullptr) == (g.out[1] == nullptr),
                 "sufhip_softmax2: out needs both parties or neither");
  SUFHIP_REQUIRE(g.out[0] || g.d_dense, "sufhip_softmax2: no output");
  SUFHIP_REQUIRE(!g.d_dense || (g.dense_a[0] && g.dense_a[1] && g.dense_cols >= g.max_row),
                 "sufhip_softmax2: the dense open needs both a shares and dense_cols >= max_row");
  A.x = g.x;
  A.pre = g.pre_truncs;
  A.pre_mask[0] = g.pre_mask[0];
  A.pre_mask[1] = g.pre_mask[1];
  A.offs = g.d_row_offsets;
  A.round_off = g.d_round_offsets;
  A.rows = g.rows;
  A.max_row = g.max_row;
  A.norm = g.norm;
  A.norm_mask = g.norm_mask;
  A.out[0] = g.out[0];
  A.out[1] = g.out[1];
  A.dense = g.d_dense;
  A.dense_a[0] = g.dense_a[0];
  A.dense_a[1] = g.dense_a[1];
  A.dense_cols = g.d_dense ? g.dense_cols : 0;
  SUFHIP_REQUIRE(!g.dense_planes.planes ||
                     (g.d_dense && kb_planes_ok(g.dense_planes, size_t(g.rows) * g.dense_cols)),
                 "sufhip_softmax2: dense_planes need d_dense and cover rows x dense_cols");
  A.dkb = g.d_dense ? g.dense_planes : sufhip_kb_planes{};
  const size_t row_bytes = tree_row_words(g.max_row) * sizeof(uint64_t);
  const int waves = kSmWaves;
  const size_t dyn = size_t(waves) * row_bytes;
  SUFHIP_REQUIRE(sizeof(SmStatic) + dyn <= kSmLdsCap,
                 "sufhip_softmax2: rows too long for the workgroup's LDS");
  A.waves = waves;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const int per_cu = int(kSmLdsCap / (sizeof(SmStatic) + dyn));
  const int groups = (g.rows + waves - 1) / waves;
  const int grid = groups < cus * per_cu ? groups : cus * per_cu;
  const dim3 block(kSmThreads);
  hipStream_t s = as_stream(stream);
  if (g.max_row <= kSmTeamMaxRow) {
    SUFHIP_REQUIRE(kSmTeamStatic + dyn <= kSmLdsCap && sm_team_lds_allowed(),
                   "sufhip_softmax2: the kernel's LDS size was refused");
    hipLaunchKernelGGL(softmax2_team_kernel, dim3(grid), dim3(kSmTeamThreads), dyn, s, A);
    return check_launch("softmax2_team_kernel");
  }
  const bool lds_ok = g.max_row <= 128   ? sm_lds_allowed<2>()
                      : g.max_row <= 256 ? sm_lds_allowed<4>()
                                         : sm_lds_allowed<8>();
  SUFHIP_REQUIRE(lds_ok, "sufhip_softmax2: the kernel's LDS size was refused");
  if (g.max_row <= 128)
    hipLaunchKernelGGL(softmax2_kernel<2>, dim3(grid), block, dyn, s, A);
  else if (g.max_row <= 256)
    hipLaunchKernelGGL(softmax2_kernel<4>, dim3(grid), block, dyn, s, A);
  else
    hipLaunchKernelGGL(softmax2_kernel<8>, dim3(grid), block, dyn, s, A);
  return check_launch("softmax2_kernel");
}

}  // extern "C"
