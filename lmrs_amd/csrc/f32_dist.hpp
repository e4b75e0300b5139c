// f32_dist.hpp -- f32 rows in two passes over the row.
//
// One workgroup of kThreads owns one row.
//
// Pass 1 streams the row once.  Every processed logit y goes to one of kBins
// linear bins of R - y, where R is the largest value of a first sample of the
// row (one 16-byte chunk per thread), and adds 1 to its bin's count and its
// weight 2^(y*log2(e) - R*log2(e)) to its bin's f64 mass (LDS atomics).  The
// pass also keeps the row maximum and the number of negative NaNs.
//
// The bins' prefix sums then place every decision of the selection in a few
// bins: the end of the top-k / min-p set (a partly kept bin, exact by rank or
// by key), the nucleus cut and the draw.  The cut and the draw targets depend
// on how much of a partly kept bin is kept, so each is bounded by the two
// extremes and every bin between is taken, widened by 1e-12 relative so that
// the order of the f64 sums cannot move a target across a bin edge.
//
// Pass 2 streams the row again and gathers the elements of those bins into
// LDS.  An exact sort by (value desc, index asc) and f64 prefix sums over the
// gathered elements, offset by the prefix sums of the bins before them, give
// each gathered element its rank and cumulative mass in the reference's
// sorted order (crates/sampling/src/strategies/mod.rs:21-25); the min-p cut
// (min_p.rs:45-53), the nucleus cut (top_p.rs:45-58) and softmax_choice's
// draw (strategies/mod.rs:27-55) are resolved on them.
//
// The weights differ from the reference's exp(f64(l - max)) by the common
// factor exp(R - max), which every ratio cancels, and by the rounding of the
// f32 exponent and of v_exp_f32 (a few 1e-7 relative per element at
// |y - R| ~ 10; over a cumulative sum the errors average out).  Decisions
// therefore agree with the reference wherever its uniform is more than 1e-6
// from a CDF boundary, the margin below which rows are flagged
// LMRS_ROW_NEAR_BOUNDARY.
//
// Rows that the bins cannot serve go to the generic engine in the same
// workgroup: greedy and invalid rows (one pass there), rows whose sample holds
// no finite value, rows whose maximum lies more than kDistHeadroom above R
// (the f32 weights would overflow) and rows whose gathered bins exceed the
// gather buffer.
#pragma once

#include <type_traits>

#include "generic_engine.hpp"

namespace lmrs {

constexpr int kDistUnroll = 4;              // 16-byte loads per batch (two batches in flight)
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kDistWindow = 40.0f;        // sample values further below R do not widen the bins
constexpr float kDistHeadroom = 80.0f;      // largest max - R the f32 weights hold
constexpr double kDistWiden = 1e-12;        // relative widening of every bin search target
constexpr int kDistRanges = 3;

static_assert(kBins == 64 * 32, "first_bin searches 64 x 32 bins");
static_assert(kGatherCap % kThreads == 0, "gather entries per thread");

// Bin and weight of a processed value.  Both are monotone in y (an fma, a
// clamp and a truncation), so bins hold contiguous stretches of the sorted
// order and equal values share a bin; the same code runs in both passes and
// in the finish, so every element gets the same bin and weight each time.
struct DistMap {
  float s;    // bins per unit of value
  float rs1;  // R * s + 1: values at R land in bin 1, larger ones in bin 0
  float rl;   // R * log2(e)
  __device__ __forceinline__ float t(float y) const { return __builtin_fmaf(-y, s, rs1); }
  __device__ __forceinline__ static uint32_t bin_of_t(float t) {
    return (uint32_t)fminf(fmaxf(t, 0.0f), (float)(kBins - 1));
  }
  __device__ __forceinline__ uint32_t bin(float y) const { return bin_of_t(t(y)); }
  __device__ __forceinline__ float weight(float y) const {
    return __builtin_amdgcn_exp2f(__builtin_fmaf(y, kLog2e, -rl));
  }
};

// Per-row values shared through LDS.
struct DistExtra {
  double dW[4];       // per range: row cumulative mass minus bucket cumulative mass
  uint32_t dN[4];     // the same for counts
  uint32_t ctr[2];    // dist_stream's batch counters, one per pass
  uint32_t gcount;    // gathered elements
  uint32_t generic;   // set by the finishing wave: the row goes to the generic engine
};

// The first bin b (0 .. kBins-1) for which pred(b) holds, pred monotone in b;
// kBins if none.  Wave-local (two ballots), so every wave gets the result
// without a barrier.
template <class P>
__device__ __forceinline__ uint32_t first_bin(P pred) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint64_t m = __ballot(pred(lane * 32u + 31u));
  if (m == 0) return (uint32_t)kBins;
  const uint32_t f = (uint32_t)__builtin_ctzll(m);
  const uint64_t m2 = __ballot(lane < 32u && pred(f * 32u + lane));
  return f * 32u + (uint32_t)__builtin_ctzll(m2);
}

// Streams the row: f4(x, idx, member bits) for each aligned 16-byte chunk
// (member bits: history membership of its four tokens), f1(x, idx) for the
// rest.  The chunks go out in batches of 64 * kDistUnroll (a wave's lanes
// read kDistUnroll consecutive kilobytes): wave w starts with batch w and
// takes each further batch from the counter *ctr (which starts at the number
// of waves), so that waves whose loads are served late do not hold up the
// workgroup's barrier.  Loads are software-pipelined: the next batch is in
// flight while one is processed.  `pre`, when given, is the wave's first
// batch, loaded by the caller (dist_first_batch).
template <class F4, class F1>
__device__ __forceinline__ void dist_stream(const float *p, int64_t V, bool vec, bool hist, const uint32_t *bitmap,
                                            uint32_t *ctr, const float4 *pre, F4 &&f4, F1 &&f1) {
  constexpr int U = kDistUnroll;
  constexpr int64_t BS = 64 * U;
  int64_t done = 0;
  if (vec) {
    const float4 *p4 = (const float4 *)p;
    const int64_t nch = V >> 2;
    const int64_t nb = (nch + BS - 1) / BS;
    const uint32_t lane = threadIdx.x & 63u;
    auto bits = [&](int64_t k) -> uint32_t {
      if (!hist) return 0u;
      const uint32_t i = (uint32_t)(k << 2);
      return (bitmap[i >> 5] >> (i & 31u)) & 0xFu;
    };
    // unconditional loads (chunks past the end re-read the last one): a
    // predicated load makes the compiler wait for every load in flight
    auto load = [&](float4(&d)[U], int64_t bi) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t k = bi * BS + (int64_t)u * 64 + lane;
        d[u] = p4[k < nch ? k : nch - 1];
      }
    };
    auto run = [&](const float4(&d)[U], int64_t bi) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t k = bi * BS + (int64_t)u * 64 + lane;
        if (k < nch) f4(d[u], (uint32_t)(k << 2), bits(k));
      }
    };
    auto grab = [&]() -> int64_t {
      uint32_t v = 0u;
      if (lane == 0u) v = atomicAdd(ctr, 1u);
      return (int64_t)uniform(v);
    };
    int64_t ba = threadIdx.x >> 6;
    float4 A[U], B[U];
    if (pre) {
#pragma unroll
      for (int u = 0; u < U; ++u) A[u] = pre[u];
    } else {
      load(A, ba);
    }
    while (ba < nb) {
      const int64_t bb = grab();
      load(B, bb);
      run(A, ba);
      if (bb >= nb) break;
      ba = grab();
      load(A, ba);
      run(B, bb);
    }
    done = nch << 2;
  }
  for (int64_t i = done + threadIdx.x; i < V; i += kThreads) f1(p[i], (uint32_t)i);
}

// The first batch of dist_stream for this thread's wave.
__device__ __forceinline__ void dist_first_batch(const float *p, int64_t nch, float4 (&pre)[kDistUnroll]) {
  constexpr int64_t BS = 64 * kDistUnroll;
  if (nch <= 0) return;
  const int64_t bi = threadIdx.x >> 6;
#pragma unroll
  for (int u = 0; u < kDistUnroll; ++u) {
    const int64_t k = bi * BS + (int64_t)u * 64 + (threadIdx.x & 63u);
    pre[u] = ((const float4 *)p)[k < nch ? k : nch - 1];
  }
}

// The processor chain on one f32 element; `member` is its history bit.
__device__ __forceinline__ float dist_process(float x, uint32_t idx, bool member, const RowCfg &c,
                                              const HistoryTables &ht) {
  if (member) return process_f32(x, idx, c, ht);
  return c.temp_on ? __builtin_fmaf(x, c.scale, 0.0f) : x;  // the chain off the history
}

// The chain on a chunk of four: temperature alone off the history, and, in a
// branch taken only by chunks holding history members, the full chain with
// the row's parameters read from LDS (they need not stay in registers).
__device__ __forceinline__ void dist_chunk_values(float4 d, uint32_t i0, uint32_t mb, bool temp_on, float scale,
                                                  const RowCfg &lds_cfg, const HistoryTables &ht, float (&y)[4]) {
  y[0] = d.x;
  y[1] = d.y;
  y[2] = d.z;
  y[3] = d.w;
  if (temp_on) {
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = __builtin_fmaf(y[e], scale, 0.0f);
  }
  if (mb) {
    const float xr[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if ((mb >> e) & 1u) y[e] = process_f32(xr[e], i0 + (uint32_t)e, lds_cfg, ht);
  }
}

// Up to three disjoint bin ranges [lo, lo + len), in bin order.
struct DistRanges {
  uint32_t lo0, len0, lo1, len1, lo2, len2;
  __device__ __forceinline__ int of(uint32_t b) const {
    if (b - lo0 < len0) return 0;
    if (b - lo1 < len1) return 1;
    if (b - lo2 < len2) return 2;
    return -1;
  }
  // appends [lo, hi]; lo is at or after the start of the last range
  __device__ __forceinline__ void add(uint32_t lo, uint32_t hi) {
    if (len0 == 0u) {
      lo0 = lo;
      len0 = hi - lo + 1u;
    } else if (len1 == 0u) {
      if (lo <= lo0 + len0) {  // overlaps or touches range 0
        if (hi + 1u > lo0 + len0) len0 = hi - lo0 + 1u;
      } else {
        lo1 = lo;
        len1 = hi - lo + 1u;
      }
    } else if (len2 == 0u) {
      if (lo <= lo1 + len1) {
        if (hi + 1u > lo1 + len1) len1 = hi - lo1 + 1u;
      } else {
        lo2 = lo;
        len2 = hi - lo + 1u;
      }
    } else if (hi + 1u > lo2 + len2) {  // three ranges hold every caller's union
      len2 = hi - lo2 + 1u;
    }
  }
};

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m);
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m);
  return ((uint64_t)hi << 32) | lo;
}

// Ascending bitonic sort of 64*E entries held by one wave: entry i = e*64 + lane
// is v[e].  Partners 64 or more apart are in the same lane; the others are
// exchanged with lane shuffles.  No LDS, no barrier.
template <int E>
__device__ __forceinline__ void wave_bitonic(uint64_t (&v)[E]) {
  const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
  for (int k = 2; k <= 64 * E; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= 64) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int pe = e ^ (j >> 6);
          if (pe > e) {
            const bool asc = ((((uint32_t)e << 6) | lane) & (uint32_t)k) == 0u;
            const uint64_t x = v[e], y = v[pe];
            const bool sw = (x > y) == asc;
            v[e] = sw ? y : x;
            v[pe] = sw ? x : y;
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const uint64_t pv = shfl_xor64(v[e], j);
          const bool asc = ((((uint32_t)e << 6) | lane) & (uint32_t)k) == 0u;
          const bool keep_min = ((lane & (uint32_t)j) == 0u) == asc;
          const uint64_t lo = v[e] < pv ? v[e] : pv, hi = v[e] < pv ? pv : v[e];
          v[e] = keep_min ? lo : hi;
        }
      }
    }
  }
}

// An element found in a bucket: its gathered entry, cumulative mass in the
// row's sorted order (through itself), weight and 1-based rank in the bucket.
struct DistPick {
  bool found;
  bool big;  // not resolved: the bucket holds more entries than one wave sorts
  uint64_t g;
  double c, w;
  uint32_t rank;
};

// One wave: sorts the m (<= 64*E) entries of a bucket, lst[0..m), and finds
// either the entry of rank `want` (want > 0) or the first entry of rank <= lim
// whose cumulative mass base + (prefix through it) reaches t.
template <int E>
__device__ __forceinline__ DistPick dist_resolve_e(const uint64_t *lst, uint32_t m, const DistMap &map,
                                                   uint32_t want, double base, double t, uint32_t lim) {
  const uint32_t lane = threadIdx.x & 63u;
  uint64_t v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const uint32_t i = ((uint32_t)e << 6) | lane;
    v[e] = i < m ? lst[i] : ~0ull;
  }
  wave_bitonic<E>(v);
  DistPick pk = {false, false, 0ull, 0.0, 0.0, 0u};
  double carry = 0.0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const uint32_t i = ((uint32_t)e << 6) | lane;
    const bool valid = i < m;
    const double w = valid ? (double)map.weight(key_value(~(uint32_t)(v[e] >> 32))) : 0.0;
    const double incl = carry + wave_inclusive<OpSum>(w, 0.0);
    carry = uniform(lane63(incl));
    if (!pk.found) {
      const bool hit = valid && (want ? i + 1u == want : (i < lim && base + incl >= t));
      const uint64_t bal = __ballot(hit);
      if (bal) {
        const int l = __builtin_ctzll(bal);
        pk.found = true;
        pk.g = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v[e] >> 32), l) << 32) |
               (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v[e], l);
        const uint64_t ib = (uint64_t)__double_as_longlong(incl), wb = (uint64_t)__double_as_longlong(w);
        pk.c = base + __longlong_as_double((long long)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(ib >> 32), l) << 32) |
                                                       (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)ib, l)));
        pk.w = __longlong_as_double((long long)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(wb >> 32), l) << 32) |
                                                (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)wb, l)));
        pk.rank = ((uint32_t)e << 6) + (uint32_t)l + 1u;
      }
    }
  }
  return pk;
}

// dist_resolve_e for the smallest E that holds m entries (64 < m <= 512):
// out of line, as buckets that large are rare.
__device__ __noinline__ DistPick dist_resolve_big(const uint64_t *lst, uint32_t m, DistMap map, uint32_t want,
                                                  double base, double t, uint32_t lim) {
  if (m <= 128u) return dist_resolve_e<2>(lst, m, map, want, base, t, lim);
  if (m <= 256u) return dist_resolve_e<4>(lst, m, map, want, base, t, lim);
  return dist_resolve_e<8>(lst, m, map, want, base, t, lim);
}

// As dist_resolve_e for m <= 64 entries without sorting: each lane holds one
// entry and counts the entries before it (and their mass) with broadcast
// reads of lst and of their weights in wl.
__device__ __forceinline__ DistPick dist_resolve_small(const uint64_t *lst, double *wl, uint32_t m,
                                                       const DistMap &map, uint32_t want, double base, double t,
                                                       uint32_t lim) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint64_t g = lane < m ? lst[lane] : ~0ull;
  const double w = lane < m ? (double)map.weight(key_value(~(uint32_t)(g >> 32))) : 0.0;
  if (lane < m) wl[lane] = w;
  __builtin_amdgcn_wave_barrier();
  uint32_t rank = 1u;  // 1-based
  double pre = 0.0;
  for (uint32_t j = 0u; j < m; ++j) {
    const uint64_t gj = lst[j];
    const double wj = wl[j];
    if (gj < g) {
      ++rank;
      pre += wj;
    }
  }
  const double incl = pre + w;
  const bool hit = lane < m && (want ? rank == want : (rank <= lim && base + incl >= t));
  const uint32_t best = uniform(wave_min(hit ? rank : ~0u));
  DistPick pk = {false, false, 0ull, 0.0, 0.0, 0u};
  if (best != ~0u) {
    const uint64_t bal = __ballot(hit && rank == best);
    const int l = __builtin_ctzll(bal);
    pk.found = true;
    pk.g = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(g >> 32), l) << 32) |
           (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)g, l);
    const uint64_t ib = (uint64_t)__double_as_longlong(incl), wb = (uint64_t)__double_as_longlong(w);
    pk.c = base + __longlong_as_double((long long)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(ib >> 32), l) << 32) |
                                                   (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)ib, l)));
    pk.w = __longlong_as_double((long long)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(wb >> 32), l) << 32) |
                                            (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)wb, l)));
    pk.rank = best;
  }
  return pk;
}

// One wave: copies the gathered entries of bucket X (the low 11 bits of an
// entry) to lst, in gathered order; returns their number.
__device__ __forceinline__ uint32_t dist_list(const uint64_t *gather, uint32_t n, uint32_t X, uint64_t *lst) {
  const uint32_t lane = threadIdx.x & 63u;
  uint32_t m = 0u;
#pragma unroll 4
  for (uint32_t b0 = 0u; b0 < n; b0 += 64u) {
    const uint32_t i = b0 + lane;
    const uint64_t g = i < n ? gather[i] : 0ull;
    const bool hit = i < n && ((uint32_t)g & 0x7FFu) == X;
    const uint64_t bal = __ballot(hit);
    if (hit) lst[m + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u))] = g;
    m += (uint32_t)__builtin_popcountll(bal);
  }
  __builtin_amdgcn_wave_barrier();
  return m;
}

// The row through the two passes; false when it belongs to the generic
// engine (decided uniformly across the workgroup).
template <int NT = kThreads>
__device__ __forceinline__ bool dist_row(GenericShared &sh, DistExtra &dx, const lmrs_sample_args &a, int r, int vec) {
  static_assert(NT == kThreads, "one row per workgroup of kThreads");
  using TR = DTypeTraits<LMRS_DTYPE_F32>;
  constexpr int NW = NT / 64, U = kDistUnroll;
  SelState &ss = sh.ss;
  const HistoryTables &ht = sh.ht;
  if (threadIdx.x == 0) sh.cfg = load_row_cfg(a, r, LMRS_DTYPE_F32);
  __syncthreads();
  const RowCfg c = uniform_cfg(sh.cfg);
  const int64_t V = a.vocab;
  if (c.status != LMRS_ROW_OK || V == 0 || c.greedy) {
    return false;
  }
  const float *row = (const float *)a.logits + (size_t)r * (size_t)a.row_stride;
  const bool v4 = vec != 0;
  const int64_t nch = v4 ? (V >> 2) : 0;
  const bool k_on = c.top_k > 0 && c.top_k < V;
  const bool mp_on = c.min_p >= 0.0;
  const bool p_on = c.top_p < 1.0;

  // ---- pass 1's first batch, requested before the history tables are built;
  //      its first chunk (or one element per thread) is the sample
  float4 pre[U];
  dist_first_batch(row, nch, pre);
  // the sample: chunk u = 0 of each wave's first batch
  const int64_t sk = (int64_t)(threadIdx.x >> 6) * 64 * U + (threadIdx.x & 63u);
  float4 sv = pre[0];
  int sn = sk < nch ? 4 : 0;
  if (!v4 && (int64_t)threadIdx.x < V) {
    sv.x = row[threadIdx.x];
    sn = 1;
  }
  for (int b = threadIdx.x; b < kBins; b += NT) {
    ss.bcnt[b] = 0u;
    ss.bw[b] = 0.0;
  }
  if (threadIdx.x == 0) {
    dx.gcount = 0u;
    dx.ctr[0] = NW;  // the batch counters of the two passes
    dx.ctr[1] = NW;
  }
  // a history beyond the tables: the generic engine reports the row
  if (c.hist_on && !build_history<NT>(sh.ht, a, c, V)) return false;
  uint32_t smax = 0u, smin = ~0u;
  {
    const float xs[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (e < sn) {
        const uint32_t idx = (uint32_t)(sn == 4 ? (uint32_t)sk * 4u + (uint32_t)e : threadIdx.x);
        const bool mem = c.hist_on && history_member(ht, idx);
        const float y = dist_process(xs[e], idx, mem, c, ht);
        if (__builtin_isfinite(y)) {
          const uint32_t k = order_key(y);
          smax = k > smax ? k : smax;
          smin = k < smin ? k : smin;
        }
      }
    }
  }
  smax = block_max<NW>(smax, ss.uscr);
  smin = block_min<NW>(smin, ss.uscr);
  if (smax == 0u) {  // no finite value in the sample
    return false;
  }
  DistMap map;
  {
    const float R = key_value(smax);
    const float L = fmaxf(key_value(smin), R - kDistWindow);
    float span = (R - L) * 1.25f;
    const float floor_span = fmaxf(fabsf(R), 1.0f) * 1e-3f;
    if (!(span >= floor_span)) span = floor_span;
    map.s = (float)(kBins - 2) / span;
    map.rs1 = __builtin_fmaf(R, map.s, 1.0f);
    map.rl = R * kLog2e;
  }

  // ---- pass 1: bin masses (and counts, which only the top-k rank needs),
  //      maximum, negative NaNs
  uint32_t kmax = 0u, nneg = 0u;
  const bool temp_on = c.temp_on != 0;
  const float scale = c.scale;
  // Negative NaNs are counted and add nothing to the bin their index lands
  // in (a valid one: the clamp of a NaN gives bin 0), so that no element
  // branches.
  auto put1 = [&](float y, auto kon) {
    const uint32_t key = order_key(y);
    kmax = key > kmax ? key : kmax;
    const bool nan = key < TR::kNegInfKey;
    nneg += nan ? 1u : 0u;
    const uint32_t b = map.bin(y);
    atomicAdd(&ss.bw[b], nan ? 0.0 : (double)map.weight(y));
    if constexpr (decltype(kon)::value) atomicAdd(&ss.bcnt[b], nan ? 0u : 1u);
  };
  auto pass1 = [&](auto kon) {
    dist_stream(
        row, V, v4, c.hist_on != 0, ht.bitmap, &dx.ctr[0], pre,
        [&](float4 d, uint32_t i0, uint32_t mb) {
          float y[4];
          dist_chunk_values(d, i0, mb, temp_on, scale, sh.cfg, ht, y);
#pragma unroll
          for (int e = 0; e < 4; ++e) put1(y[e], kon);
        },
        [&](float x, uint32_t i) { put1(dist_process(x, i, c.hist_on && history_member(ht, i), c, ht), kon); });
  };
  if (k_on)
    pass1(std::integral_constant<bool, true>());
  else
    pass1(std::integral_constant<bool, false>());
  kmax = block_max<NW>(kmax, ss.uscr);
  nneg = block_sum<NW>(nneg, ss.uscr);

  // ---- the row's checks, in select_row's order ----------------------------
  const float M = TR::value(kmax);
  int32_t flags = 0;
  uint32_t key_mp = 0u;
  if (mp_on) {
    const double thr = minp_threshold(M, c);
    if (!(thr == thr)) {  // softmax_choice of nothing (strategies/mod.rs:28-30)
      if (threadIdx.x == 0) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_EMPTY);
      return true;
    }
    key_mp = minp_low_key(TR::kNegInfKey, kmax, thr, [](uint32_t k) { return TR::value(k); });
    if (minp_near(TR::value(key_mp), M, thr) ||
        (key_mp > TR::kNegInfKey && minp_near(TR::value(key_mp - 1u), M, thr)))
      flags |= LMRS_ROW_NEAR_BOUNDARY;
  }
  const uint32_t ncand = k_on ? (uint32_t)c.top_k : (uint32_t)V;
  if (!__builtin_isfinite(M) || (!mp_on && nneg > 0u && ncand > (uint32_t)V - nneg)) {
    if (threadIdx.x == 0) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_DISTRIBUTION);
    return true;
  }
  if (!(M - key_value(smax) <= kDistHeadroom)) {
    return false;
  }

  // ---- inclusive prefix sums over the bins, in place ----------------------
  {
    constexpr int PB = kBins / NT;
    uint32_t cn[PB], ln = 0u;
    double cw[PB], lw = 0.0;
#pragma unroll
    for (int j = 0; j < PB; ++j) {
      cn[j] = k_on ? ss.bcnt[PB * threadIdx.x + j] : 0u;
      cw[j] = ss.bw[PB * threadIdx.x + j];
      ln += cn[j];
      lw += cw[j];
    }
    uint32_t tn;
    double tw;
    uint32_t xn = k_on ? block_exclusive_scan<NW>(ln, ss.uscr, &tn) : 0u;
    double xw = block_exclusive_scan<NW>(lw, ss.dscr, &tw);
#pragma unroll
    for (int j = 0; j < PB; ++j) {
      xn += cn[j];
      xw += cw[j];
      if (k_on) ss.bcnt[PB * threadIdx.x + j] = xn;
      ss.bw[PB * threadIdx.x + j] = xw;
    }
    __syncthreads();
  }
  const uint32_t *cN = ss.bcnt;  // top-k rows only
  const double *cW = ss.bw;
  auto Nx = [&](uint32_t b) -> uint32_t { return b ? cN[b - 1] : 0u; };
  auto Wx = [&](uint32_t b) -> double { return b ? cW[b - 1] : 0.0; };
  const double totalW = uniform(cW[kBins - 1]);
  if (!(totalW > 0.0 && __builtin_isfinite(totalW))) {
    return false;
  }
  // The first bin whose cumulative mass is positive and reaches t.  Every
  // element of a bin weighs more than any element of a later bin, so empty
  // bins never end the search and bins of zero mass lie only after the last
  // bin of positive mass.
  auto bin_ge = [&](double t) -> uint32_t {
    return uniform(first_bin([&](uint32_t b) { return cW[b] > 0.0 && cW[b] >= t; }));
  };

  // ---- where the decisions can lie ----------------------------------------
  const uint32_t b_k = k_on ? uniform(first_bin([&](uint32_t b) { return cN[b] >= (uint32_t)c.top_k; }))
                            : (uint32_t)kBins;
  const uint32_t b_mp = mp_on ? uniform(map.bin(TR::value(key_mp))) : (uint32_t)kBins;
  const uint32_t e = b_k < b_mp ? b_k : b_mp;  // the partly kept bin; kBins: everything is kept
  const uint32_t last = bin_ge(totalW);        // the last bin of positive mass
  const uint32_t e_eff = e < last ? e : last;
  double s_lo = totalW, s_hi = totalW;  // bounds on the kept mass
  if (e < (uint32_t)kBins) {
    s_lo = uniform(Wx(e));
    s_hi = uniform(cW[e]);
  }
  uint32_t c_lo = 0u, c_hi = 0u, lim = e_eff;
  double k_lo = s_lo, k_hi = s_hi;  // bounds on the mass after the nucleus cut
  if (p_on) {
    c_lo = bin_ge(c.top_p * s_lo * (1.0 - kDistWiden));
    c_hi = bin_ge(c.top_p * s_hi * (1.0 + kDistWiden));
    if (c_lo > e_eff) c_lo = e_eff;
    if (c_hi > e_eff) c_hi = e_eff;
    lim = c_hi;
    k_lo = uniform(Wx(c_lo));
    k_hi = uniform(cW[c_hi]);
  }
  uint32_t d_lo = bin_ge(c.u * k_lo * (1.0 - kDistWiden));
  uint32_t d_hi = bin_ge(c.u * k_hi * (1.0 + kDistWiden));
  if (d_lo > lim) d_lo = lim;
  if (d_hi > lim) d_hi = lim;
  // [d_lo, d_hi] ends at or before c_hi, which ends at or before e; a
  // nucleus range that starts first covers the draw range
  DistRanges rg = {0u, 0u, 0u, 0u, 0u, 0u};
  if (p_on && c_lo <= d_lo) {
    rg.add(c_lo, c_hi);
  } else {
    rg.add(d_lo, d_hi);
    if (p_on) rg.add(c_lo, c_hi);
  }
  if (e < (uint32_t)kBins) rg.add(e, e);
  const uint32_t rN0 = k_on ? uniform(Nx(rg.lo0)) : 0u, rN1 = k_on && rg.len1 ? uniform(Nx(rg.lo1)) : 0u,
                 rN2 = k_on && rg.len2 ? uniform(Nx(rg.lo2)) : 0u;
  const double rW0 = uniform(Wx(rg.lo0)), rW1 = rg.len1 ? uniform(Wx(rg.lo1)) : 0.0,
               rW2 = rg.len2 ? uniform(Wx(rg.lo2)) : 0.0;
  const bool k_part = k_on && b_k == e, mp_part = mp_on && b_mp == e;
  if (k_on) {
    uint32_t ng = uniform(cN[rg.lo0 + rg.len0 - 1u]) - rN0;
    if (rg.len1) ng += uniform(cN[rg.lo1 + rg.len1 - 1u]) - rN1;
    if (rg.len2) ng += uniform(cN[rg.lo2 + rg.len2 - 1u]) - rN2;
    if (ng > (uint32_t)kGatherCap) {
      return false;
    }
  }

  // ---- sub-buckets: each range bin splits into 2^lsh buckets of (R - y), so
  //      that the ranges' buckets, numbered in bin order, fill at most kBins
  const uint32_t off1 = rg.len0, off2 = rg.len0 + rg.len1, nbr = off2 + rg.len2;
  uint32_t lsh = 0u;
  while (lsh < 10u && (nbr << (lsh + 1u)) <= (uint32_t)kBins) ++lsh;
  const float fsub = (float)(1u << lsh);
  const uint32_t nbk = nbr << lsh;
  uint32_t *bkN = ss.bcnt;  // the bins' prefix sums are no longer read
  double *bkW = ss.bw;
  __syncthreads();
  for (int b = threadIdx.x; b < kBins; b += NT) {
    bkN[b] = 0u;
    bkW[b] = 0.0;
  }
  __syncthreads();

  // ---- pass 2: gather the elements of the ranges, with their bucket's count
  //      and mass ----------------------------------------------------------
  auto gather1 = [&](float y, uint32_t key, float tb, uint32_t b, uint32_t idx) {
    const int rr = rg.of(b);
    const uint32_t lb = rr == 0 ? b - rg.lo0 : (rr == 1 ? b - rg.lo1 + off1 : b - rg.lo2 + off2);
    const uint32_t sub = (uint32_t)fminf(fmaxf((tb - (float)b) * fsub, 0.0f), fsub - 1.0f);
    const uint32_t bk = (lb << lsh) | sub;
    const uint32_t s = atomicAdd(&dx.gcount, 1u);
    if (s < (uint32_t)kGatherCap) ss.gather[s] = ((uint64_t)(~key) << 32) | ((uint64_t)idx << 11) | bk;
    atomicAdd(&bkN[bk], 1u);
    atomicAdd(&bkW[bk], (double)map.weight(y));
  };
  // branch-free (bitwise, not short-circuit): evaluated for every element
  const uint32_t q_lo0 = rg.lo0, q_len0 = rg.len0, q_lo1 = rg.lo1, q_len1 = rg.len1, q_lo2 = rg.lo2,
                 q_len2 = rg.len2;
  auto in_ranges = [=](uint32_t key, uint32_t b) -> bool {
    return (key >= TR::kNegInfKey) & ((b - q_lo0 < q_len0) | (b - q_lo1 < q_len1) | (b - q_lo2 < q_len2));
  };
  dist_stream(
      row, V, v4, c.hist_on != 0, ht.bitmap, &dx.ctr[1], nullptr,
      [&](float4 d, uint32_t i0, uint32_t mb) {
        float y[4], tb[4];
        uint32_t key[4], b[4];
        bool in[4], any = false;
        dist_chunk_values(d, i0, mb, temp_on, scale, sh.cfg, ht, y);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          key[e] = order_key(y[e]);
          tb[e] = map.t(y[e]);
          b[e] = DistMap::bin_of_t(tb[e]);
          in[e] = in_ranges(key[e], b[e]);
          any |= in[e];
        }
        if (any) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (in[e]) gather1(y[e], key[e], tb[e], b[e], i0 + (uint32_t)e);
        }
      },
      [&](float x, uint32_t i) {
        const float y = dist_process(x, i, c.hist_on && history_member(ht, i), c, ht);
        const uint32_t key = order_key(y);
        const float tb = map.t(y);
        const uint32_t b = DistMap::bin_of_t(tb);
        if (in_ranges(key, b)) gather1(y, key, tb, b, i);
      });
  __syncthreads();
  const uint32_t n = uniform(dx.gcount);
  if (n > (uint32_t)kGatherCap) {  // bins too coarse for this row
    return false;
  }
  // inclusive prefix sums over the buckets, in place
  {
    constexpr int PB = kBins / NT;
    uint32_t cn[PB], ln = 0u;
    double cw[PB], lw = 0.0;
#pragma unroll
    for (int j = 0; j < PB; ++j) {
      cn[j] = bkN[PB * threadIdx.x + j];
      cw[j] = bkW[PB * threadIdx.x + j];
      ln += cn[j];
      lw += cw[j];
    }
    uint32_t tn;
    double tw;
    uint32_t xn = block_exclusive_scan<NW>(ln, ss.uscr, &tn);
    double xw = block_exclusive_scan<NW>(lw, ss.dscr, &tw);
#pragma unroll
    for (int j = 0; j < PB; ++j) {
      xn += cn[j];
      xw += cw[j];
      bkN[PB * threadIdx.x + j] = xn;
      bkW[PB * threadIdx.x + j] = xw;
    }
    if (threadIdx.x == 0) dx.generic = 0u;
    __syncthreads();
  }

  // ---- one wave resolves the row; the others wait at the barrier below ----
  if (threadIdx.x < 64u) {
    // the history tables are no longer read: their slots hold the two lists
    uint64_t *const lst = (uint64_t *)sh.ht.slots;
    double *const wl = (double *)(sh.ht.slots + kHashCap / 2);
    const uint64_t *const gat = ss.gather;
    const uint32_t fb1 = off1 << lsh, fb2 = off2 << lsh;
    // row cumulative = bucket cumulative + the range's offset, from a table
    // in LDS.  (A selection among locals captured by the lambdas below would
    // put them in scratch memory.)
    double *const tW = dx.dW;
    uint32_t *const tN = dx.dN;
    if ((threadIdx.x & 63u) == 0u) {
      tW[0] = rW0;
      tW[1] = rW1 - (fb1 ? bkW[fb1 - 1u] : 0.0);
      tW[2] = rW2 - (fb2 ? bkW[fb2 - 1u] : 0.0);
      tN[0] = rN0;
      tN[1] = rN1 - (fb1 ? bkN[fb1 - 1u] : 0u);
      tN[2] = rN2 - (fb2 ? bkN[fb2 - 1u] : 0u);
    }
    __builtin_amdgcn_wave_barrier();
    auto rng = [=](uint32_t bk) -> uint32_t { return bk < fb1 ? 0u : (bk < fb2 ? 1u : 2u); };
    auto rowW_incl = [=](uint32_t bk) -> double { return tW[rng(bk)] + bkW[bk]; };
    auto rowW_excl = [=](uint32_t bk) -> double { return tW[rng(bk)] + (bk ? bkW[bk - 1u] : 0.0); };
    auto rowN_incl = [=](uint32_t bk) -> uint32_t { return tN[rng(bk)] + bkN[bk]; };
    auto rowN_excl = [=](uint32_t bk) -> uint32_t { return tN[rng(bk)] + (bk ? bkN[bk - 1u] : 0u); };
    auto count_of = [=](uint32_t bk) -> uint32_t { return bkN[bk] - (bk ? bkN[bk - 1u] : 0u); };
    // the first non-empty bucket whose row cumulative reaches t (nbk: none)
    auto bucket_ge = [=](double t) -> uint32_t {
      return uniform(first_bin([=](uint32_t bk) { return bk >= nbk || (bkN[bk] > 0u && rowW_incl(bk) >= t); }));
    };
    // Resolves bucket X (big: it holds more entries than one wave sorts)
    auto resolve = [=](uint32_t X, uint32_t want, double t, uint32_t lim) -> DistPick {
      DistPick none = {false, false, 0ull, 0.0, 0.0, 0u};
      if (X >= nbk) return none;
      const uint32_t m = uniform(count_of(X));
      if (m == 0u || m > 512u || dist_list(gat, n, X, lst) != m) {
        none.big = true;
        return none;
      }
      const double base = uniform(rowW_excl(X));
      if (m <= 64u) return dist_resolve_small(lst, wl, m, map, want, base, t, lim);
      return dist_resolve_big(lst, m, map, want, base, t, lim);
    };
    bool generic = false;

    // the end of the top-k / min-p set: (bucket, number kept in it) and mass
    uint32_t end_bk = ~0u, end_n = 0u;
    double s_kept = totalW;
    if (e < (uint32_t)kBins) {
      if (k_part) {
        const uint32_t kk = (uint32_t)c.top_k;
        const uint32_t X = uniform(first_bin([=](uint32_t bk) { return bk >= nbk || rowN_incl(bk) >= kk; }));
        if (X < nbk) {
          const uint32_t want = kk - uniform(rowN_excl(X));
          const DistPick pk = resolve(X, want, 0.0, ~0u);
          if (pk.found) {
            end_bk = X;
            end_n = want;
            s_kept = pk.c;
          } else {
            generic = true;
          }
        } else {
          generic = true;
        }
      }
      if (mp_part && !generic) {
        // the min-p cut splits the bucket of its threshold value: kept are
        // the entries of that bucket with key >= key_mp, and every entry before
        const float vmp = TR::value(key_mp);
        const float tb = map.t(vmp);
        const uint32_t b = e;  // in one of the ranges
        const int rr = rg.of(b);
        const uint32_t lb = rr == 0 ? b - rg.lo0 : (rr == 1 ? b - rg.lo1 + off1 : b - rg.lo2 + off2);
        const uint32_t sub = (uint32_t)fminf(fmaxf((tb - (float)b) * fsub, 0.0f), fsub - 1.0f);
        const uint32_t Y = uniform((lb << lsh) | sub);
        uint32_t cnt = 0u;
        double ms = 0.0;
        for (uint32_t b0 = 0u; b0 < n; b0 += 64u) {
          const uint32_t i = b0 + (threadIdx.x & 63u);
          if (i < n) {
            const uint64_t g = gat[i];
            const uint32_t key = ~(uint32_t)(g >> 32);
            if (((uint32_t)g & 0x7FFu) == Y && key >= key_mp) {
              ++cnt;
              ms += (double)map.weight(key_value(key));
            }
          }
        }
        cnt = uniform(wave_sum(cnt));
        ms = uniform(wave_sum(ms));
        if (end_bk == ~0u || Y < end_bk || (Y == end_bk && cnt < end_n)) {
          end_bk = Y;
          end_n = cnt;
          s_kept = uniform(rowW_excl(Y)) + ms;
        }
      }
    }

    // the nucleus cut (top_p.rs:45-58)
    uint32_t cut_bk = end_bk, cut_n = end_n;
    double s_keep = s_kept;
    if (p_on && !generic) {
      const double t = c.top_p * s_kept;
      uint32_t Z = bucket_ge(t);
      if (end_bk != ~0u && Z > end_bk) Z = end_bk;
      const DistPick pk = resolve(Z, 0u, t, Z == end_bk ? end_n : ~0u);
      if (pk.big) generic = true;
      if (pk.found) {
        const double acc = pk.c / s_kept, prev = (pk.c - pk.w) / s_kept;
        double mg = c.top_p - prev;
        if (acc - c.top_p < mg) mg = acc - c.top_p;
        if (mg < 1e-6) flags |= LMRS_ROW_NEAR_BOUNDARY;
        cut_bk = Z;
        cut_n = pk.rank;
        s_keep = pk.c;
      } else if (!generic && (Z >= nbk || Z == end_bk)) {
        // the cumulative never reached top_p: everything is kept
        if (c.top_p - 1.0 > -1e-6) flags |= LMRS_ROW_NEAR_BOUNDARY;
      } else {
        generic = true;
      }
    }

    // the draw (strategies/mod.rs:27-55)
    if (!generic) {
      const double t = c.u * s_keep;
      uint32_t D = bucket_ge(t);
      if (cut_bk != ~0u && D > cut_bk) D = cut_bk;
      const DistPick pk = resolve(D, 0u, t, D == cut_bk ? cut_n : ~0u);
      if (!pk.found) {
        // the target lies beyond every gathered cumulative (rounding with u
        // within 1e-12 of 1): the generic engine applies softmax_choice's
        // last-candidate fallback (mod.rs:52-54) on the full row
        generic = true;
      } else if ((threadIdx.x & 63u) == 0u) {
        // margins to the CDF boundaries on either side; none before the first
        // candidate or after the last (whose cumulative is the whole mass)
        const double lo = (pk.c - pk.w) / s_keep, hi = pk.c / s_keep;
        double mg = 1.0;
        if (lo > 0.0 && fabs(c.u - lo) < mg) mg = fabs(c.u - lo);
        if (hi < 1.0 - 1e-15 && fabs(hi - c.u) < mg) mg = fabs(hi - c.u);
        const int32_t st = flags | (mg < 1e-6 ? LMRS_ROW_NEAR_BOUNDARY : 0);
        const uint32_t key = ~(uint32_t)(pk.g >> 32);
        // the kept mass against the row's maximum: the weights are
        // exp(y - R) up to f32 rounding, so divide by the maximum's (the
        // kept count is not tracked on this path)
        write_row(a, r, (uint32_t)(pk.g >> 11) & 0x3FFFFu, (float)log(pk.w / s_keep), key_value(key), st, -1,
                  s_keep / (double)map.weight(M));
      }
    }
    if (generic && (threadIdx.x & 63u) == 0u) dx.generic = 1u;
  }
  __syncthreads();
  return uniform(dx.generic) == 0u;
}

__global__ void __launch_bounds__(kThreads) f32_sample_kernel(lmrs_sample_args a, int vec) {
  __shared__ GenericShared sh;
  __shared__ DistExtra dx;
  const int r = xcd_spread_row((int)blockIdx.x, (int)gridDim.x);
  if (!dist_row(sh, dx, a, r, vec)) {
    __syncthreads();
    generic_row<LMRS_DTYPE_F32>(sh, a, r, vec);
  }
}

}  // namespace lmrs
