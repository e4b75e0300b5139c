// generic_engine.hpp -- the general-purpose selection engine (any dtype, any
// vocab up to LMRS_MAX_VOCAB, any parameters).
//
// One workgroup (of 1024 threads, or of the 512 threads of a fast kernel that
// hands it a row) owns one row.  The row source, StreamRow, supplies on every
// pass the total-order key of each processed element: it re-reads the row
// from memory and re-applies the processor chain.  Selection never sorts the
// row: it runs radix selections on 32-bit keys with LDS histograms
// (counts for top-k, counts plus f64 weight sums for the nucleus cut and the
// inverse-CDF draw) and resolves ties by lowest index with a radix selection
// on the index.  Small top-k candidate sets are gathered into LDS, sorted
// exactly and finished with f64 prefix sums.
//
// The order it reproduces is the reference's sorted_logits order: value
// descending under f32::total_cmp, then index ascending
// (crates/sampling/src/strategies/mod.rs:21-25).
#pragma once

#include "rowcfg.hpp"

namespace lmrs {

constexpr int kBins = 2048;        // widest radix digit: 11 bits
constexpr int kGatherCap = 4096;   // largest exactly-sorted candidate list

template <int DT>
struct DTypeTraits;

template <>
struct DTypeTraits<LMRS_DTYPE_BF16> {
  static constexpr int kElemBytes = 2;
  static constexpr int kLevels = 2;               // key bits 31..21, 20..16
  static constexpr int kWidths[3] = {11, 5, 0};
  static constexpr uint32_t kNegInfKey = 0x007F0000u;  // keys below: negative NaN
  __device__ static float value(uint32_t key) {
    uint32_t k16 = key >> 16;
    uint32_t b = (k16 & 0x8000u) ? (k16 & 0x7FFFu) : (~k16 & 0xFFFFu);
    return bf16_to_f32(b);
  }
};

template <>
struct DTypeTraits<LMRS_DTYPE_F32> {
  static constexpr int kElemBytes = 4;
  static constexpr int kLevels = 3;               // key bits 31..21, 20..10, 9..0
  static constexpr int kWidths[3] = {11, 11, 10};
  static constexpr uint32_t kNegInfKey = 0x007FFFFFu;
  __device__ static float value(uint32_t key) { return key_value(key); }
};

// LDS working set of the selection routines.
struct SelState {
  uint32_t bcnt[kBins];
  double bw[kBins];
  uint64_t gather[kGatherCap];
  double dscr[kWaves];
  uint64_t qscr[kWaves];
  uint32_t uscr[kWaves];
  int32_t iscr[kWaves];
  uint32_t sel[4];
  double dsel[4];
};

// A row streamed from global memory; every pass re-reads and re-processes it.
template <int DT, int NT_ = kThreads>
struct StreamRow {
  using TR = DTypeTraits<DT>;
  static constexpr int NT = NT_;
  const void *base;
  int64_t vocab;
  bool vec;  // 16-byte aligned rows use dwordx4 loads
  const RowCfg *cfg;
  const HistoryTables *ht;

  // Calls f(index, key) for every element, key = total-order key of the
  // processed value (bf16 keys keep only their upper 16 bits).
  template <class F>
  __device__ __forceinline__ void for_each(F &&f) const {
    const RowCfg &c = *cfg;
    if constexpr (DT == LMRS_DTYPE_BF16) {
      const uint16_t *p = (const uint16_t *)base;
      int64_t done = 0;
      if (vec) {
        const int64_t nch = vocab >> 3;
        const uint4 *p4 = (const uint4 *)p;
        for (int64_t ch = threadIdx.x; ch < nch; ch += NT) {
          uint4 d = p4[ch];
          uint32_t w[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            uint32_t raw = (w[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
            uint32_t idx = (uint32_t)(ch * 8 + e);
            uint32_t y = process_bf16(raw, idx, c, *ht);
            f(idx, order_key(bf16_to_f32(y)) & 0xFFFF0000u);
          }
        }
        done = nch << 3;
      }
      for (int64_t i = done + threadIdx.x; i < vocab; i += NT) {
        uint32_t y = process_bf16(p[i], (uint32_t)i, c, *ht);
        f((uint32_t)i, order_key(bf16_to_f32(y)) & 0xFFFF0000u);
      }
    } else {
      const float *p = (const float *)base;
      int64_t done = 0;
      if (vec) {
        const int64_t nch = vocab >> 2;
        const float4 *p4 = (const float4 *)p;
        for (int64_t ch = threadIdx.x; ch < nch; ch += NT) {
          float4 d = p4[ch];
          float w[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            uint32_t idx = (uint32_t)(ch * 4 + e);
            f(idx, order_key(process_f32(w[e], idx, c, *ht)));
          }
        }
        done = nch << 2;
      }
      for (int64_t i = done + threadIdx.x; i < vocab; i += NT)
        f((uint32_t)i, order_key(process_f32(p[i], (uint32_t)i, c, *ht)));
    }
  }
};

struct CountSel {
  uint32_t val;   // the k-th largest value
  uint32_t n_gt;  // included elements with a larger value
  uint32_t n_eq;  // included elements equal to it
};

// k-th largest of val over the included elements (1 <= k <= included count),
// by radix selection on `total_bits` bits, most significant digit first.
// vf(index, key, &val) -> bool include.
template <class Row, class VF>
__device__ __forceinline__ CountSel select_kth_largest(SelState &ss, const Row &row, VF vf, uint32_t k,
                                                       int total_bits, const int *widths, int nlev) {
  constexpr int NT = Row::NT, NW = NT / 64, P = kBins / NT;
  uint32_t prefix = 0, krem = k, ngt = 0, neq = 0;
  int fixed = 0;
  for (int lev = 0; lev < nlev; ++lev) {
    const int w = widths[lev];
    const int shift = total_bits - fixed - w;
    const uint32_t nb = 1u << w;
    for (uint32_t i = threadIdx.x; i < nb; i += NT) ss.bcnt[i] = 0u;
    __syncthreads();
    row.for_each([&](uint32_t idx, uint32_t key) {
      uint32_t val;
      if (!vf(idx, key, val)) return;
      if (fixed != 0 && (val >> (total_bits - fixed)) != prefix) return;
      atomicAdd(&ss.bcnt[(val >> shift) & (nb - 1u)], 1u);
    });
    __syncthreads();
    // Bins in descending digit order: thread t owns digits nb-1-P*t-j, j < P.
    uint32_t cj[P], sum = 0;
#pragma unroll
    for (int j = 0; j < P; ++j) {
      const int d = (int)nb - 1 - P * (int)threadIdx.x - j;
      cj[j] = d >= 0 ? ss.bcnt[d] : 0u;
      sum += cj[j];
    }
    uint32_t tot;
    uint32_t acc = block_exclusive_scan<NW>(sum, ss.uscr, &tot);
#pragma unroll
    for (int j = 0; j < P; ++j) {
      if (cj[j] > 0 && acc < krem && krem <= acc + cj[j]) {
        ss.sel[0] = (uint32_t)((int)nb - 1 - P * (int)threadIdx.x - j);
        ss.sel[1] = acc;
        ss.sel[2] = cj[j];
      }
      acc += cj[j];
    }
    __syncthreads();
    const uint32_t d = uniform(ss.sel[0]), above = uniform(ss.sel[1]);
    neq = uniform(ss.sel[2]);
    krem -= above;
    ngt += above;
    prefix = (prefix << w) | d;
    fixed += w;
    __syncthreads();
  }
  CountSel r;
  r.val = fixed < 32 ? (prefix << (total_bits - fixed)) : prefix;
  r.n_gt = ngt;
  r.n_eq = neq;
  return r;
}

struct WeightSel {
  uint32_t key;      // key of the selected token
  double above;      // kept mass strictly above `key`
  double total;      // kept mass
  uint32_t j;        // 1-based rank of the token among kept elements with `key`
  uint32_t n_kept;   // kept elements with `key`
  uint32_t n_full;   // all elements with `key`
  float w_elem;      // per-element weight at `key` (f32 exp, as accumulated)
  bool overflow;     // target beyond the accumulated total (rounding): last kept token
};

// Weighted selection: the first token, in sorted order, whose inclusive
// cumulative weight reaches frac * (kept mass).  Kept set: keys >= low_key,
// minus `clamp_excess` elements at key == clamp_key (those with the highest
// indices; their weights equal the others' at that key).
template <class Row>
__device__ __forceinline__ WeightSel select_by_weight(SelState &ss, const Row &row, double frac,
                                                      uint32_t low_key, bool clamp_on,
                                                      uint32_t clamp_key, uint32_t clamp_excess,
                                                      float M) {
  using TR = typename Row::TR;
  constexpr int NT = Row::NT, NW = NT / 64, P = kBins / NT;
  uint32_t prefix = 0;
  int fixed = 0;
  double target = 0.0, above_acc = 0.0, total = 0.0;
  WeightSel r;
  r.overflow = false;
  uint32_t sel_n = 0;
  for (int lev = 0; lev < TR::kLevels; ++lev) {
    const int w = TR::kWidths[lev];
    const int shift = 32 - fixed - w;
    const uint32_t nb = 1u << w;
    for (uint32_t i = threadIdx.x; i < nb; i += NT) {
      ss.bcnt[i] = 0u;
      ss.bw[i] = 0.0;
    }
    __syncthreads();
    row.for_each([&](uint32_t idx, uint32_t key) {
      (void)idx;
      if (key < low_key) return;
      if (fixed != 0 && (key >> (32 - fixed)) != prefix) return;
      const uint32_t d = (key >> shift) & (nb - 1u);
      atomicAdd(&ss.bcnt[d], 1u);
      atomicAdd(&ss.bw[d], (double)expf(TR::value(key) - M));
    });
    __syncthreads();
    if (threadIdx.x == 0 && clamp_on && clamp_excess > 0u &&
        (fixed == 0 || (clamp_key >> (32 - fixed)) == prefix)) {
      const uint32_t d = (clamp_key >> shift) & (nb - 1u);
      ss.bcnt[d] -= clamp_excess;
      ss.bw[d] -= (double)clamp_excess * (double)expf(TR::value(clamp_key) - M);
    }
    __syncthreads();
    // thread t owns digits nb-1-P*t-j (positions P*t+j in descending order)
    uint32_t cj[P];
    double wj[P], wsum = 0.0;
#pragma unroll
    for (int j = 0; j < P; ++j) {
      const int d = (int)nb - 1 - P * (int)threadIdx.x - j;
      cj[j] = d >= 0 ? ss.bcnt[d] : 0u;
      wj[j] = d >= 0 ? ss.bw[d] : 0.0;
      wsum += wj[j];
    }
    double tot;
    const double above_t = block_exclusive_scan<NW>(wsum, ss.dscr, &tot);
    if (lev == 0) {
      total = tot;
      target = frac * tot;
    }
    // First non-empty bin (descending) whose inclusive cumulative reaches the
    // target; last non-empty bin, for the rounding fallback.
    int pos = 0x7FFFFFFF, last = -1;
    double accw = above_t;
#pragma unroll
    for (int j = 0; j < P; ++j) {
      if (cj[j] > 0 && pos == 0x7FFFFFFF && accw + wj[j] >= target) pos = P * (int)threadIdx.x + j;
      if (cj[j] > 0) last = P * (int)threadIdx.x + j;
      accw += wj[j];
    }
    pos = block_min<NW>(pos, ss.iscr);
    last = block_max<NW>(last, ss.iscr);
    const bool ovf = pos == 0x7FFFFFFF;
    const int pick = ovf ? last : pos;
    if ((int)threadIdx.x == pick / P) {
      double accp = above_t;
#pragma unroll
      for (int j = 0; j < P; ++j) {
        if (P * (int)threadIdx.x + j == pick) {
          ss.sel[0] = (uint32_t)((int)nb - 1 - pick);
          ss.sel[1] = cj[j];
          ss.dsel[0] = accp;
          ss.dsel[1] = wj[j];
        }
        accp += wj[j];
      }
    }
    __syncthreads();
    const uint32_t d = uniform(ss.sel[0]);
    sel_n = uniform(ss.sel[1]);
    const double above = uniform(ss.dsel[0]);
    if (ovf) {
      r.overflow = true;
      target = above + uniform(ss.dsel[1]);  // lands on the bin's last element
    }
    target -= above;
    above_acc += above;
    prefix = (prefix << w) | d;
    fixed += w;
    __syncthreads();
  }
  r.key = fixed < 32 ? (prefix << (32 - fixed)) : prefix;
  r.above = above_acc;
  r.total = total;
  r.n_kept = sel_n;
  r.n_full = sel_n + ((clamp_on && r.key == clamp_key) ? clamp_excess : 0u);
  r.w_elem = expf(TR::value(r.key) - M);
  double jj = r.w_elem > 0.0f ? ceil(target / (double)r.w_elem) : 1.0;
  if (!(jj >= 1.0)) jj = 1.0;
  if (jj > (double)sel_n) jj = (double)sel_n;
  r.j = (uint32_t)jj;
  return r;
}

// Writes one row's outputs (thread 0 only).
// One row's outputs.  kept / mass: the post-filter distribution's size and
// sum of exp(l - max) (lmrs_sample_args::kept_count, kept_mass); a failed row
// writes 0 and 0; a sampled row whose path does not pass them writes -1
// ("not reported", which the tests count).
__device__ __forceinline__ void write_row(const lmrs_sample_args &a, int r, uint32_t token,
                                          float log_prob, float logit, int32_t status,
                                          int32_t kept = -1, double mass = 0.0) {
  a.token_ids[r] = token;
  if (a.log_probs) a.log_probs[r] = log_prob;
  if (a.logits_out) a.logits_out[r] = logit;
  if (a.status) a.status[r] = status;
  const bool failed = (status & 0xFF) != LMRS_ROW_OK;
  if (a.kept_count) a.kept_count[r] = failed ? 0 : kept;
  if (a.kept_mass) a.kept_mass[r] = failed ? 0.0 : mass;
}

// Sorts ss.gather[0..n) ascending (bitonic; n <= kGatherCap).  Barriers inside.
template <int NT = kThreads>
__device__ __forceinline__ void sort_gather(SelState &ss, uint32_t n) {
  uint32_t n2 = 1;
  while (n2 < n) n2 <<= 1;
  for (uint32_t i = n + threadIdx.x; i < n2; i += NT) ss.gather[i] = ~0ull;
  __syncthreads();
  for (uint32_t kk = 2; kk <= n2; kk <<= 1) {
    for (uint32_t jj = kk >> 1; jj > 0; jj >>= 1) {
      for (uint32_t i = threadIdx.x; i < n2; i += NT) {
        const uint32_t ixj = i ^ jj;
        if (ixj > i) {
          const uint64_t x = ss.gather[i], y = ss.gather[ixj];
          const bool asc = (i & kk) == 0;
          if ((x > y) == asc) {
            ss.gather[i] = y;
            ss.gather[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Finishes a row from its sorted candidate list: ss.gather[0..k) holds
// ((~key) << 32 | index) in ascending order, i.e. the reference's sorted
// order.  Applies the min-p cut (min_p.rs:45-53), the nucleus cut
// (top_p.rs:45-58) and softmax_choice
// (strategies/mod.rs:27-55) with f64 weights exp(f64(l - max)) and f64
// prefix sums, and writes the outputs.
template <class TR, int NT = kThreads>
__device__ __forceinline__ void finish_sorted(SelState &ss, const RowCfg &c, const lmrs_sample_args &a,
                                              int r, uint32_t k) {
  // Thread t owns sorted entries P*t .. P*t+P-1 of the first k.
  constexpr int P = kGatherCap / NT, NW = NT / 64;
  const float M = TR::value(~uniform((uint32_t)(ss.gather[0] >> 32)));
  if (c.greedy) {  // Greedy (greedy.rs:22-29): the first sorted candidate, no distribution
    if (threadIdx.x == 0) write_row(a, r, (uint32_t)(ss.gather[0] & 0xFFFFFFFFu), 0.0f, M, LMRS_ROW_OK, 1, 1.0);
    return;
  }
  int32_t flags = 0;
  if (c.min_p >= 0.0) {  // the min-p cut (min_p.rs:45-53): a prefix of the k candidates
    const double thr = minp_threshold(M, c);
    uint32_t nk = 0u;
#pragma unroll
    for (int q = 0; q < P; ++q) {
      const uint32_t i = (uint32_t)P * threadIdx.x + (uint32_t)q;
      if (i < k && minp_keeps(TR::value(~(uint32_t)(ss.gather[i] >> 32)), thr)) ++nk;
    }
    nk = block_sum<NW>(nk, ss.uscr);
    if (nk == 0u) {  // softmax_choice of nothing (strategies/mod.rs:28-30)
      if (threadIdx.x == 0) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_EMPTY);
      return;
    }
    int32_t near = 0;
#pragma unroll
    for (int q = 0; q < P; ++q) {
      const uint32_t i = (uint32_t)P * threadIdx.x + (uint32_t)q;
      if ((i + 1u == nk || (i == nk && i < k)) &&
          minp_near(TR::value(~(uint32_t)(ss.gather[i] >> 32)), M, thr))
        near = 1;
    }
    if (block_max<NW>(near, ss.iscr)) flags |= LMRS_ROW_NEAR_BOUNDARY;
    k = nk;
  }
  double wv[P], incl[P], local = 0.0;
#pragma unroll
  for (int q = 0; q < P; ++q) {
    const uint32_t i = (uint32_t)P * threadIdx.x + (uint32_t)q;
    wv[q] = 0.0;
    if (i < k) {
      const float y = TR::value(~(uint32_t)(ss.gather[i] >> 32));
      wv[q] = exp((double)(y - M));
    }
    local += wv[q];
    incl[q] = local;
  }
  double sum_all;
  const double excl = block_exclusive_scan<NW>(local, ss.dscr, &sum_all);
#pragma unroll
  for (int q = 0; q < P; ++q) incl[q] += excl;
  if (!(__builtin_isfinite(sum_all) && sum_all > 0.0)) {
    if (threadIdx.x == 0) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_DISTRIBUTION);
    return;
  }
  uint32_t keep = k;
  if (c.top_p < 1.0) {
    int first = 0x7FFFFFFF;
#pragma unroll
    for (int q = P - 1; q >= 0; --q) {
      const uint32_t i = (uint32_t)P * threadIdx.x + (uint32_t)q;
      if (i < k && incl[q] / sum_all >= c.top_p) first = (int)i;
    }
    first = block_min<NW>(first, ss.iscr);
    if (first != 0x7FFFFFFF) keep = (uint32_t)first + 1u;
    // nucleus margin at the cut
#pragma unroll
    for (int q = 0; q < P; ++q) {
      const uint32_t i = (uint32_t)P * threadIdx.x + (uint32_t)q;
      if (i + 1u == keep) {
        const double acc = incl[q] / sum_all, prev = (incl[q] - wv[q]) / sum_all;
        double m = c.top_p - prev;
        if (acc >= c.top_p && acc - c.top_p < m) m = acc - c.top_p;
        if (!(acc >= c.top_p)) m = c.top_p - acc;
        ss.dsel[2] = m;
      }
    }
    __syncthreads();
    if (uniform(ss.dsel[2]) < 1e-6) flags |= LMRS_ROW_NEAR_BOUNDARY;
  }
  // sum over the kept prefix, held by the owner of entry keep-1
#pragma unroll
  for (int q = 0; q < P; ++q)
    if ((uint32_t)P * threadIdx.x + (uint32_t)q + 1u == keep) ss.dsel[3] = incl[q];
  __syncthreads();
  const double sum_keep = uniform(ss.dsel[3]);
  const double target = c.u * sum_keep;
  int pick = 0x7FFFFFFF;
#pragma unroll
  for (int q = P - 1; q >= 0; --q) {
    const uint32_t i = (uint32_t)P * threadIdx.x + (uint32_t)q;
    if (i < keep && target <= incl[q]) pick = (int)i;
  }
  pick = block_min<NW>(pick, ss.iscr);
  if (pick == 0x7FFFFFFF) pick = (int)keep - 1;  // fallback: last candidate (mod.rs:52-54)
#pragma unroll
  for (int q = 0; q < P; ++q) {
    const uint32_t i = (uint32_t)P * threadIdx.x + (uint32_t)q;
    if ((int)i == pick) {
      const uint64_t g = ss.gather[i];
      const uint32_t token = (uint32_t)(g & 0xFFFFFFFFu);
      const float y = TR::value(~(uint32_t)(g >> 32));
      const double lo = (incl[q] - wv[q]) / sum_keep, hi = incl[q] / sum_keep;
      double m = 1.0;
      if (i > 0 && fabs(c.u - lo) < m) m = fabs(c.u - lo);
      if (i + 1u < keep && fabs(hi - c.u) < m) m = fabs(hi - c.u);
      const int32_t st = flags | (m < 1e-6 ? LMRS_ROW_NEAR_BOUNDARY : 0);
      write_row(a, r, token, (float)log(wv[q] / sum_keep), y, st, (int32_t)keep, sum_keep);
    }
  }
}

// Finishes a row whose top-k candidates (keys >= tk, n of them) fit the
// gather buffer: gather, exact sort by (key desc, index asc), finish.
template <class Row>
__device__ __forceinline__ void finish_small_k(SelState &ss, const Row &row, const RowCfg &c,
                                               const lmrs_sample_args &a, int r, uint32_t tk,
                                               uint32_t n, uint32_t k) {
  if (threadIdx.x == 0) ss.sel[3] = 0u;
  __syncthreads();
  row.for_each([&](uint32_t idx, uint32_t key) {
    if (key < tk) return;
    const uint32_t s = atomicAdd(&ss.sel[3], 1u);
    ss.gather[s] = ((uint64_t)(~key) << 32) | (uint64_t)idx;
  });
  __syncthreads();
  sort_gather<Row::NT>(ss, n);
  finish_sorted<typename Row::TR, Row::NT>(ss, c, a, r, k);
}

// The whole selection for one row from any row source: greedy, top-k,
// min-p cut, nucleus cut and draw.  kmax/imax/nneg come from the caller's stats pass.
template <class Row>
__device__ __forceinline__ void select_row(SelState &ss, const Row &row, const RowCfg &c,
                                           const lmrs_sample_args &a, int r, int64_t V,
                                           uint32_t kmax, uint32_t imax, uint32_t nneg) {
  using TR = typename Row::TR;
  const float M = TR::value(kmax);
  if (c.greedy) {  // Greedy (greedy.rs:22-29): sorted[0], log_prob 0
    if (threadIdx.x == 0) write_row(a, r, imax, 0.0f, M, LMRS_ROW_OK, 1, 1.0);
    return;
  }
  const bool k_on = c.top_k > 0 && c.top_k < V;
  const uint32_t ncand = k_on ? (uint32_t)c.top_k : (uint32_t)V;
  // The min-p cut (min_p.rs:45-53) keeps the keys >= key_mp: a NaN threshold
  // keeps nothing, and negative NaNs (keys below -inf) never pass.
  const bool mp_on = c.min_p >= 0.0;
  uint32_t key_mp = 0u;
  int32_t flags = 0;
  if (mp_on) {
    const double thr = minp_threshold(M, c);
    if (!(thr == thr)) {  // softmax_choice of nothing (strategies/mod.rs:28-30)
      if (threadIdx.x == 0) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_EMPTY);
      return;
    }
    key_mp = minp_low_key(TR::kNegInfKey, kmax, thr, [](uint32_t k) { return TR::value(k); });
    if (minp_near(TR::value(key_mp), M, thr) ||
        (key_mp > TR::kNegInfKey && minp_near(TR::value(key_mp - 1u), M, thr)))
      flags |= LMRS_ROW_NEAR_BOUNDARY;
  }
  // Weights exp(f64(l - max)) are all finite and the sum positive unless the
  // maximum is non-finite or a (negative) NaN is among the candidates.
  if (!__builtin_isfinite(M) || (!mp_on && nneg > 0u && ncand > (uint32_t)V - nneg)) {
    if (threadIdx.x == 0) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_DISTRIBUTION);
    return;
  }

  uint32_t tk = 0u, needed = 0u, neq_k = 0u;
  if (k_on) {
    const CountSel s = select_kth_largest(
        ss, row,
        [](uint32_t, uint32_t key, uint32_t &val) {
          val = key;
          return true;
        },
        (uint32_t)c.top_k, 32, TR::kWidths, TR::kLevels);
    tk = s.val;
    needed = (uint32_t)c.top_k - s.n_gt;
    neq_k = s.n_eq;
    if (s.n_gt + s.n_eq <= (uint32_t)kGatherCap) {
      finish_small_k(ss, row, c, a, r, tk, s.n_gt + s.n_eq, (uint32_t)c.top_k);
      return;
    }
  }

  // Weighted path.  Candidate set: keys > tk plus `needed` at tk (or all).
  uint32_t kept_low = k_on ? tk : 0u;
  bool kept_clamp = k_on;
  uint32_t kept_ckey = tk, kept_excess = k_on ? neq_k - needed : 0u;
  if (mp_on && (!k_on || key_mp > tk)) {  // the min-p cut ends above the top-k set's lowest key
    kept_low = key_mp;
    kept_clamp = false;
    kept_excess = 0u;
  }
  if (c.top_p < 1.0) {
    const WeightSel p =
        select_by_weight(ss, row, c.top_p, kept_low, kept_clamp, kept_ckey, kept_excess, M);
    const double denom = p.total;
    if (p.overflow) {
      // the nucleus cumulative never reached top_p: everything is kept
      if (c.top_p - 1.0 > -1e-6) flags |= LMRS_ROW_NEAR_BOUNDARY;
    } else {
      const double kept_mass = p.above + (double)p.j * (double)p.w_elem;
      const double acc = kept_mass / denom, prev = (kept_mass - (double)p.w_elem) / denom;
      double m = c.top_p - prev;
      if (acc - c.top_p < m) m = acc - c.top_p;
      if (m < 1e-6) flags |= LMRS_ROW_NEAR_BOUNDARY;
      kept_low = p.key;
      kept_clamp = true;
      kept_ckey = p.key;
      kept_excess = p.n_full - p.j;
    }
  }
  const WeightSel d = select_by_weight(ss, row, c.u, kept_low, kept_clamp, kept_ckey, kept_excess, M);
  // The d.j-th lowest index among elements with key d.key.
  const uint32_t want = d.key;
  const int idx_w[2] = {11, 7};
  const CountSel s = select_kth_largest(
      ss, row,
      [want](uint32_t idx, uint32_t key, uint32_t &val) {
        val = 0x3FFFFu - idx;
        return key == want;
      },
      d.j, 18, idx_w, 2);
  if (threadIdx.x == 0) {
    const uint32_t token = 0x3FFFFu - s.val;
    const float y = TR::value(d.key);
    const double w_exact = exp((double)(y - M));
    const double lo = (d.above + (double)(d.j - 1u) * (double)d.w_elem) / d.total;
    const double hi = lo + (double)d.w_elem / d.total;
    double m = 1.0;
    if (!(d.key == kmax && d.j == 1u) && fabs(c.u - lo) < m) m = fabs(c.u - lo);
    if (hi < 1.0 - 1e-15 && fabs(hi - c.u) < m) m = fabs(hi - c.u);
    if (d.overflow) m = 0.0;
    const int32_t st = flags | (m < 1e-6 ? LMRS_ROW_NEAR_BOUNDARY : 0);
    // (the kept count is not tracked on this path: its cuts are key thresholds)
    write_row(a, r, token, (float)log(w_exact / d.total), y, st, -1, d.total);
  }
}

// Stats pass: maximum key (total order), lowest index at the maximum, and the
// number of negative NaNs (which sort below -inf).
template <class Row>
__device__ __forceinline__ void row_stats(SelState &ss, const Row &row, uint32_t &kmax,
                                          uint32_t &imax, uint32_t &nneg) {
  using TR = typename Row::TR;
  uint64_t best = 0;
  uint32_t neg = 0;
  row.for_each([&](uint32_t idx, uint32_t key) {
    const uint64_t pk = ((uint64_t)key << 32) | (uint64_t)(~idx);
    best = pk > best ? pk : best;
    neg += key < TR::kNegInfKey ? 1u : 0u;
  });
  best = block_max<Row::NT / 64>(best, ss.qscr);
  nneg = block_sum<Row::NT / 64>(neg, ss.uscr);
  kmax = (uint32_t)(best >> 32);
  imax = ~(uint32_t)(best & 0xFFFFFFFFu);
}

struct GenericShared {
  HistoryTables ht;
  SelState ss;
  RowCfg cfg;
};

// One row through the generic engine (all NT threads of the workgroup).
template <int DT, int NT = kThreads>
__device__ __forceinline__ void generic_row(GenericShared &sh, const lmrs_sample_args &a, int r, int vec) {
  using TR = DTypeTraits<DT>;
  if (threadIdx.x == 0) sh.cfg = load_row_cfg(a, r, DT);
  __syncthreads();
  const RowCfg c = uniform_cfg(sh.cfg);
  const int64_t V = a.vocab;
  if (c.status != LMRS_ROW_OK || V == 0) {
    if (threadIdx.x == 0)
      write_row(a, r, 0u, 0.0f, 0.0f, c.status != LMRS_ROW_OK ? c.status : LMRS_ROW_EMPTY);
    return;
  }
  if (c.hist_on && !build_history<NT>(sh.ht, a, c, V)) {  // the history exceeds the tables
    if (threadIdx.x == 0) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_HISTORY);
    return;
  }
  StreamRow<DT, NT> row;
  row.base = (const char *)a.logits + (size_t)r * (size_t)a.row_stride * TR::kElemBytes;
  row.vocab = V;
  row.vec = vec != 0;
  row.cfg = &sh.cfg;
  row.ht = &sh.ht;
  uint32_t kmax, imax, nneg;
  row_stats(sh.ss, row, kmax, imax, nneg);
  select_row(sh.ss, row, c, a, r, V, kmax, imax, nneg);
}

template <int DT>
__global__ void __launch_bounds__(kThreads) generic_sample_kernel(lmrs_sample_args a, int vec) {
  __shared__ GenericShared sh;
  generic_row<DT>(sh, a, xcd_spread_row((int)blockIdx.x, (int)gridDim.x), vec);
}

// LogitsProcessor::process for the three reference processors, batched.
template <int DT>
__global__ void __launch_bounds__(kThreads) process_kernel(lmrs_sample_args a, void *out) {
  using TR = DTypeTraits<DT>;
  __shared__ HistoryTables ht;
  __shared__ RowCfg cfg;
  const int r = blockIdx.x;
  if (threadIdx.x == 0) cfg = load_row_cfg(a, r, DT, false);
  __syncthreads();
  RowCfg c = cfg;
  const int64_t V = a.vocab;
  if (c.status != LMRS_ROW_OK) {  // invalid rows are copied unchanged
    c.hist_on = c.rep_on = c.pres_on = c.temp_on = 0;
  }
  if (c.hist_on && !build_history(ht, a, c, V)) {  // the history exceeds the tables: copied unchanged
    c.status = LMRS_ROW_HISTORY;
    c.hist_on = c.rep_on = c.pres_on = c.temp_on = 0;
  }
  if (threadIdx.x == 0 && a.status) a.status[r] = c.status;
  const char *src = (const char *)a.logits + (size_t)r * (size_t)a.row_stride * TR::kElemBytes;
  char *dst = (char *)out + (size_t)r * (size_t)V * TR::kElemBytes;
  for (int64_t i = threadIdx.x; i < V; i += kThreads) {
    if constexpr (DT == LMRS_DTYPE_BF16) {
      ((uint16_t *)dst)[i] = (uint16_t)process_bf16(((const uint16_t *)src)[i], (uint32_t)i, c, ht);
    } else {
      ((float *)dst)[i] = process_f32(((const float *)src)[i], (uint32_t)i, c, ht);
    }
  }
}

}  // namespace lmrs
