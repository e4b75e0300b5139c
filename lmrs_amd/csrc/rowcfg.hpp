// rowcfg.hpp -- per-row parameters, history tables and the processor chain.
//
// The processor chain is the reference's Sampler::sample loop
// (crates/sampling/src/sampler/sampler.rs:178-186) over the processors
// Repetition -> Presence/Frequency -> Temperature, each with its own skip
// rule, fused into one per-element function.  bf16 rows round after every
// op exactly as the reference's chain of bf16 kernels does; f32 rows use the
// same ops without rounding.
#pragma once

#include "lmrs_sampling.h"
#include "common.hpp"

namespace lmrs {

struct RowCfg {
  int status;          // LMRS_ROW_OK or an error code decided before sampling
  int rep_on, pres_on, temp_on, hist_on;
  int greedy;          // Greedy (top_k == LMRS_GREEDY): sorted[0], no distribution
  float pf, nf;        // repetition factors (bf16-rounded for bf16 rows)
  float presence, frequency;
  float scale;         // (float)(1.0 / T)
  int64_t top_k;       // 0 = off
  double top_p;        // >= 1.0 = off
  double min_p;        // < 0 = off
  double u;
  int64_t h_begin, h_len;
};

// History tables of the generic and f32 engines: the vocab's membership
// bitmap and a hash map token -> multiplicity (the HashMap of
// presence.rs:107-110), one 32-bit slot per token: token | count << 18
// (0 = empty; an occupied slot counts at least 1).  Any history length is
// taken; a row with more than LMRS_MAX_HISTORY_DISTINCT distinct tokens (the
// table would pass 3/4 full) or a token more than LMRS_MAX_HISTORY_COUNT
// times (the count field) gets LMRS_ROW_HISTORY.
constexpr int kHashBits = 14;
constexpr int kHashCap = 1 << kHashBits;
constexpr int kBitmapWords = LMRS_MAX_VOCAB / 32;
constexpr uint32_t kSlotTokenMask = (1u << 18) - 1u;
static_assert(LMRS_MAX_VOCAB <= (1 << 18) && LMRS_MAX_HISTORY_COUNT == (1 << 14) - 1 &&
              LMRS_MAX_HISTORY_DISTINCT * 4 <= kHashCap * 3, "slot packing and load");

struct HistoryTables {
  uint32_t slots[kHashCap];
  uint32_t bitmap[kBitmapWords];
  uint32_t distinct, overflow;
};

__device__ __forceinline__ uint32_t hash_slot(uint32_t t) {
  return (t * 2654435761u) >> (32 - kHashBits);
}

__device__ __forceinline__ uint32_t history_count(const HistoryTables &ht, uint32_t t) {
  uint32_t s = hash_slot(t);
  for (uint32_t n = 0; n < (uint32_t)kHashCap; ++n) {  // ends: the table is at most 3/4 full
    const uint32_t v = ht.slots[s];
    if (v == 0u) return 0u;
    if ((v & kSlotTokenMask) == t) return v >> 18;
    s = (s + 1u) & (kHashCap - 1);
  }
  return 0u;
}

__device__ __forceinline__ bool history_member(const HistoryTables &ht, uint32_t i) {
  return (ht.bitmap[i >> 5] >> (i & 31u)) & 1u;
}

// Every field through a scalar register (see uniform()).
__device__ inline RowCfg uniform_cfg(const RowCfg &s) {
  RowCfg c;
  c.status = uniform((int32_t)s.status);
  c.rep_on = uniform((int32_t)s.rep_on);
  c.pres_on = uniform((int32_t)s.pres_on);
  c.temp_on = uniform((int32_t)s.temp_on);
  c.hist_on = uniform((int32_t)s.hist_on);
  c.greedy = uniform((int32_t)s.greedy);
  c.pf = uniform(s.pf);
  c.nf = uniform(s.nf);
  c.presence = uniform(s.presence);
  c.frequency = uniform(s.frequency);
  c.scale = uniform(s.scale);
  c.top_k = uniform(s.top_k);
  c.top_p = uniform(s.top_p);
  c.min_p = uniform(s.min_p);
  c.u = uniform(s.u);
  c.h_begin = uniform(s.h_begin);
  c.h_len = uniform(s.h_len);
  return c;
}

// Reads and validates row r's parameters (thread 0 only).  Validation
// mirrors the constructors: RepetitionPenalty::new (repetition.rs:57-64),
// FrequencyPresencePenalty::new (presence.rs:61-71), Temperature::new
// (temperature.rs:43-50), TopP::new (top_p.rs:26-31), MinP::new
// (min_p.rs:27-29, a negative value switching the cut off); top_k below
// LMRS_GREEDY invalid.  Greedy rows carry top_k = 1 with `greedy` set.
// With strategy == false (the processor chain alone) the top-k, top-p and
// min-p fields are neither read nor checked.
// Row parameters are read through the constant address space: the arrays
// are never written while a kernel runs, so the compiler reads them with
// scalar loads, all issued together and waited for on the scalar counter,
// without waiting for the row's vector loads in flight (as vector loads they
// would be read one at a time, each behind every row load issued before it).
// A NULL array reads its neutral value from kNeutral* (no branch between the
// loads).
template <class T>
__device__ __forceinline__ T param_load(const T *p) {
  return *(const __attribute__((address_space(4))) T *)p;
}
__device__ const float kNeutralRep = 1.0f, kNeutralZeroF = 0.0f;
__device__ const double kNeutralOneD = 1.0, kNeutralMinP = -1.0, kNeutralZeroD = 0.0;
__device__ const int32_t kNeutralTopK = 0;
__device__ const int64_t kNeutralOffsets[2] = {0, 0};

__device__ inline RowCfg load_row_cfg(const lmrs_sample_args &a, int r, int dtype, bool strategy = true) {
  RowCfg c;
  c.status = LMRS_ROW_OK;
  const float rep = param_load(a.repetition_penalty ? a.repetition_penalty + r : &kNeutralRep);
  const float pres = param_load(a.presence_penalty ? a.presence_penalty + r : &kNeutralZeroF);
  const float freq = param_load(a.frequency_penalty ? a.frequency_penalty + r : &kNeutralZeroF);
  const double t = param_load(a.temperature ? a.temperature + r : &kNeutralOneD);
  const int64_t k = (int64_t)param_load(strategy && a.top_k ? a.top_k + r : &kNeutralTopK);
  const double p = param_load(strategy && a.top_p ? a.top_p + r : &kNeutralOneD);
  const double mp = param_load(strategy && a.min_p ? a.min_p + r : &kNeutralMinP);
  c.u = param_load(strategy && a.uniforms ? a.uniforms + r : &kNeutralZeroD);
  const int64_t *offs = a.hist_offsets ? a.hist_offsets + r : kNeutralOffsets;
  const int64_t h0 = param_load(offs), h1 = param_load(offs + 1);
  if (!(__builtin_isfinite(rep) && rep > 0.0f) || !__builtin_isfinite(pres) ||
      !__builtin_isfinite(freq) || !(__builtin_isfinite(t) && t > 0.0) || k < LMRS_GREEDY ||
      !(__builtin_isfinite(p) && p > 0.0 && p <= 1.0) || __builtin_isnan(mp) || mp > 1.0)
    c.status = LMRS_ROW_PARAM;
  c.h_begin = h0;
  c.h_len = h1 - h0;
  if (c.h_len < 0) c.status = LMRS_ROW_PARAM;
  const bool has_hist = c.h_len > 0;
  c.rep_on = (rep != 1.0f) && has_hist;                        // repetition.rs:82-84
  c.pres_on = has_hist && !(pres == 0.0f && freq == 0.0f);     // presence.rs:102-104
  c.temp_on = (t != 1.0);                                      // temperature.rs:68-70
  c.hist_on = c.rep_on || c.pres_on;
  float inv = 1.0f / rep;                                      // repetition.rs:88 (IEEE division)
  if (dtype == LMRS_DTYPE_BF16) {
    c.pf = round_bf16_host(inv);                               // repetition.rs:104-105
    c.nf = round_bf16_host(rep);
  } else {
    c.pf = inv;
    c.nf = rep;
  }
  c.presence = pres;
  c.frequency = freq;
  c.scale = (float)(1.0 / t);                                  // temperature.rs:71
  c.greedy = k == LMRS_GREEDY;
  c.top_k = c.greedy ? 1 : k;
  c.top_p = p;
  c.min_p = mp < 0.0 ? -1.0 : mp;
  return c;
}

// ---- the min-p cut (min_p.rs:45-53) ----------------------------------------------
// A candidate l is kept when exp(f64(l)) >= exp(f64(max)) * min_p.  exp is
// monotone, so over the sorted candidates the kept set is a prefix: NaN
// thresholds keep nothing and negative NaNs, which sort last, always fail.

__device__ __forceinline__ double minp_threshold(float max, const RowCfg &c) {
  return exp((double)max) * c.min_p;
}

__device__ __forceinline__ bool minp_keeps(float l, double thr) { return exp((double)l) >= thr; }

// Whether a logit at the cut is too close to the threshold for the host's
// and the device's exp to agree on its side (each is within an ulp or two of
// the exact value); logits equal to the maximum compare exp(max) with itself.
__device__ __forceinline__ bool minp_near(float l, float max, double thr) {
  // a zero threshold (exp(max) underflows) keeps every logit on both sides
  if (l == max || __builtin_isnan(l) || !__builtin_isfinite(thr) || !(thr > 0.0)) return false;
  const double e = exp((double)l);
  return fabs(e - thr) <= 1e-12 * thr + 1e-300;
}

// The lowest key in [lo, hi] whose value the cut keeps, given that it keeps
// value(hi) (true whenever the threshold is not NaN): a binary search over
// the total-order keys, which is where the cut lies on any candidate list.
template <class VF>
__device__ __forceinline__ uint32_t minp_low_key(uint32_t lo, uint32_t hi, double thr, VF value) {
  while (lo < hi) {
    const uint32_t mid = lo + ((hi - lo) >> 1);
    if (minp_keeps(value(mid), thr))
      hi = mid;
    else
      lo = mid + 1u;
  }
  return hi;
}

// Builds the history tables for the row (all NT threads; ends with a barrier).
template <int NT = kThreads>
__device__ inline bool build_history(HistoryTables &ht, const lmrs_sample_args &a,
                                     const RowCfg &c, int64_t vocab) {
  for (int i = threadIdx.x; i < kHashCap; i += NT) ht.slots[i] = 0u;
  const int words = (int)((vocab + 31) >> 5);
  for (int i = threadIdx.x; i < words; i += NT) ht.bitmap[i] = 0u;
  if (threadIdx.x == 0) {
    ht.distinct = 0u;
    ht.overflow = 0u;
  }
  __syncthreads();
  for (int64_t j = threadIdx.x; j < c.h_len; j += NT) {
    const uint32_t t = a.hist_ids[c.h_begin + j];
    if ((int64_t)t >= vocab) continue;  // ids outside the vocab are ignored
    atomicOr(&ht.bitmap[t >> 5], 1u << (t & 31u));
    uint32_t s = hash_slot(t);
    for (uint32_t n = 0;; ++n, s = (s + 1u) & (kHashCap - 1)) {
      if (n == (uint32_t)kHashCap) {  // full (only after the distinct limit has been passed)
        ht.overflow = 1u;
        break;
      }
      const uint32_t prev = atomicCAS(&ht.slots[s], 0u, t | (1u << 18));
      if (prev == 0u) {
        if (atomicAdd(&ht.distinct, 1u) >= (uint32_t)LMRS_MAX_HISTORY_DISTINCT) ht.overflow = 1u;
        break;
      }
      if ((prev & kSlotTokenMask) == t) {
        // a count about to leave its 14 bits is not added (the row is reported)
        uint32_t cur = prev;
        for (;;) {
          if ((cur >> 18) >= (uint32_t)LMRS_MAX_HISTORY_COUNT) {
            ht.overflow = 1u;
            break;
          }
          const uint32_t seen = atomicCAS(&ht.slots[s], cur, cur + (1u << 18));
          if (seen == cur) break;
          cur = seen;
        }
        break;
      }
    }
  }
  __syncthreads();
  return ht.overflow == 0u;
}

// The processor chain on one bf16 element (16-bit pattern in, out).
// Repetition (repetition.rs:113-116): mul by the positive / negative factor
// tensors (1.0 off the history), greater_equal(x, 0), where.  Presence
// (presence.rs:114, 123-129): sub of bf16(presence + frequency * count).
// Temperature (temperature.rs:71, tensor_ffi.cu:55-56): fma(x, s, 0).
__device__ __forceinline__ uint32_t process_bf16(uint32_t x, uint32_t idx, const RowCfg &c,
                                                 const HistoryTables &ht) {
  if (!(c.hist_on | c.temp_on)) return x;
  float v = bf16_to_f32(x);
  bool member = c.hist_on ? history_member(ht, idx) : false;
  if (c.rep_on) {
    float fp = member ? c.pf : 1.0f, fn = member ? c.nf : 1.0f;
    float pos = round_bf16_dev(v * fp), neg = round_bf16_dev(v * fn);
    v = (v >= 0.0f) ? pos : neg;
  }
  if (c.pres_on) {
    float pen = 0.0f;
    if (member) {
      float cnt = (float)history_count(ht, idx);
      pen = round_bf16_host(c.presence + c.frequency * cnt);
    }
    v = round_bf16_dev(v - pen);
  }
  if (c.temp_on) v = round_bf16_dev(__builtin_fmaf(v, c.scale, 0.0f));
  return __float_as_uint(v) >> 16;
}

// The same chain on one f32 element, without bf16 rounding.
__device__ __forceinline__ float process_f32(float v, uint32_t idx, const RowCfg &c,
                                             const HistoryTables &ht) {
  if (!(c.hist_on | c.temp_on)) return v;
  bool member = c.hist_on ? history_member(ht, idx) : false;
  if (c.rep_on) {
    float fp = member ? c.pf : 1.0f, fn = member ? c.nf : 1.0f;
    v = (v >= 0.0f) ? v * fp : v * fn;
  }
  if (c.pres_on) {
    float pen = 0.0f;
    if (member) pen = c.presence + c.frequency * (float)history_count(ht, idx);
    v = v - pen;
  }
  if (c.temp_on) v = __builtin_fmaf(v, c.scale, 0.0f);
  return v;
}

}  // namespace lmrs
