/*
 * lmrs_oracle.h -- CPU restatement of lmrs's token-sampling path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP
 * sampler is compared against (parity tests, smoke check, and the CPU
 * baseline leg of bench.py).  No product code path may link, load or call
 * it; the product fails loudly when its HIP library is missing.
 *
 * Every function restates one piece of the reference (Rust crate
 * `crates/sampling` plus the CUDA elementwise kernels it drives); the
 * citation of the reference file:line sits beside each declaration.
 *
 * Parity pinning (how each function is checked, all in tests/):
 *   bf16 rounding ......... exhaustive f32 sweeps against torch.bfloat16 (RNE)
 *   next_unit ............. hand-computed 128-bit integer recurrence (Python ints)
 *   total order / sort .... brute force vs Python struct-level key + index
 *   strategies ............ reference doctest vectors, brute-force inverse CDF
 *                            at interval midpoints, chi-square of draws
 *   processors ............ reference doctest vectors, exhaustive 65536-input
 *                            sweeps against numpy f32 + torch bf16 arithmetic
 *   composition ........... reduces to each single reference strategy
 *                            (TopK / TopP / MinP / Greedy / full draw) when
 *                            the other filters are off
 */
#ifndef LMRS_ORACLE_H
#define LMRS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes (mirror SamplingError::Invalid, crates/sampling/src/error.rs:20-39). */
#define LMRS_ORACLE_OK 0
#define LMRS_ORACLE_ERR_EMPTY 1        /* "cannot sample from empty logits" */
#define LMRS_ORACLE_ERR_DISTRIBUTION 2 /* "logits produced an invalid probability distribution" */
#define LMRS_ORACLE_ERR_PARAM 3        /* a constructor's validation failed */

/* Mirrors SampleOutput {token_id:u32, log_prob:f32, logit:f32}
 * (crates/sampling/src/sampler/output.rs:14-18). */
typedef struct {
  uint32_t token_id;
  float log_prob;
  float logit;
} lmrs_oracle_output;

/* ---- scalar primitives ------------------------------------------------- */

/* IEEE f32 -> bf16, round to nearest even; NaN keeps its sign and upper
 * payload with the quiet bit set.  Host side factors are built this way
 * (half::bf16::from_f32, crates/sampling/src/logits/repetition.rs:104-106). */
uint16_t lmrs_oracle_bf16_from_f32_host(float x);
/* Device side conversion used by every elementwise kernel's store
 * (kernels/ops/activation_kernels.cuh:35-38): round to nearest even, NaN
 * becomes the canonical 0x7FFF. */
uint16_t lmrs_oracle_bf16_from_f32_dev(float x);
float lmrs_oracle_f32_from_bf16(uint16_t b); /* exact widening (cast_ffi.cu:8-13) */

/* Reference LCG: crates/sampling/src/strategies/mod.rs:57-61. */
double lmrs_oracle_next_unit(uint64_t *state);

/* f32::total_cmp (IEEE 754 totalOrder): returns -1, 0, 1. */
int lmrs_oracle_total_cmp(float a, float b);

/* sorted_logits (strategies/mod.rs:21-25): writes the permutation of
 * 0..n-1 ordered by value descending under total_cmp, then index ascending. */
void lmrs_oracle_sorted_indices(const float *logits, int64_t n, int64_t *order);

/* ---- strategies (host f32 slice in, SampleOutput out) ------------------- */
/* Each returns an LMRS_ORACLE_* status and consumes `rng` exactly as the
 * reference does (Greedy and BeamSearch consume nothing). */
int lmrs_oracle_greedy(const float *logits, int64_t n, lmrs_oracle_output *out); /* greedy.rs:22-29 */
int lmrs_oracle_beam(const float *logits, int64_t n, int64_t width, lmrs_oracle_output *out); /* beam.rs:30-50 */
int lmrs_oracle_top_k(const float *logits, int64_t n, int64_t k, uint64_t *rng, lmrs_oracle_output *out); /* top_k.rs:26-45 */
int lmrs_oracle_top_p(const float *logits, int64_t n, double p, uint64_t *rng, lmrs_oracle_output *out); /* top_p.rs:26-61 */
int lmrs_oracle_min_p(const float *logits, int64_t n, double min_p, uint64_t *rng, lmrs_oracle_output *out); /* min_p.rs:26-55 */

/* ---- logits processors (one row, in place) ------------------------------
 * dtype 0: row holds bf16 bit patterns (uint16_t); every op rounds its f32
 *          result back to bf16 (device semantics of the reference).
 * dtype 2: row holds f32; same ops without any bf16 rounding (the f32
 *          instantiation of the same kernels).
 * Each returns LMRS_ORACLE_ERR_PARAM when the constructor would reject the
 * parameter, else LMRS_ORACLE_OK (including the documented skip cases). */
int lmrs_oracle_repetition(void *row, int dtype, int64_t n, float penalty,
                           const uint32_t *history, int64_t h);        /* repetition.rs:57-117 */
int lmrs_oracle_presence(void *row, int dtype, int64_t n, float presence, float frequency,
                         const uint32_t *history, int64_t h);          /* presence.rs:61-130 */
int lmrs_oracle_temperature(void *row, int dtype, int64_t n, double temperature); /* temperature.rs:43-72 */

/* ---- composed per-row sampler ------------------------------------------- */
typedef struct {
  float repetition_penalty; /* 1.0 = off */
  float presence_penalty;   /* 0.0 = off (with frequency 0) */
  float frequency_penalty;
  double temperature;       /* 1.0 = off */
  int64_t top_k;            /* 0 = off, -1 = Greedy, k > 0 = TopK(k) */
  double top_p;             /* >= 1.0 = off; must be in (0, 1] */
  double min_p;             /* < 0 = off; else must be in [0, 1] */
} lmrs_oracle_params;

/* Diagnostics used to count ambiguous (boundary) rows.
 * cdf_margin: distance of u to the nearest internal boundary of the chosen
 *   token's CDF interval [lo, hi) in the kept candidate list (+inf when the
 *   chosen token is alone or the interval has no internal boundary).
 * top_p_margin: distance of the nucleus cumulative to p at the cut
 *   (min(acc_keep - p, p - acc_{keep-1})); +inf when top-p is off.
 * min_p_margin: smallest |exp(l) - threshold| / threshold over the
 *   candidates at the min-p cut with l != max (+inf when min-p is off).
 * cum_before: sum of kept weights before the chosen token, f64 in order.
 * sum_kept, weight: normaliser and chosen weight (prob = weight / sum_kept). */
typedef struct {
  double cdf_margin;
  double top_p_margin;
  double min_p_margin;
  double cum_before;
  double sum_kept;
  double weight;
  int64_t n_candidates; /* after top-k */
  int64_t n_kept;       /* after top-p */
} lmrs_oracle_diag;

/* The build's composition (Repetition -> Presence/Frequency -> Temperature,
 * then top-k cut, then min-p cut, then nucleus cut over what is left, then
 * the inverse-CDF draw with the caller's uniform u), built from reference
 * primitives:
 * processors as in Sampler::sample (sampler.rs:178-186), strategies as in
 * the strategies/ files.  top_k == -1 is Greedy (greedy.rs:22-29), which
 * ignores the other cuts; top_k == 1 is TopK(1) (top_k.rs:39-45), which
 * draws through softmax_choice and so reports an invalid distribution for a
 * row whose maximum is not finite.
 * logits: one row, dtype 0 (bf16 bits) or 2 (f32); not modified.
 * processed_out (optional, n floats): the processed row as f32. */
int lmrs_oracle_sample_row(const void *logits, int dtype, int64_t n,
                           const uint32_t *history, int64_t h,
                           const lmrs_oracle_params *params, double u,
                           lmrs_oracle_output *out, lmrs_oracle_diag *diag,
                           float *processed_out);

/* Batch driver over rows (CSR history), optionally on n_threads POSIX threads
 * (one row at a time per thread).  Per-row status in status[r].  Used for the
 * CPU baseline and for multi-row parity checks. */
int lmrs_oracle_sample_batch(const void *logits, int dtype, int64_t batch, int64_t n,
                             int64_t row_stride, const int64_t *hist_offsets,
                             const uint32_t *hist_ids, const lmrs_oracle_params *params,
                             const double *uniforms, lmrs_oracle_output *out,
                             lmrs_oracle_diag *diag, int32_t *status, int n_threads);

/* ---- the LM head's projection ---------------------------------------------
 * linear_kernel (kernels/ffi/tensor_ffi.cu:230-258) for bf16 without bias, as
 * LmHead::forward calls it (crates/ops/src/embedding/lm_head.rs:33-35):
 * y[r, v] = bf16(acc), acc = 0.0f then acc += f32(x[r, k]) * f32(w[v, k]) for
 * k = 0 .. in-1 in order (each product of two bf16 is exact in f32, so nvcc's
 * contraction to an fma rounds the same), bf16 round to nearest even
 * (from_float, activation_kernels.cuh:35-38).  Also returns, when sum_abs is
 * not NULL, sum_k |x w| per output (for error bounds). */
void lmrs_oracle_linear_bf16(const uint16_t *x, const uint16_t *w, int64_t rows, int64_t in, int64_t out,
                             uint16_t *y, float *acc_out, double *sum_abs);

#ifdef __cplusplus
}
#endif

#endif /* LMRS_ORACLE_H */
