/*
 * lmrs_sampling.h -- C-ABI of the MI355X batched token sampler.
 *
 * One call samples one token for each of `batch` rows of a [batch, vocab]
 * logits tensor that already lives in device memory.  It replaces, for a whole
 * decode step, the reference's per-row `Sampler::sample`
 * (crates/sampling/src/sampler/sampler.rs:178-186): the processor chain
 * (RepetitionPenalty crates/sampling/src/logits/repetition.rs:80-117,
 * FrequencyPresencePenalty logits/presence.rs:100-130, Temperature
 * logits/temperature.rs:66-72, each a chain of CUDA elementwise kernels bound
 * through crates/kernels/src/tensor_ops.rs:28-34,142-174), the cast and copy
 * to the host (tensor_ops.rs:176-186), and the host strategy (Greedy / TopK /
 * TopP / MinP / softmax_choice, crates/sampling/src/strategies/mod.rs:21-61,
 * greedy.rs:22-29, top_k.rs:39-45, top_p.rs:39-61, min_p.rs:39-55).
 *
 * Conventions follow the reference's native layer (kernels/ffi, declared in
 * crates/kernels/src/raw.rs:53-147): plain pointers and sizes, dtype codes
 * 0 = bf16, 1 = f16, 2 = f32 (raw.rs:9-14), stream last.  Two deliberate
 * differences: calls return a status instead of void, so bad arguments are
 * never silently ignored (the reference's *_fwd ignore an unknown dtype,
 * ops_ffi.cu:72-79), and per-row failures are reported in `status[r]`
 * instead of a Rust Result.
 *
 * Everything is asynchronous on `stream` (a hipStream_t; NULL = the null
 * stream).  No call allocates device memory.  All device pointers must stay
 * valid until the stream reaches the call.
 */
#ifndef LMRS_SAMPLING_H
#define LMRS_SAMPLING_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes (crates/kernels/src/raw.rs:9-14). f16 is not accepted by the
 * sampler: the reference Sampler takes bf16 only (tensor_ops.rs:177); f32 is
 * accepted and processed without bf16 rounding. */
#define LMRS_DTYPE_BF16 0
#define LMRS_DTYPE_F16 1
#define LMRS_DTYPE_F32 2

/* Return codes of the entry points. */
#define LMRS_OK 0
#define LMRS_ERR_NULL_ARGUMENT -1  /* a required pointer is NULL */
#define LMRS_ERR_BAD_DTYPE -2      /* dtype not in {BF16, F32} */
#define LMRS_ERR_BAD_SHAPE -3      /* batch < 0, vocab < 0, row_stride < vocab, or vocab > LMRS_MAX_VOCAB */
#define LMRS_ERR_LAUNCH -4         /* the HIP launch failed (see hipGetLastError) */
#define LMRS_ERR_ALIGNMENT -5      /* logits pointer not aligned to its element size */

/* Per-row status codes written to status[r] (low byte) ... */
#define LMRS_ROW_OK 0
#define LMRS_ROW_EMPTY 1        /* vocab == 0: "cannot sample from empty logits" (strategies/greedy.rs:24-26),
                                   or an empty candidate set (strategies/mod.rs:28-30) */
#define LMRS_ROW_DISTRIBUTION 2 /* non-finite or non-positive weight sum (strategies/mod.rs:39-43) */
#define LMRS_ROW_PARAM 3        /* a parameter fails its constructor's validation (repetition.rs:57-64,
                                   presence.rs:61-71, temperature.rs:43-50, top_p.rs:26-31,
                                   min_p.rs:27-29); top_k < -1 */
#define LMRS_ROW_HISTORY 4      /* more than LMRS_MAX_HISTORY_DISTINCT distinct history tokens in this row,
                                   or one token more than LMRS_MAX_HISTORY_COUNT times (any length is
                                   taken otherwise; repetition.rs:88-97 and presence.rs:107-117 have
                                   no limit) */
/* ... and flag bits above it. */
#define LMRS_ROW_NEAR_BOUNDARY 0x100 /* the uniform lies within 1e-6 of a CDF boundary of the chosen
                                        token, or the nucleus cumulative lies within 1e-6 of top_p at
                                        the cut: the reference's f64 summation order may pick a
                                        neighbouring token here; or exp() of a logit at the min-p
                                        cut lies within 1e-12 (relative) of the threshold, where
                                        the host and device exp may round to opposite sides */

/* top_k value that selects the Greedy strategy (greedy.rs:22-29): the first
 * token in sorted order, log_prob 0, no draw and no other cut, whatever the
 * values (a NaN or infinite maximum is returned as is).  top_k = 1 is TopK(1)
 * instead (top_k.rs:39-45): the same token on finite rows, but it draws
 * through softmax_choice and so reports LMRS_ROW_DISTRIBUTION for a row whose
 * maximum is +inf, NaN or -inf (strategies/mod.rs:39-43). */
#define LMRS_GREEDY (-1)

#define LMRS_MAX_VOCAB 262144  /* largest vocab accepted (2^18) */
#define LMRS_MAX_HISTORY_DISTINCT 12288 /* distinct history tokens per row accepted */
#define LMRS_MAX_HISTORY_COUNT 16383    /* occurrences of one history token accepted */

typedef struct lmrs_sample_args {
  /* logits: device, `batch` rows of `row_stride` elements of `dtype`; only the
   * first `vocab` elements of a row are read.  Never written. */
  const void *logits;
  int32_t dtype;
  int32_t batch;
  int64_t vocab;
  int64_t row_stride;

  /* Token history per row in CSR form (device): the ids of row r are
   * hist_ids[hist_offsets[r] .. hist_offsets[r+1]).  Ids >= vocab are ignored
   * (repetition.rs:93, presence.rs:113).  hist_offsets == NULL: no history. */
  const int64_t *hist_offsets;
  const uint32_t *hist_ids;

  /* Per-row parameters (device arrays of length batch; NULL = the neutral
   * value, which skips the processor exactly as the reference does). */
  const float *repetition_penalty; /* finite, > 0; 1.0 = off (repetition.rs:82) */
  const float *presence_penalty;   /* finite; 0 = off together with frequency (presence.rs:102) */
  const float *frequency_penalty;  /* finite */
  const double *temperature;       /* finite, > 0; 1.0 = off (temperature.rs:68) */
  const int32_t *top_k;            /* 0 = off; k > 0 = TopK(k) (top_k.rs:39-45); LMRS_GREEDY = Greedy
                                      (greedy.rs:22-29); below LMRS_GREEDY: LMRS_ROW_PARAM */
  const double *top_p;             /* in (0, 1]; 1.0 = off */
  const double *uniforms;          /* in [0, 1): the draw's uniform (next_unit of the reference's
                                      LCG, strategies/mod.rs:57-61, or any caller RNG).  Required
                                      unless every row is greedy; NULL reads as 0. */
  const double *min_p;             /* in [0, 1]: MinP's cut (strategies/min_p.rs:39-55), keeping
                                      the candidates with exp(f64(l)) >= exp(f64(max)) * min_p;
                                      negative = off (NULL: off for every row); NaN or > 1 is
                                      LMRS_ROW_PARAM (min_p.rs:27-29).  A cut that keeps nothing
                                      is LMRS_ROW_EMPTY. */

  /* Outputs (device, length batch).  token_ids is required. */
  uint32_t *token_ids; /* SampleOutput::token_id (sampler/output.rs:14-18) */
  float *log_probs;    /* ln of the chosen token's post-filter probability; 0 for greedy */
  float *logits_out;   /* processed logit of the chosen token */
  int32_t *status;     /* per-row LMRS_ROW_* code | flags */

  /* Optional (NULL: not written): the post-filter distribution of each row,
   * for tests and diagnostics (the reference exposes only the chosen token's
   * probability, strategies/mod.rs:47-48).  kept_count[r]: the number of
   * tokens the top-k, min-p and nucleus cuts keep (1 for Greedy, 0 for a
   * failed row); kept_mass[r]: the sum over them of exp(f64(l - max)), l
   * their processed logits and max the row's largest (softmax_choice's
   * weights and sum, strategies/mod.rs:35-37).  With the processed logits
   * (lmrs_process_logits_fwd) they give every kept token's probability:
   * exp(f64(l - max)) / kept_mass, in the sorted order's first kept_count. */
  int32_t *kept_count;
  double *kept_mass;
} lmrs_sample_args;

/* Samples one token per row (the fused replacement of Sampler::sample over a
 * batch).  Asynchronous on `stream`.  Returns LMRS_OK or an LMRS_ERR_* code;
 * per-row problems are reported in status[r] and never fail the call.
 *
 * Per row: the processors, then top_k == LMRS_GREEDY is Greedy (no other
 * strategy parameter applies); otherwise the candidates are cut by top-k (top_k.rs:39-45),
 * then by min-p (min_p.rs:45-53), then by the nucleus (top_p.rs:45-58), and
 * softmax_choice draws from what is left (strategies/mod.rs:27-55).  Each cut
 * that is off keeps everything, so a row with one strategy parameter set is
 * exactly that reference strategy. */
int lmrs_sample_fwd(const lmrs_sample_args *args, void *stream);

/* Applies the processor chain only (Repetition -> Presence/Frequency ->
 * Temperature, each skipped per its own rule) and writes the processed rows,
 * in the input dtype, to `out` ([batch, vocab] contiguous, device).  This is
 * LogitsProcessor::process (crates/sampling/src/logits/processor.rs:21-24)
 * for the three reference processors, batched.  Uses args' logits, dtype,
 * batch, vocab, row_stride, history and the three penalty / temperature
 * arrays (status[r], when given, reports a penalty, temperature or history
 * that fails its check, and such a row is copied unchanged); top_k, top_p,
 * min_p, uniforms and the other outputs are neither read nor checked. */
int lmrs_process_logits_fwd(const lmrs_sample_args *args, void *out, void *stream);

/* The LM head's vocabulary projection with the sampling prologue in its
 * epilogue: out[r, v] = bf16(sum_k input[r, k] * weight[v, k]) for `rows`
 * rows of `in_features` bf16 hidden values and a [out_features, in_features]
 * bf16 weight (row-major, out [rows, out_features] contiguous), f32
 * accumulation on the matrix cores.  Replaces, for the LM head (bf16, no
 * bias), LmHead::forward (crates/ops/src/embedding/lm_head.rs:33-35) ->
 * kernels::linear -> linear_fwd (kernels/ffi/tensor_ffi.cu:820-841,
 * linear_kernel :230-258), whose argument order it keeps; the sums run in
 * the matrix unit's order, so a logit may differ from linear_kernel's by the
 * rounding of its f32 sum.  When tile_max is not NULL it receives, for every
 * row r and 64-column tile t, the tile's largest logit in the sampler's total
 * order: tile_max[r * ceil(out_features / 64) + t] = key << 32 | ~column,
 * key the 16-bit order key of the bf16 pattern (negatives flipped, sign bit
 * set on non-negatives), ties to the lower column.  dtype must be
 * LMRS_DTYPE_BF16; in_features % 8 == 0; input and weight 16-byte aligned.
 * Asynchronous on `stream`; allocates nothing. */
int lmrs_lm_head_fwd(void *out, const void *input, const void *weight, int32_t rows, int32_t in_features,
                     int32_t out_features, int32_t dtype, uint64_t *tile_max, void *stream);

/* Device workspace, in bytes, that lmrs_sample_fwd needs for a call of this
 * shape: always 0.  Every working set (history tables, candidate lists,
 * histograms) lives in the workgroup's LDS and registers, so the caller
 * passes no workspace and no call allocates.  Kept so that a caller written
 * against a workspace-taking sampler (query, allocate, pass) binds unchanged. */
size_t lmrs_sample_workspace_size(int32_t batch, int64_t vocab, int32_t dtype, int64_t max_hist);

/* Library version string. */
const char *lmrs_sampling_version(void);

#ifdef __cplusplus
}
#endif

#endif /* LMRS_SAMPLING_H */
