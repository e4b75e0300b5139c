/*
 * lmrs_oracle.c -- CPU restatement of lmrs's token-sampling path.
 *
 * TEST INFRASTRUCTURE ONLY (see lmrs_oracle.h): the checker for the HIP
 * sampler, never part of the product path.
 *
 * Build flags matter for faithfulness: -ffp-contract=off (Rust never fuses a
 * multiply and an add; only the CUDA affine kernel is fused, and that one is
 * written as an explicit fmaf below) and no -ffast-math.  exp()/log() are
 * glibc's, which is what Rust's f64::exp / f64::ln call on linux-gnu.
 */
#include "lmrs_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* bf16 conversions                                                          */
/* ------------------------------------------------------------------------ */

static inline uint32_t f32_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}

static inline float bits_f32(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}

/* Round-to-nearest-even of the upper 16 bits: add 0x7FFF plus the lsb of the
 * kept half, then truncate.  (IEEE 754 roundTiesToEven on the bf16 grid.) */
static inline uint16_t rne16(uint32_t u) {
  uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7FFFu + lsb) >> 16);
}

uint16_t lmrs_oracle_bf16_from_f32_host(float x) {
  uint32_t u = f32_bits(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
  return rne16(u);
}

uint16_t lmrs_oracle_bf16_from_f32_dev(float x) {
  uint32_t u = f32_bits(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FFFu;
  return rne16(u);
}

float lmrs_oracle_f32_from_bf16(uint16_t b) { return bits_f32((uint32_t)b << 16); }

/* ------------------------------------------------------------------------ */
/* RNG and ordering                                                          */
/* ------------------------------------------------------------------------ */

/* strategies/mod.rs:57-61: wrapping LCG step, then the top 52 state bits as
 * the mantissa of a double in [1, 2), minus 1. */
double lmrs_oracle_next_unit(uint64_t *state) {
  *state = *state * 6364136223846793005ull + 1ull;
  uint64_t bits = (*state >> 11) | 0x3FF0000000000000ull;
  double d;
  memcpy(&d, &bits, 8);
  return d - 1.0;
}

/* totalOrder key: flip all bits of negatives, set the sign bit of
 * non-negatives; unsigned comparison of keys is f32::total_cmp. */
static inline uint32_t order_key(float x) {
  uint32_t u = f32_bits(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

int lmrs_oracle_total_cmp(float a, float b) {
  uint32_t ka = order_key(a), kb = order_key(b);
  return ka < kb ? -1 : (ka > kb ? 1 : 0);
}

/* Bottom-up merge sort of u64 (ascending). */
static void sort_u64(uint64_t *a, int64_t n) {
  if (n < 2) return;
  uint64_t *tmp = (uint64_t *)malloc((size_t)n * sizeof(uint64_t));
  uint64_t *src = a, *dst = tmp;
  /* insertion sort runs of 32 */
  const int64_t RUN = 32;
  for (int64_t s = 0; s < n; s += RUN) {
    int64_t e = s + RUN < n ? s + RUN : n;
    for (int64_t i = s + 1; i < e; ++i) {
      uint64_t v = a[i];
      int64_t j = i - 1;
      while (j >= s && a[j] > v) {
        a[j + 1] = a[j];
        --j;
      }
      a[j + 1] = v;
    }
  }
  for (int64_t w = RUN; w < n; w *= 2) {
    for (int64_t s = 0; s < n; s += 2 * w) {
      int64_t m = s + w < n ? s + w : n;
      int64_t e = s + 2 * w < n ? s + 2 * w : n;
      int64_t i = s, j = m, k = s;
      while (i < m && j < e) dst[k++] = (src[j] < src[i]) ? src[j++] : src[i++];
      while (i < m) dst[k++] = src[i++];
      while (j < e) dst[k++] = src[j++];
    }
    uint64_t *t = src;
    src = dst;
    dst = t;
  }
  if (src != a) memcpy(a, src, (size_t)n * sizeof(uint64_t));
  free(tmp);
}

/* sorted_logits (strategies/mod.rs:21-25): value descending by total_cmp,
 * ties by index ascending.  Composite key: (~order_key) high, index low. */
void lmrs_oracle_sorted_indices(const float *logits, int64_t n, int64_t *order) {
  uint64_t *keys = (uint64_t *)malloc((size_t)(n > 0 ? n : 1) * sizeof(uint64_t));
  for (int64_t i = 0; i < n; ++i)
    keys[i] = ((uint64_t)(~order_key(logits[i])) << 32) | (uint64_t)(uint32_t)i;
  sort_u64(keys, n);
  for (int64_t i = 0; i < n; ++i) order[i] = (int64_t)(keys[i] & 0xFFFFFFFFull);
  free(keys);
}

/* ------------------------------------------------------------------------ */
/* softmax_choice (strategies/mod.rs:27-55)                                  */
/* ------------------------------------------------------------------------ */

/* Validation part: weights and their sequential f64 sum.  Returns status. */
static int softmax_weights(const float *logits, const int64_t *cand, int64_t n, double *w,
                           double *sum_out) {
  if (n == 0) return LMRS_ORACLE_ERR_EMPTY;
  float max = logits[cand[0]];
  double sum = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    float d = logits[cand[i]] - max; /* f32 subtraction, then widened */
    w[i] = exp((double)d);
    sum += w[i];
  }
  if (!isfinite(sum) || sum <= 0.0) return LMRS_ORACLE_ERR_DISTRIBUTION;
  *sum_out = sum;
  return LMRS_ORACLE_OK;
}

/* Draw part: walk the candidates with target = u * sum. */
static void softmax_draw(const float *logits, const int64_t *cand, int64_t n, const double *w,
                         double sum, double u, lmrs_oracle_output *out, lmrs_oracle_diag *diag) {
  double target = u * sum;
  int64_t pick = n - 1;
  for (int64_t i = 0; i < n; ++i) {
    if (target <= w[i]) {
      pick = i;
      break;
    }
    target -= w[i];
  }
  /* The fallback (mod.rs:52-54) recomputes exp(l - max) / sum, which is w[n-1]. */
  double prob = w[pick] / sum;
  out->token_id = (uint32_t)cand[pick];
  out->log_prob = (float)log(prob);
  out->logit = logits[cand[pick]];
  if (diag) {
    double cum = 0.0;
    for (int64_t i = 0; i < pick; ++i) cum += w[i];
    double lo = cum / sum, hi = (cum + w[pick]) / sum;
    double m = INFINITY;
    if (pick > 0 && fabs(u - lo) < m) m = fabs(u - lo);
    if (pick < n - 1 && fabs(hi - u) < m) m = fabs(hi - u);
    diag->cdf_margin = m;
    diag->cum_before = cum;
    diag->sum_kept = sum;
    diag->weight = w[pick];
    diag->n_kept = n;
  }
}

static int softmax_choice_u(const float *logits, const int64_t *cand, int64_t n, double u,
                            lmrs_oracle_output *out, lmrs_oracle_diag *diag) {
  double *w = (double *)malloc((size_t)(n > 0 ? n : 1) * sizeof(double));
  double sum = 0.0;
  int st = softmax_weights(logits, cand, n, w, &sum);
  if (st == LMRS_ORACLE_OK) softmax_draw(logits, cand, n, w, sum, u, out, diag);
  free(w);
  return st;
}

static int softmax_choice_rng(const float *logits, const int64_t *cand, int64_t n, uint64_t *rng,
                              lmrs_oracle_output *out) {
  double *w = (double *)malloc((size_t)(n > 0 ? n : 1) * sizeof(double));
  double sum = 0.0;
  int st = softmax_weights(logits, cand, n, w, &sum);
  if (st == LMRS_ORACLE_OK) {
    double u = lmrs_oracle_next_unit(rng); /* drawn only after validation */
    softmax_draw(logits, cand, n, w, sum, u, out, NULL);
  }
  free(w);
  return st;
}

/* ------------------------------------------------------------------------ */
/* strategies                                                                */
/* ------------------------------------------------------------------------ */

int lmrs_oracle_greedy(const float *logits, int64_t n, lmrs_oracle_output *out) {
  if (n <= 0) return LMRS_ORACLE_ERR_EMPTY;
  /* sorted[0] == maximum under total_cmp with the lowest index among ties. */
  int64_t best = 0;
  uint32_t bk = order_key(logits[0]);
  for (int64_t i = 1; i < n; ++i) {
    uint32_t k = order_key(logits[i]);
    if (k > bk) {
      bk = k;
      best = i;
    }
  }
  out->token_id = (uint32_t)best;
  out->log_prob = 0.0f;
  out->logit = logits[best];
  return LMRS_ORACLE_OK;
}

int lmrs_oracle_beam(const float *logits, int64_t n, int64_t width, lmrs_oracle_output *out) {
  if (width <= 0) return LMRS_ORACLE_ERR_PARAM; /* beam.rs:31-33 */
  return lmrs_oracle_greedy(logits, n, out);    /* first of sorted (beam.rs:45) */
}

int lmrs_oracle_top_k(const float *logits, int64_t n, int64_t k, uint64_t *rng,
                      lmrs_oracle_output *out) {
  if (k <= 0) return LMRS_ORACLE_ERR_PARAM; /* top_k.rs:27-29 */
  int64_t *order = (int64_t *)malloc((size_t)(n > 0 ? n : 1) * sizeof(int64_t));
  lmrs_oracle_sorted_indices(logits, n, order);
  int64_t end = k < n ? k : n;
  int st = softmax_choice_rng(logits, order, end, rng, out);
  free(order);
  return st;
}

/* Nucleus length over a sorted candidate prefix (top_p.rs:45-58). */
static int64_t nucleus_keep(const float *logits, const int64_t *cand, int64_t n, double p,
                            double *margin) {
  float max = logits[cand[0]];
  double denom = 0.0;
  for (int64_t i = 0; i < n; ++i) denom += exp((double)(logits[cand[i]] - max));
  double acc = 0.0, prev = 0.0;
  int64_t keep = 0;
  for (int64_t i = 0; i < n; ++i) {
    prev = acc;
    acc += exp((double)(logits[cand[i]] - max)) / denom;
    keep += 1;
    if (acc >= p) break;
  }
  if (margin) {
    double m = fabs(p - prev);
    if (acc >= p && fabs(acc - p) < m) m = fabs(acc - p);
    if (!(acc >= p)) m = fabs(p - acc);
    *margin = m;
  }
  return keep;
}

int lmrs_oracle_top_p(const float *logits, int64_t n, double p, uint64_t *rng,
                      lmrs_oracle_output *out) {
  if (!isfinite(p) || p <= 0.0 || p > 1.0) return LMRS_ORACLE_ERR_PARAM; /* top_p.rs:27-29 */
  if (n <= 0) return LMRS_ORACLE_ERR_EMPTY;
  int64_t *order = (int64_t *)malloc((size_t)n * sizeof(int64_t));
  lmrs_oracle_sorted_indices(logits, n, order);
  int64_t keep = nucleus_keep(logits, order, n, p, NULL);
  int st = softmax_choice_rng(logits, order, keep, rng, out);
  free(order);
  return st;
}

int lmrs_oracle_min_p(const float *logits, int64_t n, double min_p, uint64_t *rng,
                      lmrs_oracle_output *out) {
  if (!isfinite(min_p) || min_p < 0.0 || min_p > 1.0) return LMRS_ORACLE_ERR_PARAM; /* min_p.rs:27-29 */
  if (n <= 0) return LMRS_ORACLE_ERR_EMPTY;
  int64_t *order = (int64_t *)malloc((size_t)n * sizeof(int64_t));
  lmrs_oracle_sorted_indices(logits, n, order);
  double threshold = exp((double)logits[order[0]]) * min_p; /* min_p.rs:45-46 */
  int64_t nk = 0;
  for (int64_t i = 0; i < n; ++i)
    if (exp((double)logits[order[i]]) >= threshold) order[nk++] = order[i];
  int st = softmax_choice_rng(logits, order, nk, rng, out);
  free(order);
  return st;
}

/* ------------------------------------------------------------------------ */
/* processors                                                                */
/* ------------------------------------------------------------------------ */

static int valid_repetition(float p) { return isfinite(p) && p > 0.0f; }      /* repetition.rs:58 */
static int valid_presence(float a, float b) { return isfinite(a) && isfinite(b); } /* presence.rs:62 */
static int valid_temperature(double t) { return isfinite(t) && t > 0.0; }    /* temperature.rs:44 */

int lmrs_oracle_repetition(void *row, int dtype, int64_t n, float penalty, const uint32_t *history,
                           int64_t h) {
  if (!valid_repetition(penalty)) return LMRS_ORACLE_ERR_PARAM;
  if (penalty == 1.0f || h == 0) return LMRS_ORACLE_OK; /* repetition.rs:82-84 */
  float inv = 1.0f / penalty;                           /* repetition.rs:88 */
  unsigned char *mark = (unsigned char *)calloc((size_t)(n > 0 ? n : 1), 1);
  for (int64_t j = 0; j < h; ++j)
    if ((int64_t)history[j] < n) mark[history[j]] = 1; /* repetition.rs:91-97 */
  if (dtype == 0) {
    uint16_t *x = (uint16_t *)row;
    /* factor tensors: bf16(inv) / bf16(p) on penalised tokens, bf16(1) elsewhere */
    float pf = lmrs_oracle_f32_from_bf16(lmrs_oracle_bf16_from_f32_host(inv));
    float nf = lmrs_oracle_f32_from_bf16(lmrs_oracle_bf16_from_f32_host(penalty));
    for (int64_t i = 0; i < n; ++i) {
      float v = lmrs_oracle_f32_from_bf16(x[i]);
      float fp = mark[i] ? pf : 1.0f, fn = mark[i] ? nf : 1.0f;
      /* mul, mul, greater_equal(x, 0), where (repetition.rs:113-116) */
      uint16_t pos = lmrs_oracle_bf16_from_f32_dev(v * fp);
      uint16_t neg = lmrs_oracle_bf16_from_f32_dev(v * fn);
      x[i] = (v >= 0.0f) ? pos : neg;
    }
  } else {
    float *x = (float *)row;
    for (int64_t i = 0; i < n; ++i) {
      float v = x[i];
      float fp = mark[i] ? inv : 1.0f, fn = mark[i] ? penalty : 1.0f;
      x[i] = (v >= 0.0f) ? v * fp : v * fn;
    }
  }
  free(mark);
  return LMRS_ORACLE_OK;
}

static int cmp_u32(const void *a, const void *b) {
  uint32_t x = *(const uint32_t *)a, y = *(const uint32_t *)b;
  return x < y ? -1 : (x > y ? 1 : 0);
}

int lmrs_oracle_presence(void *row, int dtype, int64_t n, float presence, float frequency,
                         const uint32_t *history, int64_t h) {
  if (!valid_presence(presence, frequency)) return LMRS_ORACLE_ERR_PARAM;
  if (h == 0 || (presence == 0.0f && frequency == 0.0f)) return LMRS_ORACLE_OK; /* presence.rs:102-104 */
  float *pen = (float *)calloc((size_t)(n > 0 ? n : 1), sizeof(float));
  /* multiplicity of each token (the HashMap of presence.rs:107-110) */
  uint32_t *sorted = (uint32_t *)malloc((size_t)h * sizeof(uint32_t));
  memcpy(sorted, history, (size_t)h * sizeof(uint32_t));
  qsort(sorted, (size_t)h, sizeof(uint32_t), cmp_u32);
  for (int64_t j = 0; j < h;) {
    int64_t e = j;
    while (e < h && sorted[e] == sorted[j]) ++e;
    uint32_t count = (uint32_t)(e - j);
    if ((int64_t)sorted[j] < n) pen[sorted[j]] = presence + frequency * (float)count; /* presence.rs:114 */
    j = e;
  }
  free(sorted);
  if (dtype == 0) {
    uint16_t *x = (uint16_t *)row;
    for (int64_t i = 0; i < n; ++i) {
      float pb = lmrs_oracle_f32_from_bf16(lmrs_oracle_bf16_from_f32_host(pen[i])); /* presence.rs:123-126 */
      x[i] = lmrs_oracle_bf16_from_f32_dev(lmrs_oracle_f32_from_bf16(x[i]) - pb);   /* sub (:129) */
    }
  } else {
    float *x = (float *)row;
    for (int64_t i = 0; i < n; ++i) x[i] = x[i] - pen[i];
  }
  free(pen);
  return LMRS_ORACLE_OK;
}

int lmrs_oracle_temperature(void *row, int dtype, int64_t n, double temperature) {
  if (!valid_temperature(temperature)) return LMRS_ORACLE_ERR_PARAM;
  if (temperature == 1.0) return LMRS_ORACLE_OK; /* temperature.rs:68-70 */
  float s = (float)(1.0 / temperature);          /* temperature.rs:71 */
  /* affine_kernel computes value * scale + offset, which the CUDA compiler
   * contracts to one fused multiply-add (tensor_ffi.cu:55-56). */
  if (dtype == 0) {
    uint16_t *x = (uint16_t *)row;
    for (int64_t i = 0; i < n; ++i)
      x[i] = lmrs_oracle_bf16_from_f32_dev(fmaf(lmrs_oracle_f32_from_bf16(x[i]), s, 0.0f));
  } else {
    float *x = (float *)row;
    for (int64_t i = 0; i < n; ++i) x[i] = fmaf(x[i], s, 0.0f);
  }
  return LMRS_ORACLE_OK;
}

/* ------------------------------------------------------------------------ */
/* composed per-row sampler                                                  */
/* ------------------------------------------------------------------------ */

int lmrs_oracle_sample_row(const void *logits, int dtype, int64_t n, const uint32_t *history,
                           int64_t h, const lmrs_oracle_params *pr, double u,
                           lmrs_oracle_output *out, lmrs_oracle_diag *diag, float *processed_out) {
  if (dtype != 0 && dtype != 2) return LMRS_ORACLE_ERR_PARAM;
  if (!valid_repetition(pr->repetition_penalty) ||
      !valid_presence(pr->presence_penalty, pr->frequency_penalty) ||
      !valid_temperature(pr->temperature) || pr->top_k < -1 || !isfinite(pr->top_p) ||
      pr->top_p <= 0.0 || pr->top_p > 1.0 || isnan(pr->min_p) || pr->min_p > 1.0)
    return LMRS_ORACLE_ERR_PARAM; /* min_p: min_p.rs:27-29, negative = off */
  if (diag) {
    diag->cdf_margin = INFINITY;
    diag->top_p_margin = INFINITY;
    diag->min_p_margin = INFINITY;
    diag->cum_before = 0.0;
    diag->sum_kept = 0.0;
    diag->weight = 0.0;
    diag->n_candidates = 0;
    diag->n_kept = 0;
  }
  size_t esz = dtype == 0 ? 2 : 4;
  void *row = malloc((size_t)(n > 0 ? n : 1) * esz);
  memcpy(row, logits, (size_t)n * esz);
  lmrs_oracle_repetition(row, dtype, n, pr->repetition_penalty, history, h);
  lmrs_oracle_presence(row, dtype, n, pr->presence_penalty, pr->frequency_penalty, history, h);
  lmrs_oracle_temperature(row, dtype, n, pr->temperature);
  float *v = (float *)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
  for (int64_t i = 0; i < n; ++i)
    v[i] = dtype == 0 ? lmrs_oracle_f32_from_bf16(((uint16_t *)row)[i]) : ((float *)row)[i];
  free(row);
  if (processed_out) memcpy(processed_out, v, (size_t)n * sizeof(float));
  int st;
  if (n <= 0) {
    st = LMRS_ORACLE_ERR_EMPTY;
  } else if (pr->top_k == -1) {
    /* Greedy (greedy.rs:22-29): sorted[0] whatever its value; TopK(1) below
       goes through softmax_choice and rejects a non-finite maximum */
    st = lmrs_oracle_greedy(v, n, out);
    if (diag) {
      diag->n_candidates = 1;
      diag->n_kept = 1;
      diag->sum_kept = 1.0;
      diag->weight = 1.0;
    }
  } else {
    int64_t *order = (int64_t *)malloc((size_t)n * sizeof(int64_t));
    lmrs_oracle_sorted_indices(v, n, order);
    int64_t cand = (pr->top_k > 0 && pr->top_k < n) ? pr->top_k : n;
    if (diag) diag->n_candidates = cand;
    if (pr->min_p >= 0.0) {
      /* MinP's filter (min_p.rs:44-53) over the top-k candidates */
      float max = v[order[0]];
      double threshold = exp((double)max) * pr->min_p;
      double margin = INFINITY;
      int64_t nk = 0;
      for (int64_t i = 0; i < cand; ++i) {
        float l = v[order[i]];
        double e = exp((double)l);
        if (l != max && !isnan(l) && isfinite(threshold) && threshold > 0.0 &&
            fabs(e - threshold) / threshold < margin)
          margin = fabs(e - threshold) / threshold;
        if (e >= threshold) order[nk++] = order[i];
      }
      if (diag) diag->min_p_margin = margin;
      cand = nk;
    }
    if (cand > 0 && pr->top_p < 1.0) {
      double margin = INFINITY;
      cand = nucleus_keep(v, order, cand, pr->top_p, &margin);
      if (diag) diag->top_p_margin = margin;
    }
    st = softmax_choice_u(v, order, cand, u, out, diag);
    free(order);
  }
  free(v);
  return st;
}

/* ------------------------------------------------------------------------ */
/* batch driver                                                              */
/* ------------------------------------------------------------------------ */

typedef struct {
  const void *logits;
  int dtype;
  int64_t batch, n, stride;
  const int64_t *off;
  const uint32_t *ids;
  const lmrs_oracle_params *params;
  const double *uniforms;
  lmrs_oracle_output *out;
  lmrs_oracle_diag *diag;
  int32_t *status;
  int64_t next;
  pthread_mutex_t lock;
} batch_job;

static void run_row(batch_job *j, int64_t r) {
  size_t esz = j->dtype == 0 ? 2 : 4;
  const char *row = (const char *)j->logits + (size_t)r * (size_t)j->stride * esz;
  const uint32_t *hist = j->off ? j->ids + j->off[r] : NULL;
  int64_t h = j->off ? j->off[r + 1] - j->off[r] : 0;
  int st = lmrs_oracle_sample_row(row, j->dtype, j->n, hist, h, &j->params[r], j->uniforms[r],
                                  &j->out[r], j->diag ? &j->diag[r] : NULL, NULL);
  if (j->status) j->status[r] = st;
}

static void *batch_worker(void *arg) {
  batch_job *j = (batch_job *)arg;
  for (;;) {
    pthread_mutex_lock(&j->lock);
    int64_t r = j->next++;
    pthread_mutex_unlock(&j->lock);
    if (r >= j->batch) break;
    run_row(j, r);
  }
  return NULL;
}

int lmrs_oracle_sample_batch(const void *logits, int dtype, int64_t batch, int64_t n,
                             int64_t row_stride, const int64_t *hist_offsets,
                             const uint32_t *hist_ids, const lmrs_oracle_params *params,
                             const double *uniforms, lmrs_oracle_output *out,
                             lmrs_oracle_diag *diag, int32_t *status, int n_threads) {
  batch_job j = {logits, dtype, batch, n, row_stride, hist_offsets, hist_ids, params,
                 uniforms, out, diag, status, 0, PTHREAD_MUTEX_INITIALIZER};
  if (n_threads <= 1) {
    for (int64_t r = 0; r < batch; ++r) run_row(&j, r);
    return LMRS_ORACLE_OK;
  }
  pthread_t *th = (pthread_t *)malloc((size_t)n_threads * sizeof(pthread_t));
  for (int t = 0; t < n_threads; ++t) pthread_create(&th[t], NULL, batch_worker, &j);
  for (int t = 0; t < n_threads; ++t) pthread_join(th[t], NULL);
  free(th);
  return LMRS_ORACLE_OK;
}

/* linear_kernel (kernels/ffi/tensor_ffi.cu:230-258), bf16, no bias. */
void lmrs_oracle_linear_bf16(const uint16_t *x, const uint16_t *w, int64_t rows, int64_t in, int64_t out,
                             uint16_t *y, float *acc_out, double *sum_abs) {
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t v = 0; v < out; ++v) {
      float acc = 0.0f;
      double sa = 0.0;
      for (int64_t k = 0; k < in; ++k) {
        const float p = lmrs_oracle_f32_from_bf16(x[r * in + k]) * lmrs_oracle_f32_from_bf16(w[v * in + k]);
        acc += p;
        sa += fabs((double)p);
      }
      y[r * out + v] = lmrs_oracle_bf16_from_f32_dev(acc);
      if (acc_out) acc_out[r * out + v] = acc;
      if (sum_abs) sum_abs[r * out + v] = sa;
    }
  }
}
