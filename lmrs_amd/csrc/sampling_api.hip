// sampling_api.hip -- the C-ABI entry points (include/lmrs_sampling.h).
//
// Host-side argument checks, then one launch of one workgroup per row on the
// caller's stream.  Nothing here allocates device memory.
#include "lmrs_sampling.h"
#include "f32_dist.hpp"
#include "fast_bf16.hpp"
#include "generic_engine.hpp"

namespace {

int check_args(const lmrs_sample_args *a, bool need_tokens) {
  if (!a) return LMRS_ERR_NULL_ARGUMENT;
  if (a->dtype != LMRS_DTYPE_BF16 && a->dtype != LMRS_DTYPE_F32) return LMRS_ERR_BAD_DTYPE;
  if (a->batch < 0 || a->vocab < 0 || a->vocab > LMRS_MAX_VOCAB || a->row_stride < a->vocab)
    return LMRS_ERR_BAD_SHAPE;
  if (a->batch == 0) return LMRS_OK;
  if (need_tokens && !a->token_ids) return LMRS_ERR_NULL_ARGUMENT;
  if (a->vocab > 0 && !a->logits) return LMRS_ERR_NULL_ARGUMENT;
  if (a->hist_offsets && !a->hist_ids) return LMRS_ERR_NULL_ARGUMENT;
  const size_t esz = a->dtype == LMRS_DTYPE_BF16 ? 2 : 4;
  if (((uintptr_t)a->logits) % esz != 0) return LMRS_ERR_ALIGNMENT;
  return LMRS_OK;
}

int vector_ok(const lmrs_sample_args *a) {
  const size_t esz = a->dtype == LMRS_DTYPE_BF16 ? 2 : 4;
  return (((uintptr_t)a->logits) % 16 == 0) && (((size_t)a->row_stride * esz) % 16 == 0);
}

}  // namespace

extern "C" int lmrs_sample_fwd(const lmrs_sample_args *args, void *stream) {
  const int st = check_args(args, true);
  if (st != LMRS_OK || args->batch == 0) return st;
  hipStream_t s = (hipStream_t)stream;
  const int vec = vector_ok(args);
  const int64_t V = args->vocab;
  if (args->dtype == LMRS_DTYPE_BF16 && vec && V > 0 && V % 8 == 0 && V <= lmrs::kFastMaxVocab) {
    // register-resident rows: NCH chunks of 8 logits per thread (rows the
    // fast path does not take finish in the generic engine, in the same launch)
    const dim3 grid(args->batch), block(lmrs::kFT);
    constexpr int kSlot = 8 * lmrs::kFT;  // logits per chunk slot (one 16-byte chunk per thread)
    if (V <= 8 * kSlot)
      lmrs::bf16_fast_kernel<8><<<grid, block, 0, s>>>(*args);
    else if (V <= 16 * kSlot)
      lmrs::bf16_fast_kernel<16><<<grid, block, 0, s>>>(*args);
    else if (V <= 32 * kSlot)
      lmrs::bf16_fast_kernel<32><<<grid, block, 0, s>>>(*args);
    else
      lmrs::bf16_fast_kernel<lmrs::kMaxSlots><<<grid, block, 0, s>>>(*args);
  } else if (args->dtype == LMRS_DTYPE_BF16)
    lmrs::generic_sample_kernel<LMRS_DTYPE_BF16><<<args->batch, lmrs::kThreads, 0, s>>>(*args, vec);
  else
    lmrs::f32_sample_kernel<<<args->batch, lmrs::kThreads, 0, s>>>(*args, vec);
  return hipGetLastError() == hipSuccess ? LMRS_OK : LMRS_ERR_LAUNCH;
}

extern "C" int lmrs_process_logits_fwd(const lmrs_sample_args *args, void *out, void *stream) {
  const int st = check_args(args, false);
  if (st != LMRS_OK || args->batch == 0 || args->vocab == 0) return st;
  if (!out) return LMRS_ERR_NULL_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (args->dtype == LMRS_DTYPE_BF16)
    lmrs::process_kernel<LMRS_DTYPE_BF16><<<args->batch, lmrs::kThreads, 0, s>>>(*args, out);
  else
    lmrs::process_kernel<LMRS_DTYPE_F32><<<args->batch, lmrs::kThreads, 0, s>>>(*args, out);
  return hipGetLastError() == hipSuccess ? LMRS_OK : LMRS_ERR_LAUNCH;
}

extern "C" size_t lmrs_sample_workspace_size(int32_t, int64_t, int32_t, int64_t) { return 0; }

extern "C" const char *lmrs_sampling_version(void) { return "lmrs-mi355x-sampling 0.2 (gfx950)"; }
