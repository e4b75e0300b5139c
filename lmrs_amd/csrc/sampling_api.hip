// sampling_api.hip -- the C-ABI entry points (include/lmrs_sampling.h).
//
// Host-side argument checks, then one launch on the caller's stream (the
// kernels live in their own translation units, behind launch.hpp): one
// workgroup per row, or for the widest bf16 rows in batches of more rows than
// CUs two rows per workgroup.  Nothing here allocates device memory.
#include "lmrs_sampling.h"
#include "launch.hpp"

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

// The CU count of the current device (queried once per device), at most the
// number of rows: a batch of more rows than CUs pairs the widest rows.
int fast_grid(int batch) {
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cus[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return batch < cus[dev] ? batch : cus[dev];
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
  // register-resident bf16 rows: NCH slots of one 16-byte chunk (eight
  // logits) per thread of a 512-thread workgroup (rows the fast kernel does
  // not take finish in the generic engine, in the same launch)
  constexpr int64_t kSlot = lmrs::kFastSlotLogits;
  if (args->dtype == LMRS_DTYPE_BF16 && vec && V > 0 && V % 8 == 0 && V <= lmrs::kFastVocabMax) {
    const int grid = fast_grid(args->batch);
    if (V <= 8 * kSlot)
      lmrs::launch_fast_bf16_8(*args, grid, s);
    else if (V <= 16 * kSlot)
      lmrs::launch_fast_bf16_16(*args, grid, s);
    else if (V <= 32 * kSlot)
      lmrs::launch_fast_bf16_32(*args, grid, s);
    else
      lmrs::launch_fast_bf16_40(*args, grid, s);
  } else if (args->dtype == LMRS_DTYPE_BF16) {
    lmrs::launch_generic_bf16(*args, vec, s);
  } else {
    lmrs::launch_f32(*args, vec, s);
  }
  return hipGetLastError() == hipSuccess ? LMRS_OK : LMRS_ERR_LAUNCH;
}

extern "C" int lmrs_process_logits_fwd(const lmrs_sample_args *args, void *out, void *stream) {
  const int st = check_args(args, false);
  if (st != LMRS_OK || args->batch == 0 || args->vocab == 0) return st;
  if (!out) return LMRS_ERR_NULL_ARGUMENT;
  lmrs::launch_process(*args, out, (hipStream_t)stream);
  return hipGetLastError() == hipSuccess ? LMRS_OK : LMRS_ERR_LAUNCH;
}

extern "C" size_t lmrs_sample_workspace_size(int32_t, int64_t, int32_t, int64_t) { return 0; }

extern "C" const char *lmrs_sampling_version(void) { return "lmrs-mi355x-sampling 0.2 (gfx950)"; }
