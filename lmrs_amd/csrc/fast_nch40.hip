// fast_nch40.hip -- bf16_fast_kernel<40>: rows of up to 40 slots of 512 chunks of eight logits.
#include "fast_bf16.hpp"
#include "launch.hpp"

namespace lmrs {

static_assert(kFastSlotLogits == 8 * kFT && kFastVocabMax == kFastMaxVocab, "dispatch rule of sampling_api.hip");

void launch_fast_bf16_40(const lmrs_sample_args &a, int grid, hipStream_t s) {
  if (grid < a.batch)
    launch_fast_bf16_40_pairs(a, s);  // fast_nch40_pairs.hip
  else
    bf16_fast_kernel<40><<<dim3(a.batch), dim3(kFT), 0, s>>>(a);
}

}  // namespace lmrs
