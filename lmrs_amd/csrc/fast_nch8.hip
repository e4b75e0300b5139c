// fast_nch8.hip -- bf16_fast_kernel<8>: rows of up to 8 slots of 512 chunks of eight logits.
#include "fast_bf16.hpp"
#include "launch.hpp"

namespace lmrs {

static_assert(kFastSlotLogits == 8 * kFT && kFastVocabMax == kFastMaxVocab, "dispatch rule of sampling_api.hip");

void launch_fast_bf16_8(const lmrs_sample_args &a, int grid, hipStream_t s) {
  (void)grid;  // one workgroup per row
  bf16_fast_kernel<8><<<dim3(a.batch), dim3(kFT), 0, s>>>(a);
}

}  // namespace lmrs
