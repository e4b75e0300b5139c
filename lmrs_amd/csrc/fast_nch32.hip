// fast_nch32.hip -- bf16_fast_kernel<32>: rows of up to 32 slots of 512 chunks of eight logits.
#include "fast_bf16.hpp"
#include "launch.hpp"

namespace lmrs {

static_assert(kFastSlotLogits == 8 * kFT && kFastVocabMax == kFastMaxVocab, "dispatch rule of sampling_api.hip");

void launch_fast_bf16_32(const lmrs_sample_args &a, int grid, hipStream_t s) {
  (void)grid;  // one workgroup per row
  bf16_fast_kernel<32><<<dim3(a.batch), dim3(kFT), 0, s>>>(a);
}

}  // namespace lmrs
