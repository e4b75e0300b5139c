// fast_nch16.hip -- bf16_fast_kernel<16>: rows of up to 16 slots of 512 chunks of eight logits.
#include "fast_bf16.hpp"
#include "launch.hpp"

namespace lmrs {

static_assert(kFastSlotLogits == 8 * kFT && kFastVocabMax == kFastMaxVocab, "dispatch rule of sampling_api.hip");

void launch_fast_bf16_16(const lmrs_sample_args &a, int grid, hipStream_t s) {
  (void)grid;  // one workgroup per row
  bf16_fast_kernel<16><<<dim3(a.batch), dim3(kFT), 0, s>>>(a);
}

}  // namespace lmrs
