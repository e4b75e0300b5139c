// fast_nch40_pairs.hip -- bf16_fast_rounds_kernel<40>: two rows of up to 40
// slots per workgroup, for batches of more rows than CUs (its own translation
// unit: the two inlined rows make it the library's longest compile).
#include "fast_bf16.hpp"
#include "launch.hpp"

namespace lmrs {

void launch_fast_bf16_40_pairs(const lmrs_sample_args &a, hipStream_t s) {
  bf16_fast_rounds_kernel<40><<<dim3((a.batch + 1) / 2), dim3(kFT), 0, s>>>(a);
}

}  // namespace lmrs
