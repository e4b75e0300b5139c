// f32_kernel.hip -- the f32 sampling kernel.
#include "f32_dist.hpp"
#include "launch.hpp"

namespace lmrs {

void launch_f32(const lmrs_sample_args &a, int vec, hipStream_t s) {
  f32_sample_kernel<<<a.batch, kThreads, 0, s>>>(a, vec);
}

}  // namespace lmrs
