// generic_kernels.hip -- the generic bf16 sampling kernel and the processor-chain kernels.
#include "generic_engine.hpp"
#include "launch.hpp"

namespace lmrs {

void launch_generic_bf16(const lmrs_sample_args &a, int vec, hipStream_t s) {
  generic_sample_kernel<LMRS_DTYPE_BF16><<<a.batch, kThreads, 0, s>>>(a, vec);
}

void launch_process(const lmrs_sample_args &a, void *out, hipStream_t s) {
  if (a.dtype == LMRS_DTYPE_BF16)
    process_kernel<LMRS_DTYPE_BF16><<<a.batch, kThreads, 0, s>>>(a, out);
  else
    process_kernel<LMRS_DTYPE_F32><<<a.batch, kThreads, 0, s>>>(a, out);
}

}  // namespace lmrs
