// launch.hpp -- host-side launchers of the sampling kernels, one translation
// unit per kernel family (fast_nch*.hip, generic_kernels.hip, f32_kernel.hip)
// so that the library's device code compiles in parallel.  Each launches one
// workgroup per row on `s`; the caller has checked the arguments.
#pragma once

#include <hip/hip_runtime.h>

#include "lmrs_sampling.h"

namespace lmrs {

constexpr int64_t kFastSlotLogits = 8 * 512;             // one 16-byte chunk per thread of 512
constexpr int64_t kFastVocabMax = 40 * kFastSlotLogits;  // the widest instantiation's rows

// bf16 rows of V <= 8 * 512 * NCH, V % 8 == 0, 16-byte aligned rows; one
// workgroup per row, or (the widest rows, batches of more rows than `grid`,
// the CU count) two rows per workgroup
void launch_fast_bf16_8(const lmrs_sample_args &a, int grid, hipStream_t s);
void launch_fast_bf16_16(const lmrs_sample_args &a, int grid, hipStream_t s);
void launch_fast_bf16_32(const lmrs_sample_args &a, int grid, hipStream_t s);
void launch_fast_bf16_40(const lmrs_sample_args &a, int grid, hipStream_t s);
void launch_fast_bf16_40_pairs(const lmrs_sample_args &a, hipStream_t s);  // two rows per workgroup
// bf16 rows of any shape
void launch_generic_bf16(const lmrs_sample_args &a, int vec, hipStream_t s);
// f32 rows
void launch_f32(const lmrs_sample_args &a, int vec, hipStream_t s);
// the processor chain alone, output in the input dtype
void launch_process(const lmrs_sample_args &a, void *out, hipStream_t s);

}  // namespace lmrs
