// lm_head.hip -- the LM head's vocabulary projection with the sampling
// prologue in its epilogue (lmrs_lm_head_fwd, include/lmrs_sampling.h).
//
// logits[r, v] = bf16( sum_k x[r, k] * w[v, k] ), bf16 inputs, f32
// accumulation, as LmHead::forward -> kernels::linear -> linear_fwd
// (crates/ops/src/embedding/lm_head.rs:33-35, kernels/ffi/tensor_ffi.cu:230-258,
// 820-841) computes it for bf16 without bias, on the MFMA units: each
// v_mfma_f32_16x16x32_bf16 multiplies a 16 x 32 tile of x by a 32 x 16 tile
// of w^T.  The f32 sums run in the matrix unit's order rather than the
// reference's one-product-at-a-time order, so a logit may differ from the
// reference's by the rounding of the sum (an ulp of bf16 where the two f32
// sums straddle a rounding boundary).
//
// Layout: a workgroup of four waves owns 128 vocabulary columns and up to 256
// rows (wave w: rows 64 w .. 64 w + 63, in four 16-row blocks; eight 16-column
// blocks: 32 MFMA accumulators of four floats per lane).  Each lane reads its
// operands straight from HBM/L2 as 16-byte loads (eight bf16 along k): lane l
// of a block holds row (or column) l % 16 and k = 8 (l / 16) .. + 7, the
// operand layout of the 16x16x32 bf16 MFMA, whose result gives lane l the
// column l % 16 and rows 4 (l / 16) .. + 3.  The weight matrix (the bytes
// that bound the projection) is read once per launch; the four waves of a
// workgroup read the same weight fragments, served by the CU's L1 after the
// first.  The k loop keeps the next kLhDepth steps' fragments in flight while
// a step's 32 MFMAs run (with one step in flight the projection was bound by
// the loads' latency: 807 us at 256 x 4096 x 128256).
//
// Epilogue: the logits are rounded to bf16 (round to nearest even) and
// stored, and for every row the largest logit of each 64-column tile is
// reduced across the lanes that hold it, in the sampler's total order
// (the key of crates/sampling/src/strategies/mod.rs:21-25's total_cmp, ties
// to the lower column): tile_max[r, t] = key << 32 | ~column.  The row
// maximum and greedy's token are the maximum of a row's tile entries; the
// tile maxima also bound a top-k cut from below, without a read of the logits.
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "lmrs_sampling.h"

namespace lmrs {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

constexpr int kLhWaves = 4;
constexpr int kLhThreads = 64 * kLhWaves;
constexpr int kLhRowsPerWave = 64;                    // four 16-row blocks
constexpr int kLhRows = kLhRowsPerWave * kLhWaves;    // rows of one workgroup (grid.y covers more)
constexpr int kLhCols = 128;                          // eight 16-column blocks
constexpr int kLhRB = kLhRowsPerWave / 16, kLhCB = kLhCols / 16;
constexpr int kLhStep = 32;                           // k per MFMA
constexpr int kLhDepth = 4;                           // k steps of fragments in flight
constexpr int kTileCols = 64;                         // columns per tile_max entry

// Total-order key of a bf16 pattern (larger key = later in the reference's
// descending sort): flip negatives, set the sign bit of non-negatives.
__device__ __forceinline__ uint32_t bf16_key(uint32_t b) {
  return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
}

// Eight bf16 of row `p` from k (zeros where the row or k is out of range).
__device__ __forceinline__ bf16x8 load8(const uint16_t *base, int64_t ld, int row, int nrows, int k, int K) {
  if (row < nrows && k < K) {
    const u32x4v v = *(const u32x4v *)(base + (int64_t)row * ld + k);
    return __builtin_bit_cast(bf16x8, v);
  }
  return __builtin_bit_cast(bf16x8, u32x4v{0u, 0u, 0u, 0u});
}

__global__ void __launch_bounds__(kLhThreads) lm_head_kernel(uint16_t *__restrict__ out, const uint16_t *__restrict__ x,
                                                           const uint16_t *__restrict__ w, int rows, int K, int V,
                                                           uint64_t *__restrict__ tile_max) {
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
  const int col0 = (int)blockIdx.x * kLhCols;
  const int row0 = (int)blockIdx.y * kLhRows + wave * kLhRowsPerWave;
  const int li = lane & 15, lk = (lane >> 4) * 8;  // operand row/column in a block, k offset

  f32x4 acc[kLhRB][kLhCB];
#pragma unroll
  for (int i = 0; i < kLhRB; ++i)
#pragma unroll
    for (int j = 0; j < kLhCB; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // kLhDepth k steps of fragments in flight: step d of each group of
  // kLhDepth steps uses register set d, which is refilled with the step
  // kLhDepth ahead right after its MFMAs (the compiler waits for each set's
  // own loads only).  Steps past K load zeros.
  bf16x8 a[kLhDepth][kLhRB], b[kLhDepth][kLhCB];
  auto fetch = [&](int k0, bf16x8 (&fa)[kLhRB], bf16x8 (&fb)[kLhCB]) {
#pragma unroll
    for (int i = 0; i < kLhRB; ++i) fa[i] = load8(x, K, row0 + 16 * i + li, rows, k0 + lk, K);
#pragma unroll
    for (int j = 0; j < kLhCB; ++j) fb[j] = load8(w, K, col0 + 16 * j + li, V, k0 + lk, K);
  };
#pragma unroll
  for (int d = 0; d < kLhDepth; ++d) fetch(d * kLhStep, a[d], b[d]);
  for (int k0 = 0; k0 < K; k0 += kLhDepth * kLhStep) {
#pragma unroll
    for (int d = 0; d < kLhDepth; ++d) {
#pragma unroll
      for (int i = 0; i < kLhRB; ++i)
#pragma unroll
        for (int j = 0; j < kLhCB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[d][i], b[d][j], acc[i][j], 0, 0, 0);
      fetch(k0 + (d + kLhDepth) * kLhStep, a[d], b[d]);
    }
  }

  // Epilogue.  Lane l holds column 16 j + l % 16 and rows 16 i + 4 (l / 16) + q.
  const int ntiles = (V + kTileCols - 1) / kTileCols;
#pragma unroll
  for (int i = 0; i < kLhRB; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = row0 + 16 * i + 4 * (lane >> 4) + q;
      // per 64-column tile (blocks 0-3 and 4-7): this lane's best of its four columns
      uint64_t best[2] = {0u, 0u};
#pragma unroll
      for (int j = 0; j < kLhCB; ++j) {
        const int col = col0 + 16 * j + li;
        const uint32_t bits = f32_to_bf16_dev(acc[i][j][q]);
        if (row < rows && col < V) {
          out[(int64_t)row * V + col] = (uint16_t)bits;
          const uint64_t e = ((uint64_t)bf16_key(bits) << 32) | (uint32_t)~(uint32_t)col;
          best[j / 4] = e > best[j / 4] ? e : best[j / 4];
        }
      }
      if (tile_max) {
        // across the 16 lanes of this row (lanes 16 g .. 16 g + 15)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          uint64_t v = best[t];
#pragma unroll
          for (int off = 8; off >= 1; off >>= 1) {
            const uint64_t o = (uint64_t)__shfl_xor((unsigned long long)v, off, 16);
            v = o > v ? o : v;
          }
          const int tile = (col0 / kTileCols) + t;
          if (li == 0 && row < rows && tile < ntiles && v != 0u) tile_max[(int64_t)row * ntiles + tile] = v;
        }
      }
    }
  }
}

}  // namespace
}  // namespace lmrs

extern "C" int lmrs_lm_head_fwd(void *out, const void *input, const void *weight, int32_t rows, int32_t in_features,
                                int32_t out_features, int32_t dtype, uint64_t *tile_max, void *stream) {
  if (dtype != LMRS_DTYPE_BF16) return LMRS_ERR_BAD_DTYPE;
  if (rows < 0 || in_features < 0 || out_features < 0) return LMRS_ERR_BAD_SHAPE;
  if (rows == 0 || out_features == 0) return LMRS_OK;
  if (!out || !weight || (in_features > 0 && !input)) return LMRS_ERR_NULL_ARGUMENT;
  // 16-byte operand loads: k in steps of eight, 16-byte aligned rows
  if (in_features % 8 != 0) return LMRS_ERR_BAD_SHAPE;
  if (((uintptr_t)input | (uintptr_t)weight) % 16 != 0 || ((uintptr_t)out) % 2 != 0) return LMRS_ERR_ALIGNMENT;
  const dim3 grid((unsigned)((out_features + lmrs::kLhCols - 1) / lmrs::kLhCols),
                  (unsigned)((rows + lmrs::kLhRows - 1) / lmrs::kLhRows));
  lmrs::lm_head_kernel<<<grid, lmrs::kLhThreads, 0, (hipStream_t)stream>>>(
      (uint16_t *)out, (const uint16_t *)input, (const uint16_t *)weight, rows, in_features, out_features, tile_max);
  return hipGetLastError() == hipSuccess ? LMRS_OK : LMRS_ERR_LAUNCH;
}
