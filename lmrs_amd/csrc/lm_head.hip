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
// blocks: 32 MFMA accumulators of four floats per lane).  The operand layout
// of the 16x16x32 bf16 MFMA: lane l of a block holds row (or column) l % 16
// and k = 8 (l / 16) .. + 7; the result gives lane l the column l % 16 and
// rows 4 (l / 16) .. + 3.
//
// The k loop runs over tiles of 64 k.  A tile's operands, the workgroup's
// 256 rows of x and its 128 weight columns (the weight bytes bound the
// projection and are read from HBM once per launch), are loaded once per
// workgroup, each thread fetching twelve 16-byte chunks, and stored to LDS,
// where the waves read their A and B fragments; lines are padded to 144
// bytes so the 16 lanes reading one k chunk of 16 consecutive lines spread
// over the banks.  Two LDS buffers alternate (one read by the MFMAs while
// the next tile is stored to the other, one barrier per tile), and the
// loads run two tiles ahead of the MFMAs in two register sets.  Measured at
// 256 x 4096 x 128256: 799 us with each wave loading its own fragments, 567
// us with the weight tile in LDS, 527 us with the reduction below on DPP and
// the loads two tiles ahead, 459 us with x in LDS too, 15 us less again
// with the epilogue below skipping per-element range tests for whole tiles
// (a plain hipBLASLt GEMM of the same shape, without the epilogue: 336 us).
//
// Epilogue: the logits are rounded to bf16 (round to nearest even) and
// stored, and for every row the largest logit of each 64-column tile is
// reduced across the lanes that hold it, in the sampler's total order
// (the key of crates/sampling/src/strategies/mod.rs:21-25's total_cmp, ties
// to the lower column): tile_max[r, t] = key << 32 | ~column.  The
// reduction runs on 32-bit entries key << 16 | (0xFFFF - column % 64), which
// order as the stored form does, over the 16 lanes of a DPP row.  The row
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
constexpr int kTileCols = 64;                         // columns per tile_max entry

// Total-order key of a bf16 pattern (larger key = later in the reference's
// descending sort): flip negatives, set the sign bit of non-negatives.
__device__ __forceinline__ uint32_t bf16_key(uint32_t b) {
  return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
}

__device__ __forceinline__ uint32_t umax32(uint32_t a, uint32_t b) { return a > b ? a : b; }

// A k tile: kLhTileK k (two MFMA k steps), one 128-byte line of it per row
// of x or column of w, stored every kLhColStride bytes in LDS (padded
// against bank conflicts).
constexpr int kLhTileK = 2 * kLhStep;
constexpr int kLhColStride = kLhTileK * 2 + 16;
constexpr int kLhColChunks = kLhTileK / 8;  // 16-byte chunks of a line

// Both operands of a k tile in LDS: the workgroup's kLhRows rows of x, then
// its kLhCols weight columns, one padded 128-byte line each.
constexpr int kLhLines = kLhRows + kLhCols;
constexpr int kLhBufBytes = kLhLines * kLhColStride;
constexpr int kLhLineChunksPer = kLhLines * kLhColChunks / kLhThreads;  // 16-byte chunks per thread
constexpr int kLhXChunksPer = kLhRows * kLhColChunks / kLhThreads;      // of which x
static_assert(kLhLines * kLhColChunks % kLhThreads == 0 && kLhRows * kLhColChunks % kLhThreads == 0, "chunks");

__global__ void __launch_bounds__(kLhThreads) lm_head_kernel(uint16_t *__restrict__ out, const uint16_t *__restrict__ x,
                                                           const uint16_t *__restrict__ w, int rows, int K, int V,
                                                           uint64_t *__restrict__ tile_max) {
  __shared__ __attribute__((aligned(16))) unsigned char tb[2][kLhBufBytes];
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int col0 = (int)blockIdx.x * kLhCols;
  const int xrow0 = (int)blockIdx.y * kLhRows;
  const int row0 = xrow0 + wave * kLhRowsPerWave;
  const int li = lane & 15;  // operand row/column in a block

  f32x4 acc[kLhRB][kLhCB];
#pragma unroll
  for (int i = 0; i < kLhRB; ++i)
#pragma unroll
    for (int j = 0; j < kLhCB; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // this thread's chunks of a tile: line c / kLhColChunks (x rows first),
  // k chunk c % kLhColChunks.  Two register sets: the tile two ahead is in
  // flight in one while the other (the next tile, issued an iteration
  // earlier) lands and is stored to LDS.  Chunks past K or past the last
  // row / column load a clamped address (in bounds: K > 0 is a multiple of
  // 8, rows and V are positive) and store zeros.
  u32x4v s0[kLhLineChunksPer], s1[kLhLineChunksPer];
  auto fetch = [&](int k0, u32x4v (&st)[kLhLineChunksPer]) {
#pragma unroll
    for (int q = 0; q < kLhLineChunksPer; ++q) {
      const int c = tid + q * kLhThreads, line = c / kLhColChunks, k = k0 + (c % kLhColChunks) * 8;
      const int kc = k < K ? k : 0;
      if (q < kLhXChunksPer) {
        const int r = xrow0 + line, rc = r < rows ? r : rows - 1;
        st[q] = *(const u32x4v *)(x + (int64_t)rc * K + kc);
      } else {
        const int col = col0 + line - kLhRows, cc = col < V ? col : V - 1;
        st[q] = *(const u32x4v *)(w + (int64_t)cc * K + kc);
      }
    }
  };
  auto store = [&](int k0, const u32x4v (&st)[kLhLineChunksPer], int buf) {
#pragma unroll
    for (int q = 0; q < kLhLineChunksPer; ++q) {
      const int c = tid + q * kLhThreads, line = c / kLhColChunks, k = k0 + (c % kLhColChunks) * 8;
      const bool in = (q < kLhXChunksPer ? xrow0 + line < rows : col0 + line - kLhRows < V) && k < K;
      const u32x4v z = {0u, 0u, 0u, 0u};
      *(u32x4v *)&tb[buf][line * kLhColStride + (c % kLhColChunks) * 16] = in ? st[q] : z;
    }
  };
  auto frag = [&](int buf, int line, int h) {
    return __builtin_bit_cast(bf16x8, *(const u32x4v *)&tb[buf][line * kLhColStride + h * 64 + (lane >> 4) * 16]);
  };
  // one tile: issue tile t + 2 into `fill`, run tile t's MFMAs from LDS
  // buffer `buf`, store tile t + 1 (in `land`) to the other buffer
  auto tile = [&](int k0, u32x4v (&fill)[kLhLineChunksPer], const u32x4v (&land)[kLhLineChunksPer], int buf) {
    fetch(k0 + 2 * kLhTileK, fill);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      bf16x8 av[kLhRB], b[kLhCB];
#pragma unroll
      for (int i = 0; i < kLhRB; ++i) av[i] = frag(buf, wave * kLhRowsPerWave + 16 * i + li, h);
#pragma unroll
      for (int j = 0; j < kLhCB; ++j) b[j] = frag(buf, kLhRows + 16 * j + li, h);
#pragma unroll
      for (int i = 0; i < kLhRB; ++i)
#pragma unroll
        for (int j = 0; j < kLhCB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i], b[j], acc[i][j], 0, 0, 0);
    }
    store(k0 + kLhTileK, land, buf ^ 1);
    __syncthreads();  // the other buffer is written; this one's reads are done
  };
  if (K > 0) {  // (K = 0: no weight row to clamp to; the logits are zeros)
    fetch(0, s0);
    fetch(kLhTileK, s1);
    store(0, s0, 0);
    __syncthreads();
    for (int k0 = 0; k0 < K; k0 += 2 * kLhTileK) {
      tile(k0, s0, s1, 0);
      if (k0 + kLhTileK < K) tile(k0 + kLhTileK, s1, s0, 1);
    }
  }

  // Epilogue.  Lane l holds column 16 j + l % 16 and rows 16 i + 4 (l / 16) + q.
  const int ntiles = (V + kTileCols - 1) / kTileCols;
  // every row and column of this wave's tile in range (the common case): no per-element test
  const bool whole = row0 + kLhRowsPerWave <= rows && col0 + kLhCols <= V;
  const uint32_t lowc = 0xFFFFu - (uint32_t)li;  // 0xFFFF - column % 64 in a tile's first block
#pragma unroll
  for (int i = 0; i < kLhRB; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = row0 + 16 * i + 4 * (lane >> 4) + q;
      // per 64-column tile (blocks 0-3 and 4-7): this lane's best of its four columns
      uint32_t best[2] = {0u, 0u};
      uint16_t *orow = out + (int64_t)row * V + col0 + li;
      if (whole) {
#pragma unroll
        for (int j = 0; j < kLhCB; ++j) {
          const uint32_t bits = f32_to_bf16_dev(acc[i][j][q]);
          orow[16 * j] = (uint16_t)bits;
          const uint32_t e = (bf16_key(bits) << 16) | (lowc - 16u * (uint32_t)(j % 4));
          best[j / 4] = e > best[j / 4] ? e : best[j / 4];
        }
      } else {
#pragma unroll
        for (int j = 0; j < kLhCB; ++j) {
          const int col = col0 + 16 * j + li;
          const uint32_t bits = f32_to_bf16_dev(acc[i][j][q]);
          if (row < rows && col < V) {
            orow[16 * j] = (uint16_t)bits;
            const uint32_t e = (bf16_key(bits) << 16) | (0xFFFFu - (uint32_t)(col % kTileCols));
            best[j / 4] = e > best[j / 4] ? e : best[j / 4];
          }
        }
      }
      if (tile_max) {
        // across the 16 lanes of this row (lanes 16 g .. 16 g + 15, one DPP
        // row): 32-bit entries key << 16 | (0xFFFF - column % 64), the same
        // order as the stored form; quad swaps, then the half-row and row
        // mirrors reach all 16 lanes.  Out-of-range lanes hold 0.
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          uint32_t v = best[t];
          v = umax32(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
          v = umax32(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
          v = umax32(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));  // row_half_mirror
          v = umax32(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));  // row_mirror
          const int tile = (col0 / kTileCols) + t;
          if (li == 0 && row < rows && tile < ntiles && v != 0u) {
            const uint32_t col = (uint32_t)(tile * kTileCols) + (0xFFFFu - (v & 0xFFFFu));
            tile_max[(int64_t)row * ntiles + tile] = ((uint64_t)(v >> 16) << 32) | (uint32_t)~col;
          }
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
