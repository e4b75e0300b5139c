// common.hpp -- device helpers shared by the sampling kernels (gfx950).
//
// Numerics follow the reference's device ops exactly: every processor op
// computes in f32 and rounds its result to bf16 with round-to-nearest-even
// (kernels/ops/activation_kernels.cuh:35-38 stores through __float2bfloat16;
// kernels/ffi/ops_ffi.cu:24-38, tensor_ffi.cu:43-90).  This file is compiled
// with -ffp-contract=off; the one fused op of the reference (affine, which
// the CUDA compiler contracts to an FMA) is spelled as __builtin_fmaf.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lmrs {

constexpr int kThreads = 1024;  // one workgroup per row: 16 waves of 64
constexpr int kWaves = kThreads / 64;

// ---- bf16 <-> f32 ----------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// Device-side rounding of an op result (NaN -> canonical 0x7FFF).
__device__ __forceinline__ uint32_t f32_to_bf16_dev(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FFFu;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Host-side rounding used for the reference's factor tensors
// (half::bf16::from_f32: NaN keeps sign and payload with the quiet bit).
__device__ __forceinline__ uint32_t f32_to_bf16_host(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return ((u >> 16) | 0x40u) & 0xFFFFu;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float round_bf16_dev(float f) { return bf16_to_f32(f32_to_bf16_dev(f)); }
__device__ __forceinline__ float round_bf16_host(float f) { return bf16_to_f32(f32_to_bf16_host(f)); }

// ---- total order keys (f32::total_cmp) -------------------------------------
// Unsigned comparison of keys equals IEEE totalOrder of the values.

__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __uint_as_float(u);
}

// ---- wave / block collectives ----------------------------------------------

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    T w = __shfl_xor(v, o, 64);
    v = w > v ? w : v;
  }
  return v;
}

template <typename T>
__device__ __forceinline__ T wave_min(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    T w = __shfl_xor(v, o, 64);
    v = w < v ? w : v;
  }
  return v;
}

// Block-wide reductions.  `scratch` holds kWaves elements of T; every
// thread returns the result.  Contains two barriers.
template <typename T>
__device__ T block_sum(T v, T *scratch) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  T r = scratch[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) r += scratch[i];
  return r;
}

template <typename T>
__device__ T block_max(T v, T *scratch) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  T r = scratch[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) r = scratch[i] > r ? scratch[i] : r;
  return r;
}

template <typename T>
__device__ T block_min(T v, T *scratch) {
  v = wave_min(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  T r = scratch[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) r = scratch[i] < r ? scratch[i] : r;
  return r;
}

// Exclusive prefix sum over the block in thread order.  Returns the
// exclusive prefix of `v`; *total receives the block total.  Two barriers.
template <typename T>
__device__ T block_exclusive_scan(T v, T *scratch, T *total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  T x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    T y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  __syncthreads();
  if (lane == 63) scratch[wave] = x;
  __syncthreads();
  T excl = __shfl_up(x, 1, 64);
  if (lane == 0) excl = T(0);
  T off = T(0), tot = T(0);
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    T s = scratch[i];
    if (i < wave) off += s;
    tot += s;
  }
  *total = tot;
  return off + excl;
}

}  // namespace lmrs
