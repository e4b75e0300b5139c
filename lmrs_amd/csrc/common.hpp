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

constexpr int kThreads = 1024;  // workgroup of the generic engine: 16 waves of 64
constexpr int kWaves = kThreads / 64;  // the most waves any workgroup here has

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

// ---- uniform values -------------------------------------------------------
// Values that every lane holds identically (block reductions, LDS
// broadcasts) are moved to scalar registers, so that branches on them are
// uniform to the compiler as well: an early return then really leaves, and
// values live only on the other side of a branch do not stay live across it.

__device__ __forceinline__ uint32_t uniform(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int32_t uniform(int32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float uniform(float v) {
  return __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(v)));
}
__device__ __forceinline__ uint64_t uniform(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ int64_t uniform(int64_t v) { return (int64_t)uniform((uint64_t)v); }
__device__ __forceinline__ double uniform(double v) {
  return __longlong_as_double((long long)uniform((uint64_t)__double_as_longlong(v)));
}

// ---- wave / block collectives ----------------------------------------------
// Wave-level steps use DPP lane moves (row_shr within rows of 16 lanes, then
// row_bcast:15 / row_bcast:31 across rows), which complete in a few cycles,
// instead of LDS-routed shuffles.  Lanes a DPP move cannot source keep `old`
// (bound_ctrl off), which is chosen as the operation's identity.

template <int CTRL, int ROWMASK = 0xF>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROWMASK, 0xF, false);
}

constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118;
constexpr int kRowBcast15 = 0x142, kRowBcast31 = 0x143;

struct OpSum {
  template <class T> __device__ static T apply(T a, T b) { return a + b; }
};
struct OpMax {
  template <class T> __device__ static T apply(T a, T b) { return a > b ? a : b; }
};
struct OpMin {
  template <class T> __device__ static T apply(T a, T b) { return a < b ? a : b; }
};
struct OpOr {
  template <class T> __device__ static T apply(T a, T b) { return a | b; }
};

template <class T>
struct Bits;
template <>
struct Bits<uint32_t> {
  template <int C, int M = 0xF>
  __device__ static uint32_t mov(uint32_t old, uint32_t v) { return dpp_mov<C, M>(old, v); }
};
template <>
struct Bits<int32_t> {
  template <int C, int M = 0xF>
  __device__ static int32_t mov(int32_t old, int32_t v) { return (int32_t)dpp_mov<C, M>((uint32_t)old, (uint32_t)v); }
};
template <>
struct Bits<uint64_t> {
  template <int C, int M = 0xF>
  __device__ static uint64_t mov(uint64_t old, uint64_t v) {
    const uint32_t lo = dpp_mov<C, M>((uint32_t)old, (uint32_t)v);
    const uint32_t hi = dpp_mov<C, M>((uint32_t)(old >> 32), (uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
  }
};
template <>
struct Bits<double> {
  template <int C, int M = 0xF>
  __device__ static double mov(double old, double v) {
    return __longlong_as_double((long long)Bits<uint64_t>::mov<C, M>((uint64_t)__double_as_longlong(old),
                                                                      (uint64_t)__double_as_longlong(v)));
  }
};

// Inclusive scan across the 64 lanes of a wave (lane 63 holds the total).
template <class Op, class T>
__device__ __forceinline__ T wave_inclusive(T v, T id) {
  v = Op::apply(v, Bits<T>::template mov<kRowShr1>(id, v));
  v = Op::apply(v, Bits<T>::template mov<kRowShr2>(id, v));
  v = Op::apply(v, Bits<T>::template mov<kRowShr4>(id, v));
  v = Op::apply(v, Bits<T>::template mov<kRowShr8>(id, v));
  v = Op::apply(v, Bits<T>::template mov<kRowBcast15, 0xA>(id, v));
  v = Op::apply(v, Bits<T>::template mov<kRowBcast31, 0xC>(id, v));
  return v;
}

template <class T>
__device__ __forceinline__ T lane63(T v) {
  if constexpr (sizeof(T) == 8) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)u, 63);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(u >> 32), 63);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  } else {
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(uint32_t, v), 63));
  }
}

template <class T>
__device__ __forceinline__ T wave_sum(T v) { return lane63(wave_inclusive<OpSum>(v, T(0))); }
template <class T>
__device__ __forceinline__ T wave_max(T v) { return lane63(wave_inclusive<OpMax>(v, T(0))); }
__device__ __forceinline__ int32_t wave_max(int32_t v) { return lane63(wave_inclusive<OpMax>(v, (int32_t)0x80000000)); }
template <class T>
__device__ __forceinline__ T wave_min(T v) { return lane63(wave_inclusive<OpMin>(v, (T)~T(0))); }
__device__ __forceinline__ int32_t wave_min(int32_t v) { return lane63(wave_inclusive<OpMin>(v, (int32_t)0x7FFFFFFF)); }

// Block-wide reductions over NW waves.  `scratch` holds NW elements of T;
// every thread returns the (scalar) result.  Contains two barriers.
template <int NW, class Op, class T>
__device__ __forceinline__ T block_reduce(T w, T *scratch) {
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = w;
  __syncthreads();
  T r = scratch[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = Op::apply(r, scratch[i]);
  return uniform(r);
}

template <int NW = kWaves, typename T>
__device__ __forceinline__ T block_sum(T v, T *scratch) { return block_reduce<NW, OpSum>(wave_sum(v), scratch); }
template <int NW = kWaves, typename T>
__device__ __forceinline__ T block_max(T v, T *scratch) { return block_reduce<NW, OpMax>(wave_max(v), scratch); }
template <int NW = kWaves, typename T>
__device__ __forceinline__ T block_min(T v, T *scratch) { return block_reduce<NW, OpMin>(wave_min(v), scratch); }

// Exclusive prefix sum over the block (NW waves) in thread order.  Returns
// the exclusive prefix of `v`; *total receives the block total.  Two barriers.
template <int NW = kWaves, typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T *scratch, T *total) {
  const int wave = threadIdx.x >> 6;
  const T incl = wave_inclusive<OpSum>(v, T(0));
  const T wtot = lane63(incl);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[wave] = wtot;
  __syncthreads();
  T off = T(0), tot = T(0);
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const T s = scratch[i];
    if (i < wave) off += s;
    tot += s;
  }
  *total = uniform(tot);
  return off + (incl - v);
}

// The row of workgroup b in a launch of n.  The dispatcher hands workgroup b
// to XCD b mod 8; within each full group of eight workgroups the rows are
// permuted by the group index, so that an XCD's rows are not a fixed residue
// of the row index.  Measured on MI355X (same-box A/B, cold HBM): the C3 step
// (256 rows of 128256 bf16) drops from 22.3 to 21.6 us; C2 and C4 move by a
// few percent either way.  A bijection on [0, n).
__device__ __forceinline__ int xcd_spread_row(int b, int n) {
  const int g = b >> 3;
  if ((g + 1) * 8 > n) return b;
  return (g << 3) | ((b & 7) ^ (g & 7));
}

// The rows of slots in rounds of G: slot s runs on the CU of slot s mod G
// (a persistent workgroup's slots s, s + G, ...; with one workgroup per row
// and G = the CU count, MI355X's dispatcher gave CU c exactly the workgroups
// c, c + 256, ... of a 1024-row launch, one workgroup per CU fitting its
// LDS).  Every other round takes its rows in reverse order, so that the rows
// of one CU come from both ends of each pair of rounds: alternating and
// half-and-half batches of cheap and costly rows (C4's greedy and
// multinomial rows) give every CU the same mix.  Within a round, the XCD
// spread as above.  A bijection from slots [0, n) to rows.
constexpr int kRoundWGs = 256;  // MI355X CUs: the rounds of a launch of one workgroup per row
__device__ __forceinline__ int round_row(int slot, int n, int G) {
  const int x = xcd_spread_row(slot, n);
  const int base = x / G * G;
  if ((x / G) % 2 == 0 || base + G > n) return x;
  return base + (G - 1) - (x - base);
}
}  // namespace lmrs
