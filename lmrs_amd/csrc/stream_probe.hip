// stream_probe.hip -- a read-only kernel with the sampler's access shape, for
// the measured streaming ceiling that bench.py reports beside the 8 TB/s peak.
//
// One workgroup of 512 threads per row; thread t reads 16-byte chunks
// s * 512 + t of its row, NCH slots, each as an inline-asm global_load_dwordx4
// with the non-temporal hint, kAhead slots in flight; every load is waited
// for with an explicit vmcnt before its data is used (the bf16 kernel's load
// pass without its work).  The row's chunk-wise maximum word is written out so
// the loads cannot be dropped.  Not part of the sampling ABI.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kT = 512;
constexpr int kAhead = 8;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 load_nt(const void *p) {
  u32x4 d;
  asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(d) : "v"(p));
  return d;
}

template <int N>
__device__ __forceinline__ void wait_for(u32x4 &d) {
  asm volatile("s_waitcnt vmcnt(%1)" : "+v"(d) : "n"(N));
}

template <int I>
struct Ix {
  static constexpr int value = I;
};
template <int B, int E, class F>
__device__ __forceinline__ void unrolled(F &&f) {
  if constexpr (B < E) {
    f(Ix<B>{});
    unrolled<B + 1, E>(f);
  }
}

template <int NCH>
__global__ void __launch_bounds__(kT) probe_kernel(const uint4 *base, int64_t stride_chunks, int nchunks,
                                                   uint32_t *out) {
  __shared__ uint32_t red[kT / 64];
  const int t = threadIdx.x;
  const uint4 *row = base + (int64_t)blockIdx.x * stride_chunks;
  const uint4 *last = row + (nchunks - 1);
  auto addr = [&](int s) {
    const int c = s * kT + t;
    return c < nchunks ? row + c : last;
  };
  u32x4 v[NCH];
  constexpr int kPre = kAhead < NCH ? kAhead : NCH;
  unrolled<0, kPre>([&](auto S) { v[decltype(S)::value] = load_nt(addr(decltype(S)::value)); });
  uint32_t m = 0u;
  unrolled<0, NCH>([&](auto S) {
    constexpr int s = decltype(S)::value;
    if constexpr (s + kAhead < NCH) v[s + kAhead] = load_nt(addr(s + kAhead));
    constexpr int issued = (s + kAhead < NCH) ? s + kAhead : NCH - 1;
    wait_for<issued - s>(v[s]);
    m = max(m, max(max(v[s].x, v[s].y), max(v[s].z, v[s].w)));
  });
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o));
  if ((t & 63) == 0) red[t >> 6] = m;
  __syncthreads();
  if (t == 0) {
    uint32_t r = red[0];
    for (int i = 1; i < kT / 64; ++i) r = max(r, red[i]);
    out[blockIdx.x] = r;
  }
}

}  // namespace

// Reads `rows` rows of `row_bytes` bytes (a multiple of 16, at most 40 * 512
// chunks of 16 bytes), `stride_bytes` apart, from 16-byte aligned device
// memory; writes one word per row to out.  0 on success, -1 on bad arguments,
// -4 if the launch failed.
extern "C" int lmrs_stream_probe(const void *base, int64_t row_bytes, int64_t stride_bytes, int32_t rows,
                                 uint32_t *out, void *stream) {
  if (!base || !out || rows <= 0 || row_bytes <= 0 || row_bytes % 16 || stride_bytes % 16 ||
      stride_bytes < row_bytes || ((uintptr_t)base) % 16)
    return -1;
  const int64_t nchunks = row_bytes / 16;
  const dim3 grid(rows), block(kT);
  hipStream_t s = (hipStream_t)stream;
  const uint4 *b = (const uint4 *)base;
  const int64_t st = stride_bytes / 16;
  if (nchunks <= 8 * kT)
    probe_kernel<8><<<grid, block, 0, s>>>(b, st, (int)nchunks, out);
  else if (nchunks <= 16 * kT)
    probe_kernel<16><<<grid, block, 0, s>>>(b, st, (int)nchunks, out);
  else if (nchunks <= 32 * kT)
    probe_kernel<32><<<grid, block, 0, s>>>(b, st, (int)nchunks, out);
  else if (nchunks <= 40 * kT)
    probe_kernel<40><<<grid, block, 0, s>>>(b, st, (int)nchunks, out);
  else
    return -1;
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
