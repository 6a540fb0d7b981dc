// Device-side helpers shared by the DetLLM HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "intops.h"

#define DI_WAVE 64
#define DI_ROW_THREADS 256

// Error codes returned by every extern "C" entry point (0 = success,
// > 0 = the hipError_t of a failed launch, < 0 = argument errors).
#define DI_OK 0
#define DI_EINVAL (-22)
#define DI_ERANGE (-34)
#define DI_ENOSYS (-38)

#define DI_LAUNCH_CHECK()                          \
  do {                                             \
    hipError_t e_ = hipGetLastError();             \
    if (e_ != hipSuccess) return (int)e_;          \
  } while (0)

namespace di {

__device__ __forceinline__ i64 shfl_xor64(i64 v, int mask) {
  int lo = (int)(v & 0xffffffff);
  int hi = (int)((u64)v >> 32);
  lo = __shfl_xor(lo, mask, DI_WAVE);
  hi = __shfl_xor(hi, mask, DI_WAVE);
  return (i64)(((u64)(unsigned)hi << 32) | (u64)(unsigned)lo);
}

__device__ __forceinline__ i64 wave_max(i64 v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = imax(v, shfl_xor64(v, o));
  return v;
}

__device__ __forceinline__ i64 wave_sum(i64 v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = wadd(v, shfl_xor64(v, o));
  return v;
}

// Reductions over the lanes that share (lane % 16): masks 16 and 32.
__device__ __forceinline__ i64 group4_max(i64 v) {
  v = imax(v, shfl_xor64(v, 16));
  return imax(v, shfl_xor64(v, 32));
}
__device__ __forceinline__ i64 group4_sum(i64 v) {
  v = wadd(v, shfl_xor64(v, 16));
  return wadd(v, shfl_xor64(v, 32));
}

// Block-wide reductions (blockDim.x a multiple of 64, <= 1024). `red` is a
// __shared__ i64[16]; the leading barrier makes back-to-back calls safe.
__device__ __forceinline__ i64 block_max(i64 v, i64* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  i64 r = red[0];
  const int nw = blockDim.x >> 6;
  for (int i = 1; i < nw; ++i) r = imax(r, red[i]);
  return r;
}

__device__ __forceinline__ i64 block_sum(i64 v, i64* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  i64 r = red[0];
  const int nw = blockDim.x >> 6;
  for (int i = 1; i < nw; ++i) r = wadd(r, red[i]);
  return r;
}

__device__ __forceinline__ i64 to_i32(i64 v) { return (i64)(int32_t)(uint32_t)(u64)v; }

}  // namespace di
