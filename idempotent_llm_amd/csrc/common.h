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

// One DPP move of a 64-bit value (two 32-bit halves, same control). Lanes the
// row mask disables keep `old`. CTRL: 0xB1 / 0x4E quad permutations (lane ^ 1,
// lane ^ 2), 0x141 row_half_mirror, 0x140 row_mirror, 0x142 row_bcast15,
// 0x143 row_bcast31 (CDNA data-parallel primitives).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ i64 dpp64(i64 v, i64 old) {
  const int lo = __builtin_amdgcn_update_dpp((int)(u64)old, (int)(u64)v, CTRL, ROW_MASK, 0xF,
                                             false);
  const int hi = __builtin_amdgcn_update_dpp((int)((u64)old >> 32), (int)((u64)v >> 32), CTRL,
                                             ROW_MASK, 0xF, false);
  return (i64)(((u64)(unsigned)hi << 32) | (u64)(unsigned)lo);
}

__device__ __forceinline__ i64 readlane64(i64 v, int lane) {
  const int lo = __builtin_amdgcn_readlane((int)(u64)v, lane);
  const int hi = __builtin_amdgcn_readlane((int)((u64)v >> 32), lane);
  return (i64)(((u64)(unsigned)hi << 32) | (u64)(unsigned)lo);
}

// Wave-wide max / wrapping sum with DPP moves (a few cycles each, against an
// LDS round trip per step for a shuffle). After the six steps lane 63 holds
// the result, which is broadcast. Integer max and modular sum are
// associative and commutative, so the combine order cannot change the value.
// Every lane of the wave must be active.
__device__ __forceinline__ i64 wave_max(i64 v) {
  v = imax(v, dpp64<0xB1, 0xF>(v, v));
  v = imax(v, dpp64<0x4E, 0xF>(v, v));
  v = imax(v, dpp64<0x141, 0xF>(v, v));
  v = imax(v, dpp64<0x140, 0xF>(v, v));
  v = imax(v, dpp64<0x142, 0xA>(v, v));
  v = imax(v, dpp64<0x143, 0xC>(v, v));
  return readlane64(v, 63);
}

__device__ __forceinline__ i64 wave_sum(i64 v) {
  v = wadd(v, dpp64<0xB1, 0xF>(v, 0));
  v = wadd(v, dpp64<0x4E, 0xF>(v, 0));
  v = wadd(v, dpp64<0x141, 0xF>(v, 0));
  v = wadd(v, dpp64<0x140, 0xF>(v, 0));
  v = wadd(v, dpp64<0x142, 0xA>(v, 0));
  v = wadd(v, dpp64<0x143, 0xC>(v, 0));
  return readlane64(v, 63);
}

// Sum over each aligned group of 8 lanes, result in all 8 (int32).
__device__ __forceinline__ int sum8_i32(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
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
