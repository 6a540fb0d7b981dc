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

// Bits of the device error word (an int32 the caller passes as `err`):
// an index the reference would reject with IndexError.
#define DI_ERR_TOKEN 1     // token id outside [-vocab, vocab)
#define DI_ERR_POSITION 2  // position outside [-max_pos, max_pos)
#define DI_ERR_SLOTS 4     // device slot count beyond the launch's slot bound

// Slots per page of the paged KV cache.
#define DI_PAGE 128

namespace di {

// The paged int8 KV cache of one layer. A row's slot s lives in page
// table[b][s / DI_PAGE] (-1: not mapped) at offset s % DI_PAGE; pages hold
// every kv head:
//   K page [n_kv][DI_PAGE][128]   (a slot's K row: 128 contiguous bytes)
//   V page [n_kv][128][DI_PAGE]   (V transposed: a channel's slots contiguous)
// so both attention passes read slot-contiguous bytes, as the contiguous
// layout did, and a page is the unit a growing cache hands out.
struct KVPages {
  int8_t* k;
  int8_t* v;
  const int32_t* table;  // [B][width]
  int width;             // pages per row
  int n_kv;

  __device__ __forceinline__ i64 cap() const { return (i64)width * DI_PAGE; }
  // page of row b's slot s (-1 when s is outside the table or not mapped)
  __device__ __forceinline__ int page(int b, i64 s) const {
    return (s >= 0 && s < cap()) ? table[(i64)b * width + (s >> 7)] : -1;
  }
  __device__ __forceinline__ int8_t* krow(int pg, int h, int off) const {
    return k + (((i64)pg * n_kv + h) * DI_PAGE + off) * 128;
  }
  __device__ __forceinline__ int8_t* vchan(int pg, int h, int d) const {
    return v + (((i64)pg * n_kv + h) * 128 + d) * DI_PAGE;
  }
};
static_assert(DI_PAGE == 128, "page lookups shift by 7");

// torch's advanced-indexing rule for a table of n rows (the reference's
// embed_e8[ids] and cos_t[positions]): -n <= x < 0 reads row x + n, any other
// x outside [0, n) raises IndexError. Here such an x reads row 0 (memory
// safety) and ORs `bit` into *err when err is non-null; the host raises from
// the word at its next check.
__device__ __forceinline__ i64 torch_index(i64 x, i64 n, int32_t* err, int bit) {
  if (x < 0) x += n;
  if (x < 0 || x >= n) {
    if (err) atomicOr(err, bit);
    return 0;
  }
  return x;
}

// A wave-uniform value the optimizer cannot trace back to the load it came
// from (no code: readfirstlane of a scalar register is free). Used on kernel
// arguments that are selected between, which it would otherwise turn into a
// load from the selected argument's address.
__device__ __forceinline__ int opaque_i32(int v) { return __builtin_amdgcn_readfirstlane(v); }
template <class T>
__device__ __forceinline__ T* opaque_ptr(T* p) {
  const u64 u = (u64)p;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)u);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(u >> 32));
  return (T*)(((u64)hi << 32) | lo);
}

// A load through a pointer known to be global memory (a pointer rebuilt from
// integers, as opaque_ptr returns, would otherwise be loaded as a flat
// address, which scalar-load waits also cover).
__device__ __forceinline__ i64 ld_global(const int64_t* p) {
  return *(const __attribute__((address_space(1))) int64_t*)p;
}

// Raw buffer views. A descriptor of n bytes at p (stride 0, unswizzled): a
// load at a byte offset at or past n reads 0 and a store there is dropped
// (the buffer unit's range check on the VGPR + instruction offset), and the
// offset is one 32-bit VGPR. Row kernels read and write a row's columns
// through them: no index clamp, no 64-bit address arithmetic and no select
// that zeroes the columns past the row's end. A null p with n = 0 reads 0
// everywhere. p and n must be uniform across the wave (row scalars), n below
// 2^32, offsets multiples of the access size.
typedef __amdgpu_buffer_rsrc_t bufv_t;
__device__ __forceinline__ bufv_t buf_view(const void* p, i64 nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)(uint32_t)nbytes, 0x00020000);
}
__device__ __forceinline__ i64 buf_ld_i64(bufv_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
  return (i64)(((u64)v[1] << 32) | v[0]);
}
__device__ __forceinline__ int32_t buf_ld_i32(bufv_t r, uint32_t off) {
  return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
// 16 bytes; an offset of BUF_OOB (beyond any view, no 32-bit wrap with the
// access size added) reads 0, so a lane masks its load with a select
constexpr uint32_t BUF_OOB = 0x7FFFFFF0u;
template <class V4>
__device__ __forceinline__ V4 buf_ld_16(bufv_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return V4{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
}
__device__ __forceinline__ int32_t buf_ld_i8(bufv_t r, uint32_t off) {
  return (int32_t)(int8_t)__builtin_amdgcn_raw_buffer_load_b8(r, (int)off, 0, 0);
}
__device__ __forceinline__ void buf_st_i8(bufv_t r, uint32_t off, int32_t v) {
  __builtin_amdgcn_raw_buffer_store_b8((uint8_t)v, r, (int)off, 0, 0);
}
__device__ __forceinline__ void buf_st_i32(bufv_t r, uint32_t off, int32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32((uint32_t)v, r, (int)off, 0, 0);
}

// Every kernel starts with this: a reference to its hidden (implicit) launch
// arguments on a path no launch takes (a workgroup id of 2^31 - 2), so that
// its argument segment carries the hidden block. rocprofv3's counter
// collection (ROCm 7.2) reads that block and crashes the profiled process
// (a host SIGSEGV at the launch) on kernels whose segment ends without it.
// Costs one scalar compare; the argument segment grows by 256 bytes.
__device__ __forceinline__ void keep_hidden_args() {
  if (__builtin_amdgcn_workgroup_id_x() == 0x7ffffffeu) {
    const int h = *(const int*)__builtin_amdgcn_implicitarg_ptr();
    asm volatile("" ::"s"(h));
  }
}

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

// floor(sqrt(n)) for a wave-uniform n: the same integer as isqrt (intops.h,
// int_prims.py:31-44; 0 for n <= 0), found by a 64-way search instead of 32
// serial bit steps. Invariant: the root lies in [lo, lo + 64 * sub); lane l
// tests lo + l * sub, and the highest passing lane (the test is monotone)
// becomes the new lo. sub = 2^26, 2^20, 2^14, 2^8, 2^2, 1 covers [0, 2^32),
// which holds every root of a non-negative int64; candidates stay below 2^32,
// so their squares fit in uint64. Every lane of the wave must be active.
__device__ __forceinline__ i64 isqrt_wave(i64 n) {
  if (n <= 0) return 0;
  const u64 un = (u64)n;
  const u64 lane = threadIdx.x & 63;
  u64 lo = 0;
#pragma unroll
  for (int sh = 26; sh >= -4; sh -= 6) {
    const int s = sh < 0 ? 0 : sh;
    const u64 cand = lo + (lane << s);
    const bool ok = cand * cand <= un;
    const u64 mask = __ballot(ok);
    lo += (u64)(63 - clz64(mask)) << s;
  }
  return (i64)lo;
}

// Block-wide reductions (n = the block's thread count, a multiple of 64,
// <= 1024, given by the caller: reading blockDim.x costs a dependent load of
// the launch's hidden arguments), one barrier
// each: every wave's lane 63 publishes its DPP partial, and calls alternate
// between two 16-entry slots of `buf`, so a call never overwrites a slot that
// a slower thread may still be reading (the call in between has a barrier
// that every thread passes only after its reads). Max and wrapping sum are
// associative and commutative: any combine order gives the same integer.
// NWS > 0: the launch fixes the block at NWS waves (n = 64 NWS), so the
// combine of the wave partials is straight-line code over exactly NWS slots
// instead of a loop over up to 16 with masked entries.
template <int NWS = 0>
struct BlockRedT {
  static_assert(NWS >= 0 && NWS <= 16, "waves per block");
  static constexpr bool kBlock = true;
  i64* buf;  // __shared__ i64[32]
  int k;
  int n;     // threads in the block (64 NWS when NWS > 0)

  // the row's threads: the whole block
  __device__ __forceinline__ int tid() const { return (int)threadIdx.x; }
  __device__ __forceinline__ int nt() const { return NWS ? 64 * NWS : n; }
  __device__ __forceinline__ int waves() const { return NWS ? NWS : n >> 6; }

  template <bool MAX>
  __device__ __forceinline__ i64 reduce(i64 v) {
    v = wave_part<MAX>(v);
    i64* slot = buf + (k & 1) * 16;
    ++k;
    if ((threadIdx.x & 63) == 63) slot[threadIdx.x >> 6] = v;
    __syncthreads();
    const int nw = waves();
    i64 r = MAX ? INT64_MIN : 0;
    for (int i = 0; i < nw; i += 4) {
      const i64 a0 = slot[i], a1 = slot[i + 1], a2 = slot[i + 2], a3 = slot[i + 3];
      const i64 id = MAX ? INT64_MIN : 0;
      const i64 b1 = i + 1 < nw ? a1 : id, b2 = i + 2 < nw ? a2 : id, b3 = i + 3 < nw ? a3 : id;
      r = MAX ? imax(imax(r, a0), imax(imax(b1, b2), b3)) : wadd(wadd(r, a0), wadd(wadd(b1, b2), b3));
    }
    return r;
  }
  __device__ __forceinline__ i64 max(i64 v) { return reduce<true>(v); }
  __device__ __forceinline__ i64 sum(i64 v) { return reduce<false>(v); }

  // Block sums of two values (one barrier; blocks of at most 512 threads)
  __device__ __forceinline__ void sum2(i64& a, i64& b) {
    a = wave_part<false>(a);
    b = wave_part<false>(b);
    i64* slot = buf + (k & 1) * 16;
    ++k;
    if ((threadIdx.x & 63) == 63) {
      slot[threadIdx.x >> 6] = a;
      slot[8 + (threadIdx.x >> 6)] = b;
    }
    __syncthreads();
    const int nw = waves();
    i64 ra = 0, rb = 0;
    for (int i = 0; i < nw; ++i) {
      ra = wadd(ra, slot[i]);
      rb = wadd(rb, slot[8 + i]);
    }
    a = ra;
    b = rb;
  }

  // Block maxima of two values (one barrier; blocks of at most 512 threads)
  __device__ __forceinline__ void max2(i64& a, i64& b) {
    a = wave_part<true>(a);
    b = wave_part<true>(b);
    i64* slot = buf + (k & 1) * 16;
    ++k;
    if ((threadIdx.x & 63) == 63) {
      slot[threadIdx.x >> 6] = a;
      slot[8 + (threadIdx.x >> 6)] = b;
    }
    __syncthreads();
    const int nw = waves();
    i64 ra = INT64_MIN, rb = INT64_MIN;
    for (int i = 0; i < nw; ++i) {
      ra = imax(ra, slot[i]);
      rb = imax(rb, slot[8 + i]);
    }
    a = ra;
    b = rb;
  }

  // Block maxima of one or two 32-bit unsigned values (one barrier). A row
  // shift that depends only on the bit length of max |x| reduces bit lengths
  // (bitlen_abs below) here instead of 64-bit magnitudes.
  __device__ __forceinline__ uint32_t max_u32(uint32_t v) {
    uint32_t b = 0;
    max2_u32(v, b);
    return v;
  }
  __device__ __forceinline__ void max2_u32(uint32_t& a, uint32_t& b) {
    a = wave_max_u32(a);
    b = wave_max_u32(b);
    uint32_t* slot = (uint32_t*)(buf + (k & 1) * 16);
    ++k;
    if ((threadIdx.x & 63) == 63) {
      slot[threadIdx.x >> 6] = a;
      slot[16 + (threadIdx.x >> 6)] = b;
    }
    __syncthreads();
    const int nw = waves();
    uint32_t ra = 0, rb = 0;
    for (int i = 0; i < nw; i += 4) {  // 4 reads in flight; entries past nw ignored
      const uint32_t a0 = slot[i], a1 = slot[i + 1], a2 = slot[i + 2], a3 = slot[i + 3];
      const uint32_t b0 = slot[16 + i], b1 = slot[17 + i], b2 = slot[18 + i], b3 = slot[19 + i];
      ra = ::max(ra, ::max(::max(a0, i + 1 < nw ? a1 : 0u),
                           ::max(i + 2 < nw ? a2 : 0u, i + 3 < nw ? a3 : 0u)));
      rb = ::max(rb, ::max(::max(b0, i + 1 < nw ? b1 : 0u),
                           ::max(i + 2 < nw ? b2 : 0u, i + 3 < nw ? b3 : 0u)));
    }
    a = ra;
    b = rb;
  }

  // DPP maximum of a 32-bit unsigned value, result in lane 63 (no broadcast)
  static __device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = ::max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xF, 0xF, false));
    v = ::max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false));
    v = ::max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x141, 0xF, 0xF, false));
    v = ::max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x140, 0xF, 0xF, false));
    v = ::max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xA, 0xF, false));
    v = ::max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xC, 0xF, false));
    return v;
  }

  // DPP reduction leaving the wave's result in lane 63 (no broadcast)
  template <bool MAX>
  static __device__ __forceinline__ i64 wave_part(i64 v) {
    if (MAX) {
      v = imax(v, dpp64<0xB1, 0xF>(v, v));
      v = imax(v, dpp64<0x4E, 0xF>(v, v));
      v = imax(v, dpp64<0x141, 0xF>(v, v));
      v = imax(v, dpp64<0x140, 0xF>(v, v));
      v = imax(v, dpp64<0x142, 0xA>(v, v));
      v = imax(v, dpp64<0x143, 0xC>(v, v));
    } else {
      v = wadd(v, dpp64<0xB1, 0xF>(v, 0));
      v = wadd(v, dpp64<0x4E, 0xF>(v, 0));
      v = wadd(v, dpp64<0x141, 0xF>(v, 0));
      v = wadd(v, dpp64<0x140, 0xF>(v, 0));
      v = wadd(v, dpp64<0x142, 0xA>(v, 0));
      v = wadd(v, dpp64<0x143, 0xC>(v, 0));
    }
    return v;
  }
};

using BlockRed = BlockRedT<0>;

// Reductions over one wave's 64 lanes (DPP, no LDS, no barrier): a row
// handled by a single wave, several rows per block side by side. Same
// integers as BlockRed (max and wrapping sum are order-independent).
struct WaveRed {
  static constexpr bool kBlock = false;
  __device__ __forceinline__ int tid() const { return (int)(threadIdx.x & 63); }
  __device__ __forceinline__ int nt() const { return 64; }
  __device__ __forceinline__ i64 max(i64 v) { return wave_max(v); }
  __device__ __forceinline__ i64 sum(i64 v) { return wave_sum(v); }
  __device__ __forceinline__ uint32_t max_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_readlane((int)BlockRed::wave_max_u32(v), 63);
  }
  __device__ __forceinline__ void max2_u32(uint32_t& a, uint32_t& b) {
    a = max_u32(a);
    b = max_u32(b);
  }
};

// Bit length of |x| (0 for x == 0): ilog2(max(max_j |x_j|, 1)) is
// max(max_j bitlen_abs(x_j) - 1, 0). |INT64_MIN| wraps to a negative int64,
// as torch's abs does, and never wins a maximum of magnitudes (every amax
// here is clamped to >= 1 first), so it counts as 0 too.
__device__ __forceinline__ uint32_t bitlen_abs(i64 x) {
  const i64 a = wabs(x);
  return a > 0 ? 64u - (uint32_t)clz64((u64)a) : 0u;
}

// ilog2(max(m, 1)) from the bit length of m >= 0
__device__ __forceinline__ i64 ilog2_from_bitlen(uint32_t len) { return len > 1 ? len - 1 : 0; }

__device__ __forceinline__ i64 to_i32(i64 v) { return (i64)(int32_t)(uint32_t)(u64)v; }

// Direct-to-LDS loads (global_load_lds_dwordx4: lane l's 16 bytes land at the
// wave-uniform LDS base + 16 l) take these pointer types.
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(1))) void* gbl_ptr_t;

// s_waitcnt with vmcnt = n (n < 64) and no wait on the other counters
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

}  // namespace di
