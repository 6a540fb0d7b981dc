// Skinny GEMM tile (decode GEMV, M <= 64 rows) of k_gemv_nt.
//
// C[ks][M][N] = A[M][Kchunk] . B[N][Kchunk]^T on v_mfma_i32_16x16x64_i8. A
// wave computes one 16-column group over a K range. Lane l supplies column
// (l % 16) and U consecutive 16-byte K slices starting at 16*U*(l / 16): a
// wave-load reads 16U*4 contiguous bytes of each of its 16 weight rows (whole
// 128-byte lines for U >= 2). The K order inside an MFMA does not matter as
// long as A and B use the same one, so A is loaded with the identical mapping.
// The 16x16 int32 result lands as C[4*(l/16) + r][l % 16] in element r of
// lane l.
//
// Latency bounds these launches (a decode layer's matrices are 1-6 MB), so
// each wave issues all loads of NB iterations before the first MFMA. KW waves
// of a block split the K range of one column group and reduce their int32
// accumulators through LDS.
#pragma once

#include "common.h"

typedef int v4i __attribute__((ext_vector_type(4)));

namespace di {

__device__ __forceinline__ v4i mfma16(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v4i zero4() { return v4i{0, 0, 0, 0}; }

struct GemvArgs {
  const int8_t* A;  // [M][K]
  const int8_t* B;  // [N][K]
  int32_t* C;       // [ksplit][M][N], split_stride elements apart
  int M, N, K;
  int kchunk;
  i64 split_stride;
};

template <int MB, int KW>
struct GemvLds {
  int32_t red[KW > 1 ? (KW - 1) * (4 / KW) : 1][MB * 4][64];
};

// The default epilogue of gemv_block: the int32 product (or K-split
// partial) to C.
struct GemvStore {
  __device__ __forceinline__ void operator()(const GemvArgs& g, int by, int row, int col,
                                             int32_t v) const {
    g.C[by * g.split_stride + (i64)row * g.N + col] = v;
  }
};

// One 256-thread GEMV block: column group(s) `bx`, K range `by`; every
// in-range (row, col) result goes to epi(g, by, row, col, value).
template <int MB, int KW, int NB, class Epi = GemvStore>
__device__ __forceinline__ void gemv_block(const GemvArgs& g, int bx, int by, GemvLds<MB, KW>& L,
                                           const Epi& epi = Epi()) {
  constexpr int U = 4;           // 16-byte slices per lane per iteration
  constexpr int CG = 4 / KW;     // column groups per block
  constexpr int KSTEP = 64 * U;  // K covered by one wave-iteration
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int cg = wave % CG, kw = wave / CG;
  const int r16 = lane & 15, grp = lane >> 4;
  const int col = (bx * CG + cg) * 16 + r16;
  const bool colok = col < g.N;
  const int kbeg = by * g.kchunk;
  const int kend = min(g.K, kbeg + g.kchunk);
  const int8_t* brow = g.B + (i64)(colok ? col : 0) * g.K;
  const int M = g.M, K = g.K;
  v4i acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = zero4();
  const int kfirst = kbeg + kw * KSTEP;
  v4i b[NB][U];
  auto load_b = [&](int k0) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kk = k0 + nb * KSTEP * KW + grp * 16 * U + u * 16;
        b[nb][u] = (colok && kk < kend) ? *(const v4i*)(brow + kk) : zero4();
      }
  };
  for (int k0 = kfirst; k0 < kend; k0 += KSTEP * KW * NB) {
    load_b(k0);
    v4i a[NB][U][MB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kk = k0 + nb * KSTEP * KW + grp * 16 * U + u * 16;
        const bool kok = kk < kend;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const int row = mb * 16 + r16;
          a[nb][u][mb] = (row < M && kok) ? *(const v4i*)(g.A + (i64)row * K + kk) : zero4();
        }
      }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[mb] = mfma16(a[nb][u][mb], b[nb][u], acc[mb]);
  }
  if (KW > 1) {
    if (kw > 0) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) L.red[(kw - 1) * CG + cg][mb * 4 + r][lane] = acc[mb][r];
    }
    __syncthreads();
    if (kw > 0) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int32_t s = acc[mb][r];
#pragma unroll
        for (int w = 0; w < KW - 1; ++w) s += L.red[w * CG + cg][mb * 4 + r][lane];
        acc[mb][r] = s;
      }
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = mb * 16 + grp * 4 + r;
      if (row < M && colok) epi(g, by, row, col, acc[mb][r]);
    }
}

// Up to four byte ranges that the kernels after this launch read (their
// per-column scale vectors): each thread of the first K split touches one
// 128-byte line of them, so they are fetched into the memory-side cache while
// this launch streams its weights and the next launch finds them there.
// A performance hint only: the loaded words are discarded (stored to `sink`
// only when it is non-null, which keeps the loads), results do not change.
struct Prefetch {
  const int8_t* p[4];
  i64 n[4];  // bytes; 0 = unused
  int32_t* sink;
};

// The touched word, held until the end of the kernel (prefetch_keep): a
// consumer right after the load, or a register reused while the load is in
// flight, would make the kernel wait for it before its own loads.
struct PrefetchHold {
  int32_t v;
  bool hit;
};

__device__ __forceinline__ PrefetchHold prefetch_issue(const Prefetch& pf, i64 t) {
  const int8_t* q = nullptr;  // thread t's line: the ranges laid end to end
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const i64 lines = (pf.n[i] + 127) >> 7;
    if (q == nullptr && t >= 0 && t < lines) q = pf.p[i] + (t << 7);  // 128 t < n, n % 4 == 0
    t -= lines;
  }
  PrefetchHold h;
  h.hit = q != nullptr;
  h.v = 0;
  if (h.hit) h.v = *(const int32_t*)q;
  return h;
}

__device__ __forceinline__ void prefetch_keep(const Prefetch& pf, const PrefetchHold& h) {
  if (h.hit && pf.sink) *pf.sink = h.v;
}

// K range per split (a multiple of 64)
__host__ __device__ inline int gemv_kchunk(int K, int ksplit) {
  int kchunk = (K + ksplit - 1) / ksplit;
  return (kchunk + 63) / 64 * 64;
}

// The weights of the skinny GEMM that runs next, pulled into the L2 caches
// by extra blocks of the launch before it (a row kernel, which keeps only a
// few CUs busy). The blocks of a launch are dispatched to the 8 XCDs in turn
// (block b to XCD b % 8), each XCD has its own L2, and clean lines stay in
// an L2 across launches; so a warming block on XCD x touches the weight
// slices of the GEMM blocks with ids = x (mod 8) — GEMM block (bx, by), id
// bx + gx by, reads rows 16 bx .. 16 bx + 15 over K range [by kchunk, ...) —
// and those blocks then read their weights from their own L2 instead of HBM
// (a 4 MB product measured 2.8 against 3.9 us per launch). A performance
// hint only: a warming block writes nothing but its own LDS.
struct L2Warm {
  const int8_t* W;  // [N][K]; null: no warming blocks
  int N, K, kchunk;
  int gx, nblk;     // the GEMM's grid: gx column groups x (nblk / gx) K ranges
  int first;        // this launch's first warming block
  int nwarm;        // warming blocks, a multiple of 8
};

constexpr int L2WARM_BLOCKS = 32;

// Host side: the warming blocks for the next igemv(A, W, ., M, N, K, ksplit),
// block ids first .. first + L2WARM_BLOCKS - 1 of a launch (W null: none).
inline L2Warm make_l2warm(const int8_t* W, int N, int K, int ksplit, int first) {
  L2Warm w{};
  if (W == nullptr || N <= 0 || K <= 0 || ksplit < 1) return w;
  w.W = W;
  w.N = N;
  w.K = K;
  w.kchunk = gemv_kchunk(K, ksplit);
  w.gx = (N + 15) / 16;
  w.nblk = w.gx * ksplit;
  w.first = first;
  w.nwarm = L2WARM_BLOCKS;
  return w;
}

// Block j (>= w.first) of nt threads: one 4-byte direct-to-LDS load per
// 128-byte line of its GEMM blocks' slices (as fast for the GEMM as touching
// every 64 bytes; no registers to wait on: the wave ends when they land).
// `sink`: 256 bytes of this block's LDS, overwritten.
constexpr int L2WARM_SLEEP = 0;  // s_sleep units (64 clocks) before the loads

__device__ __forceinline__ void l2_warm(const L2Warm& w, int j, int nt, void* sink) {
  if (L2WARM_SLEEP > 0) __builtin_amdgcn_s_sleep(L2WARM_SLEEP);
  const int t = (j - w.first) >> 3;  // rank among the warming blocks on this XCD
  const int step = w.nwarm;          // 8 x (warming blocks per XCD)
  const int kl = (w.kchunk + 127) >> 7;  // lines per row of a K range
  const int per = 16 * kl;
  for (int L = (j & 7) + 8 * t; L < w.nblk; L += step) {
    const int bx = L % w.gx, by = L / w.gx;
    for (int u = (int)threadIdx.x; u < per; u += nt) {
      const int row = 16 * bx + u / kl;
      const int k = by * w.kchunk + (u % kl) * 128;
      if (row < w.N && k < w.K)
        __builtin_amdgcn_global_load_lds((gbl_ptr_t)(w.W + (i64)row * w.K + k), (lds_ptr_t)sink,
                                         4, 0, 0);
    }
  }
}

}  // namespace di
