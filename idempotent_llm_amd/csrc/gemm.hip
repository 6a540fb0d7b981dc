// Exact int8 x int8 -> int32 GEMMs on CDNA4 i8 MFMA (gfx950), plus the
// integer arg-max of greedy decoding.
//
// Layout: C[M,N] = A[M,K] . B[N,K]^T with both operands K-contiguous ("NT").
// The model keeps every weight matrix in this [out, in] layout (a load-time
// integer permutation of the artifact's [in, out] ``w8t``), so a lane's
// 16-byte load is directly one MFMA operand fragment.
//
// Exactness: every partial sum is an int32 integer sum of int8 products;
// |sum| <= K * 128 * 128 < 2^31 for K <= 131071, so no accumulation order
// can change the result (the reference's backends.py:1-11 argument).
//
// MFMA fragment convention (v_mfma_i32_16x16x64_i8): lane l supplies row (A)
// or column (B) l % 16 and a 16-byte K slice chosen by l / 16; the product
// sums over all 64 K values, so A and B only have to agree on which K value
// sits in which slot. The 16x16 int32 result lands as C[4*(l/16) + r][l % 16]
// in element r of lane l.
//
// Kernels:
//   k_gemm_nt2  — M > 64, K % 128 == 0 (prefill): 32x32x32 MFMA, direct-to-LDS
//                 operand ring with swizzled rows, XCD-blocked tile order.
//   k_gemm_nt   — other M > 64 shapes: 128x128x64 block tiles, 4 waves of
//                 64x64, LDS double buffer.
//   k_gemv_nt   — M <= 64 (decode): a wave owns 16 output columns and a
//                 K range; weight fragments stream straight from HBM into
//                 MFMA operands, every load of a batch issued before the
//                 first MFMA; an optional K split (detllm_igemv_plan) writes
//                 int32 partials that the consuming row kernel sums in a
//                 fixed order (exact integer addition).
//   k_gemv_dec  — the same tile, straight-line, for M <= 16 and K ranges of
//                 at most 1024 (every decode shape of the model).
//   k_argmax_*  — greedy_pick (model.py:482-490): argmax of logits * head_m
//                 in int64 with the lowest-id tie-break.

#include <mutex>

#include "common.h"
#include "gemv.h"

using namespace di;

namespace {

constexpr int TBM = 128, TBN = 128, TBK = 64, TPAD = 16;

__global__ __launch_bounds__(256) void k_gemm_nt(const int8_t* __restrict__ A,
                                                 const int8_t* __restrict__ B,
                                                 int32_t* __restrict__ C, int M, int N, int K,
                                                 i64 sA, i64 sB, i64 sC, int tiles_n) {
  keep_hidden_args();
  __shared__ __attribute__((aligned(16))) int8_t As[2][TBM][TBK + TPAD];
  __shared__ __attribute__((aligned(16))) int8_t Bs[2][TBN][TBK + TPAD];
  const int bz = blockIdx.z;
  A += bz * sA;
  B += bz * sB;
  C += bz * sC;
  const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int r16 = lane & 15, kq = (lane >> 4) * 16;

  v4i ra[2], rb[2];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + i * 256;
      const int row = c >> 2, kc = (c & 3) * 16;
      const int gk = k0 + kc;
      const int ga = tm * TBM + row, gb = tn * TBN + row;
      ra[i] = (ga < M && gk < K) ? *(const v4i*)(A + (i64)ga * K + gk) : zero4();
      rb[i] = (gb < N && gk < K) ? *(const v4i*)(B + (i64)gb * K + gk) : zero4();
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + i * 256;
      const int row = c >> 2, kc = (c & 3) * 16;
      *(v4i*)&As[buf][row][kc] = ra[i];
      *(v4i*)&Bs[buf][row][kc] = rb[i];
    }
  };

  v4i acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = zero4();

  const int nk = (K + TBK - 1) / TBK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * TBK);
    v4i af[4], bf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) af[i] = *(const v4i*)&As[buf][wm * 64 + i * 16 + r16][kq];
#pragma unroll
    for (int j = 0; j < 4; ++j) bf[j] = *(const v4i*)&Bs[buf][wn * 64 + j * 16 + r16][kq];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = mfma16(af[i], bf[j], acc[i][j]);
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = tm * TBM + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
        const int col = tn * TBN + wn * 64 + j * 16 + r16;
        if (row < M && col < N) C[(i64)row * N + col] = acc[i][j][r];
      }
}

// ---------------------------------------------------------------------------
// k_gemm_nt2 — the prefill GEMM (M > 64, K % 128 == 0), on
// v_mfma_i32_32x32x32_i8: both i8 forms run at the same rate on gfx950
// (measured, about 4.4 POP/s), but a 32x32x32 tile needs half the operand
// bytes per multiply-add of a 16x16x64 one, so half the LDS reads.
//
// Operands stream into LDS with direct-to-LDS loads (global_load_lds_dwordx4:
// lane l's 16 bytes land at base + 16 l) through an S-stage ring of 128-byte
// K slices. A load instruction covers 8 operand rows x 128 bytes, i.e. 8 whole
// cache lines. In LDS each slice is row-major (128 bytes per row) with the
// 16-byte chunks of row r permuted, physical chunk = logical chunk ^
// ((r / 2) % 8), so the MFMA operand reads (32 rows, one chunk each) hit
// distinct banks; the loader lanes fetch the logical chunk that belongs at
// their physical position. Rows past M / N are clamped to the last row (valid
// memory; their results are never stored). Waits are explicit: each wave
// waits for its own loads of the slice it is about to use (vmcnt), then one
// barrier makes every wave's part visible and frees the slot that the next
// issue overwrites. Tiles are ordered so that each XCD (blocks are dispatched
// round-robin over the 8 XCDs) owns one contiguous block of the tile grid,
// keeping its share of A and B in its own L2.
// ---------------------------------------------------------------------------
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int g2_swz(int row) { return (row >> 1) & 7; }

// tile order: XCD x (= blockIdx % 8) owns block (x / 4, x % 4) of a 2 x 4
// split of the tile grid when the grid divides evenly, else row-major order
__device__ __forceinline__ void g2_tile(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  if ((tiles_m & 1) != 0 || (tiles_n & 3) != 0) {
    tm = bid / tiles_n;
    tn = bid - tm * tiles_n;
    return;
  }
  const int xcd = bid & 7, j = bid >> 3;
  const int bm = tiles_m >> 1, bn = tiles_n >> 2;
  tm = (xcd >> 2) * bm + j / bn;
  tn = (xcd & 3) * bn + j % bn;
}

constexpr int G2_BK = 128;

template <int BM, int BN, int S, int WGM, int WGN, int MINB>
__global__ __launch_bounds__(64 * WGM * WGN, MINB) void k_gemm_nt2(const int8_t* __restrict__ A,
                                                        const int8_t* __restrict__ B,
                                                        int32_t* __restrict__ C, int M, int N,
                                                        int K, i64 sA, i64 sB, i64 sC,
                                                        int tiles_m, int tiles_n) {
  keep_hidden_args();
  constexpr int ROWS = BM + BN;       // 128-byte rows per slice: A rows, then B rows
  constexpr int NW = WGM * WGN;       // waves, WGM x WGN over the tile
  constexpr int NI = ROWS / 8;        // load instructions per slice (8 rows each)
  static_assert(NI % NW == 0, "loads per wave");
  constexpr int LPW = NI / NW;
  constexpr int STAGE = ROWS * G2_BK;
  constexpr int WA = BM / 32 / WGM, WB = BN / 32 / WGN;  // 32x32 blocks per wave
  static_assert(WA >= 1 && WB >= 1, "wave tile");
  __shared__ __attribute__((aligned(1024))) int8_t lds[S * STAGE];

  const int bz = blockIdx.z;
  A += bz * sA;
  B += bz * sB;
  C += bz * sC;
  int tm, tn;
  g2_tile(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave / WGN, wn = wave % WGN;

  // this wave's loads: instruction i covers slice rows 8i..8i+7; lane l takes
  // row 8i + l/8 at physical chunk l%8, i.e. logical chunk (l%8) ^ swz(row)
  const int8_t* src[LPW];
  int dst_off[LPW];
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    const int ins = wave * LPW + j;
    const int srow = ins * 8 + (lane >> 3);
    const int lch = (lane & 7) ^ g2_swz(srow);
    if (srow < BM) {
      const int row = min(tm * BM + srow, M - 1);
      src[j] = A + (i64)row * K + lch * 16;
    } else {
      const int col = min(tn * BN + (srow - BM), N - 1);
      src[j] = B + (i64)col * K + lch * 16;
    }
    dst_off[j] = __builtin_amdgcn_readfirstlane(ins * 1024);
  }
  auto issue = [&](int kt) {
    int8_t* base = lds + (kt % S) * STAGE;
#pragma unroll
    for (int j = 0; j < LPW; ++j)
      __builtin_amdgcn_global_load_lds((gbl_ptr_t)(src[j] + (i64)kt * G2_BK),
                                       (lds_ptr_t)(base + dst_off[j]), 16, 0, 0);
  };

  // MFMA operands: lane l reads row l%32 of a 32-row block, logical chunk
  // 2s + l/32 of sub-slice s (32 K values); A and B use the same K order
  const int r32 = lane & 31, half = lane >> 5;
  v16i acc[WA][WB];
#pragma unroll
  for (int i = 0; i < WA; ++i)
#pragma unroll
    for (int j = 0; j < WB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  const int nk = K / G2_BK;
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < nk) issue(s);
  for (int kt = 0; kt < nk; ++kt) {
    // slices issued after kt so far: min(S - 2, nk - 1 - kt)
    const int after = min(S - 2, nk - 1 - kt);
    static_assert(S <= 5 && 3 * LPW < 64, "vmcnt range");
    if (after >= 3) wait_vmcnt<3 * LPW>();
    else if (after == 2) wait_vmcnt<2 * LPW>();
    else if (after == 1) wait_vmcnt<LPW>();
    else wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    if (kt + S - 1 < nk) issue(kt + S - 1);
    const int8_t* base = lds + (kt % S) * STAGE;
#pragma unroll
    for (int s = 0; s < G2_BK / 32; ++s) {
      v4i af[WA], bf[WB];
#pragma unroll
      for (int i = 0; i < WA; ++i) {
        const int r = (wm * WA + i) * 32 + r32;
        af[i] = *(const v4i*)(base + r * G2_BK + ((2 * s + half) ^ g2_swz(r)) * 16);
      }
#pragma unroll
      for (int j = 0; j < WB; ++j) {
        const int r = BM + (wn * WB + j) * 32 + r32;
        bf[j] = *(const v4i*)(base + r * G2_BK + ((2 * s + half) ^ g2_swz(r)) * 16);
      }
#pragma unroll
      for (int i = 0; i < WA; ++i)
#pragma unroll
        for (int j = 0; j < WB; ++j) acc[i][j] = mfma32(af[i], bf[j], acc[i][j]);
    }
  }
  // 32x32 result block: lane l, element r -> row 8(r/4) + 4(l/32) + r%4, col l%32
#pragma unroll
  for (int i = 0; i < WA; ++i)
#pragma unroll
    for (int j = 0; j < WB; ++j) {
      const int col = tn * BN + (wn * WB + j) * 32 + r32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = tm * BM + (wm * WA + i) * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        // streaming stores: the product is written once and read by the
        // next launch (measured 5-6 % faster at the M = 2048 shapes)
        if (row < M && col < N) __builtin_nontemporal_store(acc[i][j][r], &C[(i64)row * N + col]);
      }
    }
}

// Skinny GEMM (decode GEMV), M <= 64 rows: the tile of gemv.h, one
// 256-thread block per (column group, K range).
template <int MB, int KW, int NB>
__global__ __launch_bounds__(256) void k_gemv_nt(GemvArgs g, Prefetch pf) {
  keep_hidden_args();
  __shared__ GemvLds<MB, KW> lds;
  const PrefetchHold ph =
      prefetch_issue(pf, blockIdx.y == 0 ? (i64)blockIdx.x * 256 + threadIdx.x : (i64)-1);
  gemv_block<MB, KW, NB>(g, blockIdx.x, blockIdx.y, lds);
  prefetch_keep(pf, ph);
}

// The decode form of the skinny GEMM: M <= 16 rows and a K range of at most
// 1024 per block, so each of the four waves makes one 256-wide K step of the
// block's 16-column group and the kernel is straight-line: the weight and
// operand loads issue as soon as the kernel arguments arrive (the prefetch
// hint after them: before them it delays every weight load), then four
// MFMAs, the cross-wave sum through LDS and the store. Same tile and K order
// as gemv_block; measured 0.3 us per launch faster than k_gemv_nt at every
// decode shape.
constexpr int DEC_KMAX = 4 * 256;

__global__ __launch_bounds__(256) void k_gemv_dec(GemvArgs g, Prefetch pf) {
  __shared__ int32_t red[3][4][64];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r16 = lane & 15, grp = lane >> 4;
  const int col = blockIdx.x * 16 + r16;
  const bool colok = col < g.N;
  const int kbeg = blockIdx.y * g.kchunk;
  const int kend = min(g.K, kbeg + g.kchunk);
  const int k0 = kbeg + wave * 256 + grp * 64;
  // buffer views of the block's 16 weight rows (those below N) and of the M
  // operand rows: a lane's row past either end reads 0 by the range check,
  // and a slice past the block's K range gets an offset beyond both views,
  // so every load is unconditional (no branch around it) and addressed by
  // one 32-bit offset (16 K < 2^21)
  const int ncols = min(16, g.N - (int)blockIdx.x * 16);
  const bufv_t bv = buf_view(g.B + (i64)blockIdx.x * 16 * g.K, (i64)ncols * g.K);
  const bufv_t av = buf_view(g.A, (i64)g.M * g.K);
  const uint32_t rowoff = (uint32_t)(r16 * g.K);
  v4i b[4], a[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int kk = k0 + u * 16;
    b[u] = buf_ld_16<v4i>(bv, kk < kend ? rowoff + (uint32_t)kk : BUF_OOB);
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int kk = k0 + u * 16;
    a[u] = buf_ld_16<v4i>(av, kk < kend ? rowoff + (uint32_t)kk : BUF_OOB);
  }
  const PrefetchHold ph =
      prefetch_issue(pf, blockIdx.y == 0 ? (i64)blockIdx.x * 256 + tid : (i64)-1);
  v4i acc = zero4();
#pragma unroll
  for (int u = 0; u < 4; ++u) acc = mfma16(a[u], b[u], acc);
  if (wave > 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave - 1][r][lane] = acc[r];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = grp * 4 + r;
      const int32_t s = acc[r] + red[0][r][lane] + red[1][r][lane] + red[2][r][lane];
      if (row < g.M && colok) g.C[blockIdx.y * g.split_stride + (i64)row * g.N + col] = s;
    }
  }
  prefetch_keep(pf, ph);
  keep_hidden_args();
}

// requant_i8_static of a skinny GEMM's product (M <= 64 rows), applied in
// the GEMV's epilogue so the int32 product never leaves registers: config
// c0's int_gemm + requant (dyadic.py:142-163, canonical form (P, 1, 0, m, 20,
// 1, 0)). A block owns 16 columns; its eight waves split K (128 bytes each
// per 1024-byte step: measured 5.1 us per c0 call against 5.8 with four
// waves and 5.4 with sixteen), all eight write their partial products to LDS
// and wave w then sums and requantises two of the four rows per lane of row
// group w % 4.
//
// Per row, computed once per block into LDS: row_m (rm), the shift split into
// up / down, the divisor den = s_m << down (wrapping; 1 when it is 0, where
// the reference's division raises) and its fp64 estimate constants. Per
// element y = clamp_i8(rhad((P col_m rm) << up, den)):
//  * fp64 path, when 0 < den < 2^49, |col_m| < 2^22, |rm| < 2^31 and up <
//    32: n = fl(fl(P col_m) * rm 2^up). P col_m is exact (|P| < 2^31), and
//    the second product is exact whenever the true |n| is below 2^49 (an
//    integer below 2^53), while a true |n| >= 2^49 rounds to at least 2^49;
//    so the test |n| < 2^49 on the computed value is exact, and then no step
//    of the int64 chain wraps (|rm| >= 1, or rm = 0 and n = 0) and
//    rhad_est_i8 applies (2 |n| + den < 2^51);
//  * otherwise the int64 chain and the integer division (torch's floor
//    division also for a divisor that wrapped negative).
// Same integers as k_static_cols after the GEMV.
#ifndef GEMV_STATIC_NW
#define GEMV_STATIC_NW 8
#endif

struct StaticRows {
  i64 rm[64], up[64], den[64];
  double rmu[64], dr[64], dk[64];
  int fast[64];
};

template <int NW>
__global__ __launch_bounds__(64 * NW) void k_gemv_static(GemvArgs g, const int64_t* row_m,
                                                         const int64_t* row_k,
                                                         const int64_t* __restrict__ col_m,
                                                         i64 col_k, i64 s_m, i64 s_k,
                                                         int8_t* __restrict__ y8) {
  keep_hidden_args();
  constexpr int U = 16 / NW;            // 16-byte slices per lane per 1024-byte K step
  __shared__ int32_t red[NW][4][4][64];  // [wave][row group][r][lane]
  __shared__ StaticRows sr;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r16 = lane & 15, grp = lane >> 4;
  const int col = blockIdx.x * 16 + r16;
  const bool colok = col < g.N;
  const int M = g.M, K = g.K;
  const i64 cm = col_m[colok ? col : 0];
  // buffer views of the block's weight rows below N and of the M operand
  // rows (rows past either end read 0; a slice past K gets an offset beyond
  // both views): unconditional loads on 32-bit offsets (64 K < 2^23)
  const bufv_t bv = buf_view(g.B + (i64)blockIdx.x * 16 * K, (i64)min(16, g.N - (int)blockIdx.x * 16) * K);
  const bufv_t av = buf_view(g.A, (i64)M * K);
  v4i acc[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) acc[mb] = zero4();
  // wave w covers bytes [w 64 U, (w + 1) 64 U) of every 1024-byte K step;
  // lane (r16, grp) takes 16 U of them at grp 16 U (A and B in the same order)
  v4i b[U], a[U][4];
  auto load = [&](int k0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = k0 + grp * 16 * U + u * 16;
      b[u] = buf_ld_16<v4i>(bv, kk < K ? (uint32_t)(r16 * K + kk) : BUF_OOB);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = k0 + grp * 16 * U + u * 16;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const int row = mb * 16 + r16;
        a[u][mb] = buf_ld_16<v4i>(av, kk < K ? (uint32_t)(row * K + kk) : BUF_OOB);
      }
    }
  };
  auto mma = [&]() {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) acc[mb] = mfma16(a[u][mb], b[u], acc[mb]);
  };
  load(wave * 64 * U);
  // the per-row constants while the first K step's loads are in flight
  static_assert(NW == 4 || NW == 8 || NW == 16, "waves per block");
  if (tid < M) {
    const i64 rm = row_m ? row_m[tid] : 1;
    const i64 rk = row_k ? row_k[tid] : 0;
    const i64 shift = wsub(wadd(rk, col_k), s_k);
    const i64 down = imax(shift, 0), up = imax(wneg(shift), 0);
    i64 den = shl(s_m, down);
    if (den == 0) den = 1;  // the reference's division raises there
    const bool dfast = den > 0 && den < ((i64)1 << 49);
    const DivEst D = make_divest(dfast ? den : 1, 1.0);
    sr.rm[tid] = rm;
    sr.up[tid] = up;
    sr.den[tid] = den;
    sr.rmu[tid] = ldexp((double)rm, up < 32 ? (int)up : 0);
    sr.dr[tid] = D.r;
    sr.dk[tid] = D.k;
    sr.fast[tid] = dfast && rm > -((i64)1 << 31) && rm < ((i64)1 << 31) && up < 32;
  }
  mma();
  for (int k0 = wave * 64 * U + 1024; k0 < K; k0 += 1024) {
    load(k0);
    mma();
  }
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][mb][r][lane] = acc[mb][r];
  __syncthreads();
  const bool cfast = cm > -((i64)1 << 22) && cm < ((i64)1 << 22);
  const double cmd = (double)cm;
  // wave w finalises row group w % 4, elements r of its lanes' four rows
  // with r % (NW / 4) == w / 4
  const int mbf = wave & 3;
#pragma unroll
  for (int rr = 0; rr < 4 / (NW / 4); ++rr) {
    const int r = rr * (NW / 4) + (wave >> 2);
    const int row = mbf * 16 + grp * 4 + r;
    if (row >= M || !colok) continue;
    int32_t v = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += red[w][mbf][r][lane];
    int y;
    const double nd = (double)v * cmd * sr.rmu[row];
    constexpr double lim = 0x1p49;
    if (DI_LIKELY(cfast && sr.fast[row] && nd > -lim && nd < lim)) {
      const double e = fmin(fma(fabs(nd), sr.dr[row], sr.dk[row]), 255.0);
      const int q = (int)(uint32_t)e;
      const int sq = nd < 0 ? -q : q;
      y = sq < -128 ? -128 : (sq > 127 ? 127 : sq);
    } else {
      const i64 n = shl(wmul(wmul((i64)v, cm), sr.rm[row]), sr.up[row]);
      y = (int)clamp_i8(rhad(n, sr.den[row]));
    }
    y8[(i64)row * g.N + col] = (int8_t)y;
  }
}

// Skinny GEMM over many columns (the LM head) for M <= 16 rows: the A rows
// are staged in LDS once per block, and each wave walks its own 16-column
// groups over the whole K range (grid-stride), with all of a group's weight
// loads (up to 1024 bytes of K per lane) in flight before its MFMAs; no
// cross-wave reduction. At the LM-head shape (N = 151936, K = 1024) it
// streams 5.9 TB/s at M = 8 against 4.8 TB/s for the K-split tile.
constexpr int GS_BLOCKS = 512;
constexpr int GS_KMAX = 4096;  // A in LDS: 16 rows x K bytes

__global__ __launch_bounds__(256) void k_gemv_stream(const int8_t* __restrict__ A,
                                                     const int8_t* __restrict__ B,
                                                     int32_t* __restrict__ C, int M, int N,
                                                     int K, Prefetch pf) {
  keep_hidden_args();
  extern __shared__ __attribute__((aligned(16))) int8_t sa[];  // [16][K]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const PrefetchHold ph = prefetch_issue(pf, (i64)blockIdx.x * 256 + tid);
  for (int i = tid * 16; i < 16 * K; i += 256 * 16)
    *(v4i*)(sa + i) = i / K < M ? *(const v4i*)(A + i) : zero4();
  __syncthreads();
  const int r16 = lane & 15, grp = lane >> 4;
  const int groups = (N + 15) / 16;
  for (int gidx = blockIdx.x * 4 + wave; gidx < groups; gidx += gridDim.x * 4) {
    const int col = gidx * 16 + r16;
    const int8_t* brow = B + (i64)(col < N ? col : N - 1) * K;
    v4i acc = zero4();
    for (int k0 = 0; k0 < K; k0 += 1024) {
      // lane (r16, grp) takes bytes grp * 16 .. + 15 of every 64-byte K slice
      // of column r16 and of A row r16 (the same K order on both operands)
      v4i b[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int kk = k0 + u * 64 + grp * 16;
        b[u] = kk < K ? *(const v4i*)(brow + kk) : zero4();
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int kk = k0 + u * 64 + grp * 16;
        const v4i a = kk < K ? *(const v4i*)(sa + r16 * K + kk) : zero4();
        acc = mfma16(a, b[u], acc);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = grp * 4 + r;
      if (row < M && col < N) C[(i64)row * N + col] = acc[r];
    }
  }
  prefetch_keep(pf, ph);
}

__global__ void k_transpose_i8(const int8_t* __restrict__ src, int8_t* __restrict__ dst, int R,
                               int Cc, i64 sS, i64 sD) {
  keep_hidden_args();
  __shared__ int8_t tile[64][65];
  src += blockIdx.z * sS;
  dst += blockIdx.z * sD;
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  for (int i = threadIdx.x; i < 64 * 64; i += blockDim.x) {
    const int rr = i >> 6, cc = i & 63;
    if (r0 + rr < R && c0 + cc < Cc) tile[rr][cc] = src[(i64)(r0 + rr) * Cc + c0 + cc];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += blockDim.x) {
    const int cc = i >> 6, rr = i & 63;
    if (r0 + rr < R && c0 + cc < Cc) dst[(i64)(c0 + cc) * R + r0 + rr] = tile[rr][cc];
  }
}

struct Best {
  i64 v;
  i64 i;
};

__device__ __forceinline__ Best better(Best a, Best b) {
  return (a.v > b.v || (a.v == b.v && a.i < b.i)) ? a : b;
}

__device__ __forceinline__ Best block_best(Best x, i64* sv, i64* si) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    Best y{shfl_xor64(x.v, o), shfl_xor64(x.i, o)};
    x = better(x, y);
  }
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    sv[w] = x.v;
    si[w] = x.i;
  }
  __syncthreads();
  Best r{sv[0], si[0]};
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) r = better(r, Best{sv[i], si[i]});
  return r;
}

__global__ __launch_bounds__(256) void k_argmax_partial(const int32_t* __restrict__ logits,
                                                        const int64_t* __restrict__ head_m, int V,
                                                        int chunk, int64_t* pv, int64_t* pi) {
  keep_hidden_args();
  __shared__ i64 sv[4], si[4];
  const int r = blockIdx.y, ch = blockIdx.x, nch = gridDim.x;
  const int beg = ch * chunk, end = min(V, beg + chunk);
  Best b{INT64_MIN, (i64)V};
  const int32_t* row = logits + (i64)r * V;
  for (int i = beg + threadIdx.x; i < end; i += blockDim.x) {
    b = better(b, Best{wmul((i64)row[i], head_m[i]), (i64)i});
  }
  b = block_best(b, sv, si);
  if (threadIdx.x == 0) {
    pv[(i64)r * nch + ch] = b.v;
    pi[(i64)r * nch + ch] = b.i;
  }
}

__global__ __launch_bounds__(256) void k_argmax_final(const int64_t* pv, const int64_t* pi,
                                                      int nch, int64_t* out) {
  keep_hidden_args();
  __shared__ i64 sv[4], si[4];
  const int r = blockIdx.x;
  Best b{INT64_MIN, INT64_MAX};
  for (int i = threadIdx.x; i < nch; i += blockDim.x)
    b = better(b, Best{pv[(i64)r * nch + i], pi[(i64)r * nch + i]});
  b = block_best(b, sv, si);
  if (threadIdx.x == 0) out[r] = b.i;
}

// 64-bit digest of a logits row: the wrapping sum over i of the splitmix64
// finaliser of (i << 32) | (uint32) x_i. Addition modulo 2^64 is associative
// and commutative, so the block's reduction order cannot change the value.
__device__ __forceinline__ u64 mix64(u64 z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ __launch_bounds__(1024) void k_logits_digest(const int32_t* __restrict__ rows, int V,
                                                        int64_t* out) {
  keep_hidden_args();
  __shared__ i64 red_buf[32];
  BlockRedT<16> red{red_buf, 0, 1024};
  const int32_t* row = rows + (i64)blockIdx.x * V;
  i64 acc = 0;
  for (int i = threadIdx.x; i < V; i += blockDim.x)
    acc = wadd(acc, (i64)mix64(((u64)(uint32_t)i << 32) | (u64)(uint32_t)row[i]));
  acc = red.sum(acc);
  if (threadIdx.x == 0) out[blockIdx.x] = acc;
}

// Recommended K split of the skinny GEMM for an [M, K] x [N, K]^T product:
// enough (block, K-range) pairs to spread the weight stream over the CUs,
// at most 8 partials. The caller sizes the partial buffer with it. With
// several rows, a column count between one and four 16-column groups per CU
// splits K in two: the blocks then spread evenly over the CUs (gate|up at
// M = 8, N = 6144, K = 1024: 4.16 against 4.55 us per launch; one row takes
// the fused-operand kernels, planned for one split, at that shape).
int gemv_plan(int M, int N, int K) {
  const int groups = (N + 15) / 16;
  if (groups >= 1024) return 1;
  int ks = (256 + groups - 1) / groups;
  if (M > 1 && groups > 256) ks = 2;
  ks = ks < 1 ? 1 : (ks > 8 ? 8 : ks);
  const int kmax = K / 256 > 0 ? K / 256 : 1;
  if (ks > kmax) ks = kmax;
  int kchunk = (K + ks - 1) / ks;
  kchunk = (kchunk + 63) / 64 * 64;
  return (K + kchunk - 1) / kchunk;
}

template <int MB, int KW, int NB>
void launch_gemv(dim3 grid, hipStream_t s, const int8_t* A, const int8_t* B, int32_t* C,
                        int M, int N, int K, int kchunk, i64 split_stride, const Prefetch& pf) {
  const GemvArgs g{A, B, C, M, N, K, kchunk, split_stride};
  hipLaunchKernelGGL((k_gemv_nt<MB, KW, NB>), grid, dim3(256), 0, s, g, pf);
}

// Skinny GEMM for M <= 64: writes ksplit int32 partials C[ks][M][N]
// (split_stride elements apart); ksplit = 1 gives the plain product. Four
// waves share one 16-column group and split its K range (measured faster than
// a column group per wave at every layer shape); the LM head (N >= 32768,
// M <= 16, no split) takes k_gemv_stream instead.
int igemv(const int8_t* A, const int8_t* B, int32_t* C, int M, int N, int K, int ksplit,
          int64_t split_stride, const Prefetch& pf, hipStream_t s) {
  if (M <= 0 || N <= 0) return DI_OK;
  if (M > 64 || K <= 0 || (K % 16) != 0 || K > 131071 || ksplit < 1 || !A || !B || !C)
    return DI_EINVAL;
  if (ksplit > 1 && split_stride < (int64_t)M * N) return DI_EINVAL;
  const int kchunk = gemv_kchunk(K, ksplit);
  const int nsp = (K + kchunk - 1) / kchunk;
  if (nsp != ksplit) return DI_EINVAL;  // caller must size partial buffers to ksplit
  if (ksplit == 1 && M <= 16 && N >= 32768 && K <= GS_KMAX) {
    const int groups = (N + 15) / 16;
    const int blocks = (groups + 3) / 4 < GS_BLOCKS ? (groups + 3) / 4 : GS_BLOCKS;
    hipLaunchKernelGGL(k_gemv_stream, dim3(blocks), dim3(256), (size_t)16 * K, s, A, B, C, M, N,
                       K, pf);
    DI_LAUNCH_CHECK();
    return DI_OK;
  }
  const dim3 grid((N + 15) / 16, ksplit);
  const i64 ss = (i64)split_stride;
  if (M <= 16 && kchunk <= DEC_KMAX) {
    const GemvArgs g{A, B, C, M, N, K, kchunk, ss};
    hipLaunchKernelGGL(k_gemv_dec, grid, dim3(256), 0, s, g, pf);
    DI_LAUNCH_CHECK();
    return DI_OK;
  }
  switch ((M + 15) / 16) {
    case 1: launch_gemv<1, 4, 2>(grid, s, A, B, C, M, N, K, kchunk, ss, pf); break;
    case 2: launch_gemv<2, 4, 2>(grid, s, A, B, C, M, N, K, kchunk, ss, pf); break;
    case 3: launch_gemv<3, 4, 1>(grid, s, A, B, C, M, N, K, kchunk, ss, pf); break;
    default: launch_gemv<4, 4, 1>(grid, s, A, B, C, M, N, K, kchunk, ss, pf); break;
  }
  DI_LAUNCH_CHECK();
  return DI_OK;
}

}  // namespace

// Scratch of the allocation-free greedy pick: the per-chunk partial maxima
// (values, then ids) of k_argmax_partial, NOALLOC_PARTIALS int64 each. A
// file-scope device array: each GPU holds its own copy for the life of the
// process. Host code reaches it only through the address hipGetSymbolAddress
// returns for the current device (the array's name is not a device address
// on the host).
constexpr int NOALLOC_PARTIALS = 32768;
static __device__ __align__(256) int64_t scratch[2 * NOALLOC_PARTIALS];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
int64_t* g_scratch_ptr[MAX_DEVICES] = {};

// Address of this device's scratch, resolved once per device (with that
// device current); nullptr when the lookup fails.
int64_t* device_scratch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    g_scratch_ptr[dev] = (int64_t*)ptr;
  }
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" {

// C[b] = A[b] . B[b]^T; A [batch][M][K], B [batch][N][K], C [batch][M][N]
// (contiguous per batch, batch strides sA, sB, sC in elements). K % 16 == 0.
int detllm_igemm_nt(const int8_t* A, const int8_t* B, int32_t* C, int M, int N, int K, int batch,
                    int64_t sA, int64_t sB, int64_t sC, hipStream_t s) {
  if (M <= 0 || N <= 0 || batch <= 0) return DI_OK;
  if (K <= 0 || (K % 16) != 0 || K > 131071 || !A || !B || !C) return DI_EINVAL;
  if (batch > 65535) return DI_ERANGE;
  if (M > 64 && K % G2_BK == 0) {
    // Tile shape by tile count (a sweep of shapes over the four M = 2048
    // products picked these): 256x256 only for large products (c4 prefill),
    // 128x192 (two blocks per CU) where it divides N (gate|up), 128x128 (two
    // per CU) at >= 448 tiles (q|k|v), else 128x64 with a 4-slice ring (o,
    // down).
    auto tiles = [&](int bm, int bn) { return (i64)((M + bm - 1) / bm) * ((N + bn - 1) / bn) * batch; };
#define DI_GEMM2(BM, BN, S, WGM, WGN, MINB)                                                      \
  do {                                                                                          \
    const int tm_ = (M + BM - 1) / BM, tn_ = (N + BN - 1) / BN;                                 \
    if ((i64)tm_ * tn_ > 0x7fffffff) return DI_ERANGE;                                          \
    hipLaunchKernelGGL((k_gemm_nt2<BM, BN, S, WGM, WGN, MINB>), dim3(tm_ * tn_, 1, batch),     \
                       dim3(64 * WGM * WGN), 0, s, A, B, C, M, N, K, (i64)sA, (i64)sB, (i64)sC, \
                       tm_, tn_);                                                               \
  } while (0)
    if (tiles(256, 256) >= 448) DI_GEMM2(256, 256, 2, 4, 2, 1);
    else if (N % 192 == 0 && tiles(128, 192) >= 448) DI_GEMM2(128, 192, 2, 2, 2, 2);
    else if (tiles(128, 128) >= 448) DI_GEMM2(128, 128, 2, 2, 2, 2);
    else DI_GEMM2(128, 64, 4, 4, 2, 1);
#undef DI_GEMM2
    DI_LAUNCH_CHECK();
    return DI_OK;
  }
  const int tiles_m = (M + TBM - 1) / TBM, tiles_n = (N + TBN - 1) / TBN;
  if ((i64)tiles_m * tiles_n > 0x7fffffff) return DI_ERANGE;
  hipLaunchKernelGGL(k_gemm_nt, dim3(tiles_m * tiles_n, 1, batch), dim3(256), 0, s, A, B, C, M,
                     N, K, (i64)sA, (i64)sB, (i64)sC, tiles_n);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

// int_gemm + requant_i8_static for M <= 64 rows in one launch (k_gemv_static).
int detllm_igemv_requant_static(const int8_t* A, const int8_t* B, int M, int N, int K,
                                const int64_t* row_m, const int64_t* row_k,
                                const int64_t* col_m, int64_t col_k, int64_t s_m, int64_t s_k,
                                int8_t* y8, hipStream_t s) {
  if (M <= 0 || N <= 0) return DI_OK;
  if (M > 64 || K <= 0 || (K % 16) != 0 || K > 131071 || !A || !B || !col_m || !y8)
    return DI_EINVAL;
  const GemvArgs g{A, B, nullptr, M, N, K, K, 0};
  hipLaunchKernelGGL(k_gemv_static<GEMV_STATIC_NW>, dim3((N + 15) / 16), dim3(64 * GEMV_STATIC_NW),
                     0, s, g, row_m, row_k, col_m, (i64)col_k, (i64)s_m, (i64)s_k, y8);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_igemv_plan(int M, int N, int K, int* ksplit) {
  if (!ksplit || M <= 0 || M > 64 || N <= 0 || K <= 0 || (K % 16) != 0) return DI_EINVAL;
  *ksplit = gemv_plan(M, N, K);
  return DI_OK;
}

// Skinny GEMM for M <= 64 (igemv above).
int detllm_igemv_nt(const int8_t* A, const int8_t* B, int32_t* C, int M, int N, int K,
                    int ksplit, int64_t split_stride, hipStream_t s) {
  const Prefetch none{};
  return igemv(A, B, C, M, N, K, ksplit, split_stride, none, s);
}

// detllm_igemv_nt that also pulls up to four byte ranges, which the next
// kernels read, into the memory-side cache (see Prefetch); same results.
int detllm_igemv_nt_pf(const int8_t* A, const int8_t* B, int32_t* C, int M, int N, int K,
                       int ksplit, int64_t split_stride, const void* pf0, int64_t n0,
                       const void* pf1, int64_t n1, const void* pf2, int64_t n2,
                       const void* pf3, int64_t n3, hipStream_t s) {
  const void* ps[4] = {pf0, pf1, pf2, pf3};
  const int64_t ns[4] = {n0, n1, n2, n3};
  Prefetch pf{};
  for (int i = 0; i < 4; ++i) {
    if (ns[i] < 0 || (ns[i] > 0 && (!ps[i] || (ns[i] & 3) != 0 || ((uintptr_t)ps[i] & 3) != 0)))
      return DI_EINVAL;
    pf.p[i] = (const int8_t*)ps[i];
    pf.n[i] = ps[i] ? ns[i] : 0;
  }
  return igemv(A, B, C, M, N, K, ksplit, split_stride, pf, s);
}

// dst[b] = src[b]^T for int8 [R][C] matrices
int detllm_transpose_i8(const int8_t* src, int8_t* dst, int R, int Cc, int batch, int64_t sS,
                        int64_t sD, hipStream_t s) {
  if (R <= 0 || Cc <= 0 || batch <= 0) return DI_OK;
  if (!src || !dst || batch > 65535 || (R + 63) / 64 > 65535) return DI_EINVAL;
  hipLaunchKernelGGL(k_transpose_i8, dim3((Cc + 63) / 64, (R + 63) / 64, batch), dim3(256), 0, s,
                     src, dst, R, Cc, (i64)sS, (i64)sD);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

// greedy_pick: out[r] = lowest v maximising logits[r][v] * head_m[v].
// Scratch: pv, pi of R * nchunk int64 each; nchunk = ceil(V / chunk).
int detllm_greedy_pick(const int32_t* logits, const int64_t* head_m, int R, int V, int chunk,
                       int64_t* pv, int64_t* pi, int64_t* out, hipStream_t s) {
  if (R <= 0) return DI_OK;
  if (V <= 0 || chunk <= 0 || !logits || !head_m || !pv || !pi || !out) return DI_EINVAL;
  const int nch = (V + chunk - 1) / chunk;
  hipLaunchKernelGGL(k_argmax_partial, dim3(nch, R), dim3(256), 0, s, logits, head_m, V, chunk,
                     pv, pi);
  DI_LAUNCH_CHECK();
  hipLaunchKernelGGL(k_argmax_final, dim3(R), dim3(256), 0, s, pv, pi, nch, out);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

// detllm_greedy_pick without caller scratch and without any allocation: the
// partials live in the library's per-device `scratch` array (chunk 2048, so
// R * ceil(V / 2048) <= NOALLOC_PARTIALS). Every partial slot a call reads
// is written earlier in the same call, so nothing needs clearing; calls that
// overlap on one GPU (different streams) share the array and race.
int detllm_greedy_pick_noalloc(const int32_t* logits, const int64_t* head_m, int R, int V,
                               int64_t* out, hipStream_t s) {
  if (R <= 0) return DI_OK;
  if (V <= 0 || !logits || !head_m || !out) return DI_EINVAL;
  constexpr int chunk = 2048;
  const int nch = (V + chunk - 1) / chunk;
  if ((int64_t)R * nch > NOALLOC_PARTIALS) return DI_ERANGE;
  int64_t* ptr = device_scratch();
  if (!ptr) return (int)hipErrorInvalidSymbol;
  int64_t* pv = ptr;
  int64_t* pi = ptr + NOALLOC_PARTIALS;
  hipLaunchKernelGGL(k_argmax_partial, dim3(nch, R), dim3(256), 0, s, logits, head_m, V, chunk,
                     pv, pi);
  DI_LAUNCH_CHECK();
  hipLaunchKernelGGL(k_argmax_final, dim3(R), dim3(256), 0, s, pv, pi, nch, out);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

// One 64-bit digest per int32 row [R][V] (k_logits_digest).
int detllm_logits_digest(const int32_t* rows, int R, int V, int64_t* out, hipStream_t s) {
  if (R <= 0) return DI_OK;
  if (V <= 0 || !rows || !out || R > 0x7fffffff) return DI_EINVAL;
  hipLaunchKernelGGL(k_logits_digest, dim3(R), dim3(1024), 0, s, rows, V, out);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

}  // extern "C"
