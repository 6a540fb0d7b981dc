// Integer GQA attention over the int8 KV cache (gfx950).
//
// Semantics (bit-exact): scores = q8 . k8 (int32); DI-Softmax with the TRUE
// row max over visible slots (ops/di_softmax.py:33-61 — DI-Exp is not
// multiplicative, so no online rescaling); probabilities
// p = round_half_away_div(exp << 14, max(sum exp, 1)) in [0, 2^14]; context
// = sum_s p_s * v_s exactly in int64 (model.py:363-402 and the hi/lo GEMM of
// backends.py:152-164 produce the same integer). Slot s is visible to the
// query at absolute slot S_past + t iff s <= S_past + t and valid[b][s]
// (model.py:259-266).
//
// Cache layout in HBM: paged (common.h KVPages). A row's slots map through
// its page table to pages of DI_PAGE = 128 slots; a page holds K rows
// [n_kv][128 slots][128] and V transposed [n_kv][128 channels][128 slots], so
// both the MFMA B-fragments of P.V (16 consecutive slots per lane) and the
// decode reduction over slots read slot-contiguous bytes. A prefill key tile
// is exactly one page.
//
// Prefill (k_attn_prefill): block = 64 queries of one head, 4 waves of 16.
// Scores are computed transposed, S^T = K . Q^T, with v_mfma_i32_16x16x64_i8:
// lane l then holds ONE query (l % 16) and 16 slots of each 64-slot tile, so
// the row max, the denominator and the DI-Exp / normalisation divisors are
// per-lane scalars. Three passes over the key tiles (max, denominator,
// normalise + P.V) recompute S^T on MFMA. P.V uses the same fragments: the
// 15-bit p is split as p = 128*hi + lo, and sum p.v =
// 128*(sum (hi-64).v + 64*colsum(v)) + sum lo.v, both products on i8 MFMA
// (hi-64 in [-64, 64], lo in [0, 127]).
//
// Decode (k_attn_decode): block = one (batch row, kv head), all q heads of
// its group; scores live in LDS (or a global scratch when they do not fit);
// every reduction is an exact integer max/sum.

#include <type_traits>

#include "common.h"
#include "qkv_epilogue.h"

using namespace di;

typedef int v4i __attribute__((ext_vector_type(4)));

namespace {

__device__ __forceinline__ v4i mfma16(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

struct PrefillArgs {
  const int8_t* q8;      // [B][n_q][T][128]
  const int64_t* tpos;   // [B][n_q][T]
  KVPages kv;
  const uint8_t* valid;  // [B][valid_stride]
  int64_t* out;          // [B][T][n_q * 128]
  int T, S, S_past, n_q, n_kv, B;
  i64 valid_stride;
};

constexpr int PF_KBYTES = 128 * 128;      // K tile: 128 slot rows of 128 B
constexpr int PF_VBYTES = 128 * 128;      // V^T tile: 128 dim rows of 128 B
constexpr int PF_RING = 64 * 1024;        // 4 K stages, or 2 K+V stages
constexpr int PF_CSUM = 128 * 4;          // column sums of V (int32 per dim)
constexpr uint32_t PF_SMALL_T = 1u << 23;  // estimated DI-Exp below this tpos
constexpr i64 PF_SMALL_DEN = (i64)1 << 34;  // estimated p below this den

// 16-byte chunk swizzles of the LDS tiles (128-byte rows, physical chunk =
// logical ^ swz). An MFMA operand read takes one chunk column of 16 rows per
// 16 lanes: K rows 16(i/4) + 4 blk + i%4 and V^T rows (dims) 16 j + i for
// i = 0..15. With swz = bits 0, 1 and 4 of the K row (i % 4 and i / 4 % 2)
// and the low 3 bits of the V^T row, both reads run at the full LDS rate of
// 16 bytes per lane (measured on gfx950; an unswizzled read takes 4 times as
// long, swizzles on other row bits twice as long).
__device__ __forceinline__ int pf_kswz(int row) { return (row & 3) | ((row >> 2) & 4); }
__device__ __forceinline__ int pf_vswz(int d) { return d & 7; }

// Per-query constants of the estimated DI-Exp and division (intops.h).
struct PfFast {
  ExpEst E;    // tpos < 2^23
  double kx;   // dexp_sp_const(E)
  int32_t cx;  // t - mx: the score MFMAs of passes 2 and 3 start from it
  DivEst D;    // make_divest(den, 2^14): p = rhad(ex << 14, den), den < 2^34
};

// Four probabilities (slot order = byte order) as the two MFMA operands of
// the hi/lo split p = 128 hi + lo: bytes hi - 64 = (p - 8192) >> 7 in
// [-64, 64] (byte 1 of 2p - 16384) and lo = p & 127.
__device__ __forceinline__ void pf_pack(const uint32_t (&p)[4], int& whi, int& wlo) {
  uint32_t y[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) y[r] = (p[r] << 1) - 16384u;
  const uint32_t h01 = __builtin_amdgcn_perm(y[1], y[0], 0x0c0c0501u);
  const uint32_t h23 = __builtin_amdgcn_perm(y[3], y[2], 0x05010c0cu);
  const uint32_t l01 = __builtin_amdgcn_perm(p[1], p[0], 0x0c0c0400u);
  const uint32_t l23 = __builtin_amdgcn_perm(p[3], p[2], 0x04000c0cu);
  whi = (int)(h01 | h23);
  wlo = (int)((l01 | l23) & 0x7f7f7f7fu);
}

__global__ __launch_bounds__(256, 2) void k_attn_prefill(PrefillArgs a) {
  keep_hidden_args();
  __shared__ __attribute__((aligned(1024))) int8_t ring[PF_RING];
  // PF_CSUM + 8 per 64 slots (tile masks) + 4 per page (page ids)
  extern __shared__ __attribute__((aligned(16))) int8_t dyn[];
  int32_t* const csum_lds = (int32_t*)dyn;
  u64* const vmask = (u64*)(dyn + PF_CSUM);  // per 64-slot key tile
  int32_t* const pages = (int32_t*)(dyn + PF_CSUM + 8 * ((a.S + 63) / 64));
  // Causal work per query tile grows with its index. Pair pi = (b, h, k)
  // (k fastest) stands for the heavy tile nqt - 1 - k and its light partner
  // k. Blocks are dispatched round-robin over the 8 XCDs (XCD = blockIdx % 8);
  // when the pairs split evenly, XCD x takes the contiguous pairs
  // [x pairs/8, (x + 1) pairs/8) — whole heads, so each XCD's L2 holds only
  // its own heads' K and V — heavy tiles first, then the light ones, so the
  // two blocks a CU holds together add up to about the same work. Otherwise
  // the first half of the grid takes the heavy tiles and the second half the
  // light ones. The middle tile of an odd count appears once.
  const int nqt = (a.T + 63) / 64, np = (nqt + 1) / 2;
  const int pairs = np * a.n_q * a.B;
  int half, pi;
  if (pairs % 8 == 0) {
    const int per = pairs / 8, j = blockIdx.x >> 3;
    half = j >= per;
    pi = (blockIdx.x & 7) * per + (j - half * per);
  } else {
    half = blockIdx.x >= pairs;
    pi = blockIdx.x - half * pairs;
  }
  const int kk = pi % np, hb = pi / np;
  if (half && kk == nqt - 1 - kk) return;  // middle tile: done by the first half
  const int qt = half ? kk : nqt - 1 - kk;
  const int h = hb % a.n_q, b = hb / a.n_q;
  const int kvh = h / (a.n_q / a.n_kv);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int qi = lane & 15, g = lane >> 4;
  const int t = qt * 64 + wave * 16 + qi;  // this lane's query
  const bool tok = t < a.T;
  const i64 qrow = ((i64)b * a.n_q + h) * a.T + (tok ? t : 0);
  v4i qf0 = v4i{0, 0, 0, 0}, qf1 = v4i{0, 0, 0, 0};
  if (tok) {
    qf0 = *(const v4i*)(a.q8 + qrow * 128 + g * 16);
    qf1 = *(const v4i*)(a.q8 + qrow * 128 + 64 + g * 16);
  }
  const i64 tpos = tok ? a.tpos[qrow] : 1;
  const int limit = a.S_past + t;              // last visible slot of this query
  const int wlim = a.S_past + qt * 64 + wave * 16;  // the smallest limit in the wave
  const int kend = min(a.S, a.S_past + qt * 64 + 64);
  const int ntiles = (kend + 63) / 64;
  const uint8_t* vrow = a.valid + (i64)b * a.valid_stride;
  const int ntiles2 = (ntiles + 1) / 2;  // 128-slot tiles = pages
  for (int i = tid; i < ntiles2; i += 256) pages[i] = a.kv.page(b, (i64)i * DI_PAGE);

  // validity bitmask of every key tile (bit s - 64 i of tile i: slot s < S
  // and valid), made once and read by all three passes for the tiles that
  // are not valid in full; nfull = the first tile that is not
  int nf = ntiles;
  for (int i0 = wave; i0 < ntiles; i0 += 16) {
    uint32_t f[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int s = (i0 + 4 * u) * 64 + lane;
      const uint32_t v = vrow[s < a.S ? s : 0];  // unconditional: one wait for all four
      f[u] = (i0 + 4 * u < ntiles && s < a.S) ? v : 0u;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + 4 * u;
      const u64 m = __ballot(f[u] != 0);
      if (lane == 0 && i < ntiles) vmask[i] = m;
      if (i < ntiles && m != ~0ull) nf = min(nf, i);
    }
  }
  if (lane == 0) csum_lds[wave] = nf;  // the column-sum area is free until the end
  __syncthreads();
  const int nfull = min(min(csum_lds[0], csum_lds[1]), min(csum_lds[2], csum_lds[3]));
  wait_vmcnt<0>();  // query operands in registers before the ring's loads count

  // Key tiles of 128 slots stream into an LDS ring with direct-to-LDS loads,
  // issued STAGES - 1 tiles ahead; each tile is processed as two 64-slot
  // halves (the 64-slot tiles `it` of the masks) between one barrier and the
  // next. K: instruction j of wave w covers tile rows 8(4w + j) .. +7, lane l
  // row 8(4w + j) + l/8 at physical chunk l % 8; V^T likewise with dims for
  // rows. A tile is one page; the buffer resources span that page's
  // (kv head) part, 16 KB of K and of V^T. A page that is not mapped gets a
  // zero-length resource, so its loads read 0. Slots past the scanned range
  // in a mapped page read whatever the page holds; such slots are never
  // visible (p = 0: their hi byte -64 and the +64 column-sum term cancel).
  int koffl[4], voffl[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = (wave * 4 + j) * 8 + (lane >> 3);
    koffl[j] = row * 128 + ((lane & 7) ^ pf_kswz(row)) * 16;
    voffl[j] = row * DI_PAGE + ((lane & 7) ^ pf_vswz(row)) * 16;
  }
  auto issue = [&](int tile, int8_t* st, bool with_v) {
    const int pg = __builtin_amdgcn_readfirstlane(pages[tile]);
    const int pgc = pg < 0 ? 0 : pg;
    const int nrec = pg < 0 ? 0 : DI_PAGE * 128;
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.kv.krow(pgc, kvh, 0), (short)0, nrec, 0x00020000);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_ptr_t)(st + (wave * 4 + j) * 1024), 16,
                                               koffl[j], 0, 0, 0);
    if (with_v) {
      const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
          (void*)a.kv.vchan(pgc, kvh, 0), (short)0, nrec, 0x00020000);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            vrs, (lds_ptr_t)(st + PF_KBYTES + (wave * 4 + j) * 1024), 16, voffl[j], 0, 0, 0);
    }
  };
  // one pass over the key tiles; body(it2, stage) runs with tile it2 in LDS.
  // Each wave waits for its own loads of the tile (vmcnt: loads complete in
  // order), then one barrier publishes every wave's part and frees the
  // stage that the next issue overwrites.
  auto pass = [&](auto kv, auto&& body) {
    constexpr bool KV = decltype(kv)::value;
    constexpr int STAGE = KV ? PF_KBYTES + PF_VBYTES : PF_KBYTES;
    constexpr int ST = PF_RING / STAGE;
    constexpr int LPT = KV ? 8 : 4;  // loads per tile per wave
    static_assert(ST >= 2 && ST <= 4 && 2 * LPT < 64, "ring stages");
    __builtin_amdgcn_s_barrier();  // the previous pass is done with the ring
#pragma unroll
    for (int s = 0; s < ST - 1; ++s)
      if (s < ntiles2) issue(s, ring + s * STAGE, KV);
    for (int it2 = 0; it2 < ntiles2; ++it2) {
      const int after = min(ST - 2, ntiles2 - 1 - it2);  // tiles issued after it2
      if (after >= 2) wait_vmcnt<2 * LPT>();
      else if (after == 1) wait_vmcnt<LPT>();
      else wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();
      if (it2 + ST - 1 < ntiles2) issue(it2 + ST - 1, ring + ((it2 + ST - 1) % ST) * STAGE, KV);
      body(it2, ring + (it2 % ST) * STAGE);
    }
  };

  // S^T = K . Q^T for one 64-slot half: MFMA block blk takes K rows
  // 16(i/4) + 4 blk + i%4 as its rows i, so lane (qi, g) receives the scores
  // of query qi for the 16 consecutive slots 16 g + 4 blk + r (blk, r < 4):
  // st[blk][r]. Those are also the 16 bytes of its P operand for P.V, in
  // the slot order of the V^T rows.
  const int kr = 16 * (qi >> 2) + (qi & 3);
  const int koff0 = kr * 128 + ((g ^ pf_kswz(kr)) << 4);
  const int koff1 = kr * 128 + (((g + 4) ^ pf_kswz(kr)) << 4);
  auto load_k = [&](const int8_t* st_k, v4i (&kf)[8]) {
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      kf[2 * blk] = *(const v4i*)(st_k + koff0 + blk * 512);
      kf[2 * blk + 1] = *(const v4i*)(st_k + koff1 + blk * 512);
    }
  };
  // both halves' K operands read at once (one LDS latency), then their
  // score MFMAs from accumulator z: the first 64 dims of all 8 blocks, then
  // the second 64 — the
  // two MFMAs of a block are 8 issues apart, so none waits on the previous
  // one's result — overlapping the first half's VALU work; then
  // fn(st, it, half) per half that holds key slots
  auto halves = [&](const int8_t* stg, int it2, const v4i z, auto&& fn) {
    v4i ka[8], kb[8], sa[4], sb[4];
    load_k(stg, ka);
    load_k(stg + 64 * 128, kb);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) sa[blk] = mfma16(ka[2 * blk], qf0, z);
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) sb[blk] = mfma16(kb[2 * blk], qf0, z);
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) sa[blk] = mfma16(ka[2 * blk + 1], qf1, sa[blk]);
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) sb[blk] = mfma16(kb[2 * blk + 1], qf1, sb[blk]);
    __builtin_amdgcn_sched_barrier(0);
    fn(sa, 2 * it2, 0);
    if (2 * it2 + 1 < ntiles) fn(sb, 2 * it2 + 1, 1);
  };
  // tile `it` is visible in full to every query of the wave (wave-uniform)
  auto full_tile = [&](int it) { return it < nfull && it * 64 + 63 <= wlim; };
  // this lane's visibility bits: bit 4 blk + r for slot 16 g + 4 blk + r
  auto lane_bits = [&](int it, u64 vm) -> uint32_t {
    const int e = limit - it * 64 - 16 * g;  // last visible offset in the lane's 16
    const uint32_t cb = e >= 15 ? 0xFFFFu : (e < 0 ? 0u : (2u << e) - 1u);
    return (uint32_t)(vm >> (16 * g)) & cb;
  };

  // ---- pass 1: row max over visible slots (scores are int32)
  int mx = INT32_MIN;
  pass(std::false_type{}, [&](int it2, const int8_t* stg) { halves(stg, it2, v4i{0, 0, 0, 0}, [&](const v4i (&st)[4], int it, int) {
    if (full_tile(it)) {
#pragma unroll
      for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = max(mx, st[blk][r]);
    } else {
      const uint32_t bits = lane_bits(it, vmask[it]);
#pragma unroll
      for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if ((bits >> (4 * blk + r)) & 1u) mx = max(mx, st[blk][r]);
    }
  }); });
  mx = max(mx, __shfl_xor(mx, 16));
  mx = max(mx, __shfl_xor(mx, 32));
  if (mx == INT32_MIN) mx = 0;  // no visible slot: max := 0, every p = 0

  // ---- pass 2: denominator. The estimated DI-Exp runs when every query of
  // the wave has tpos < 2^23 (then every exp is below 2^23 and 16 of them sum
  // in 32 bits); otherwise the general 64-bit form. Masked slots enter the
  // estimate as st = mx (a defined conversion) and are then dropped.
  const bool fexp = __ballot(tpos >= (i64)PF_SMALL_T) == 0;
  PfFast F;
  F.E = make_expest(tpos);
  F.kx = dexp_sp_const(F.E);
  F.cx = (int32_t)(F.E.t - (uint32_t)mx);
  // fast path: scores arrive as st + t - mx; the general path subtracts it
  const int32_t soff = fexp ? F.cx : 0;
  const v4i cinit = v4i{soff, soff, soff, soff};
  const ExpR Et = make_exp(tpos);
  i64 den = 0;
  pass(std::false_type{}, [&](int it2, const int8_t* stg) { halves(stg, it2, cinit, [&](const v4i (&st)[4], int it, int) {
    if (fexp && full_tile(it)) {
      uint32_t sum = 0;
#pragma unroll
      for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int r = 0; r < 4; ++r) sum += dexp_est_sp(st[blk][r], F.E, F.kx);
      den += sum;
      return;
    }
    const uint32_t bits = lane_bits(it, vmask[it]);
    if (fexp) {
      uint32_t sum = 0;
#pragma unroll
      for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool vis = (bits >> (4 * blk + r)) & 1u;
          const uint32_t e = dexp_est_sp(vis ? st[blk][r] : (int32_t)F.E.t, F.E, F.kx);
          sum += vis ? e : 0u;
        }
      den += sum;
    } else {
#pragma unroll
      for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if ((bits >> (4 * blk + r)) & 1u)
            den = wadd(den, di_exp_neg((u64)(uint32_t)(mx - (st[blk][r] - soff)), Et));
    }
  }); });
  den = imax(group4_sum(den), 1);
  const bool fdiv = fexp && __ballot(den >= PF_SMALL_DEN) == 0;
  F.D = make_divest(den, 16384.0);
  const Recip Rd = make_recip(den);

  // ---- pass 3: p, then P.V on MFMA with the hi/lo split; wave w also sums
  // the V^T rows of dims 32w .. 32w + 31 (an all-ones A operand) for the
  // +64 correction of the hi bytes
  v4i ohi[8], olo[8], ocs[2];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    ohi[j] = v4i{0, 0, 0, 0};
    olo[j] = v4i{0, 0, 0, 0};
  }
  ocs[0] = ocs[1] = v4i{0, 0, 0, 0};
  const v4i ones = v4i{0x01010101, 0x01010101, 0x01010101, 0x01010101};
  // V^T operand of half `hf`: dim 16 j + qi, slots 64 hf + 16 g .. + 15
  // (the swizzle of dim 16 j + qi does not depend on j)
  int voff[2];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) voff[hf] = PF_KBYTES + qi * 128 + (((4 * hf + g) ^ pf_vswz(qi)) << 4);
  pass(std::true_type{}, [&](int it2, const int8_t* stg) { halves(stg, it2, cinit, [&](const v4i (&st)[4], int it, int hf) {
    v4i vf[8], vc[2];
#pragma unroll
    for (int j = 0; j < 8; ++j) vf[j] = *(const v4i*)(stg + voff[hf] + j * 2048);
#pragma unroll
    for (int c = 0; c < 2; ++c) vc[c] = *(const v4i*)(stg + voff[hf] + (2 * wave + c) * 2048);
    __builtin_amdgcn_sched_barrier(0);
    const bool full = full_tile(it);
    uint32_t bits = 0xFFFFu;
    if (!full) bits = lane_bits(it, vmask[it]);
    v4i phi, plo;
    auto put = [&](int blk, const uint32_t (&p)[4]) {
      int whi, wlo;
      pf_pack(p, whi, wlo);
      phi[blk] = whi;
      plo[blk] = wlo;
    };
    if (fdiv && full) {
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        uint32_t p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) p[r] = rhad_est((double)dexp_est_sp(st[blk][r], F.E, F.kx), F.D);
        put(blk, p);
      }
    } else if (fdiv) {
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        uint32_t p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool vis = (bits >> (4 * blk + r)) & 1u;
          const uint32_t e = dexp_est_sp(vis ? st[blk][r] : (int32_t)F.E.t, F.E, F.kx);
          p[r] = rhad_est((double)(vis ? e : 0u), F.D);
        }
        put(blk, p);
      }
    } else {
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        uint32_t p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          i64 pv = 0;
          if ((bits >> (4 * blk + r)) & 1u) {
            const i64 ex = di_exp_neg((u64)(uint32_t)(mx - (st[blk][r] - soff)), Et);
            pv = to_i32(rhad_r(shl(ex, 14), Rd));
          }
          p[r] = (uint32_t)pv;
        }
        put(blk, p);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ohi[j] = mfma16(phi, vf[j], ohi[j]);
      olo[j] = mfma16(plo, vf[j], olo[j]);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) ocs[c] = mfma16(ones, vc[c], ocs[c]);
  }); });
  // column sums: every row of ocs[c] holds sum_s v[s][32 wave + 16 c + qi]
  if (g == 0) {
    csum_lds[32 * wave + qi] = ocs[0][0];
    csum_lds[32 * wave + 16 + qi] = ocs[1][0];
  }
  __syncthreads();
  // write: lane holds O[query 4g + r][d = 16j + qi]
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const i64 cs = csum_lds[16 * j + qi];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tq = qt * 64 + wave * 16 + g * 4 + r;
      if (tq < a.T) {
        const i64 v = (i64)ohi[j][r] * 128 + cs * 8192 + (i64)olo[j][r];
        a.out[((i64)b * a.T + tq) * (a.n_q * 128) + h * 128 + j * 16 + qi] = v;
      }
    }
  }
}

struct DecodeArgs {
  const int8_t* q8;      // [B][n_q][128]
  const int64_t* tpos;   // [B][n_q]
  KVPages kv;
  const uint8_t* valid;  // [B][valid_stride]
  int64_t* out;          // [B][n_q * 128]
  int32_t* scratch;      // [B][n_q][S] when scores do not fit in LDS, else null
  const int64_t* s_dev;  // optional device bound on the scanned slots
  int S, n_q, n_kv;
  i64 valid_stride;
  int32_t* err;          // optional device error word (DI_ERR_SLOTS)
  // optional (both or neither): the attention-output merge's per-column
  // factor om [n_q * 128] and its row statistics ext [B][n_kv][2] — per
  // (row, kv head) block the largest v and the largest ~v over the block's
  // outputs v = out * om (int64, wrapping) and 0
  const int64_t* om;
  int64_t* ext;
};

constexpr int DEC_MAX_PAGES = 1024;  // ceil(131071 / DI_PAGE)

constexpr int MAXG = 8;
constexpr i64 DECODE_LDS_BYTES = 48 * 1024;

constexpr int32_t SCORE_MASKED = INT32_MIN;  // |q.k| <= 128*128*128 < 2^31: never a score
constexpr int DEC_MAX_S = 131071;            // int32 MFMA accumulators of P.V
constexpr int VPRE = 4;                      // 64-slot steps of V loaded before the scores
// The same for the fused eight-wave kernel (one 16-channel block per wave):
// six steps (384 slots) measured fastest at c3's ~320 slots (4: 1.595, 6:
// 1.561, 8: 1.569 ms per b8 step): loads past the row's steps are wasted
// traffic through the CU's load path, and the steps past the prefetch cost a
// round trip in the P.V loop.
constexpr int VPRE_FUSED = 6;

// DPP max over each aligned row of 16 lanes (result in every lane of the row)
__device__ __forceinline__ int32_t row16_max(int32_t v) {
  v = ::max(v, __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false));
  v = ::max(v, __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false));
  v = ::max(v, __builtin_amdgcn_update_dpp(v, v, 0x141, 0xF, 0xF, false));
  v = ::max(v, __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, false));
  return v;
}

// Attention of one (batch row b, kv head kvh) over its G query heads, whose
// int8 rows sit at qsrc[hh * 128] and DI-Exp constants at tsrc[hh] (global
// memory or LDS). NW waves (decode_body's template argument, 4 or 8).
//
// Scores and P.V run on v_mfma_i32_16x16x64_i8 with the G query heads as the
// 16 MFMA rows (rows >= G zero):
//   * scores: C[hh][slot] = sum_d q[hh][d] k[slot][d]; a wave takes blocks of
//     16 slots, B-fragment lane l = slot l % 16, bytes 16 (l / 16) (+ 64) of
//     the slot's K row (two MFMAs over the 128 channels);
//   * P.V with the prefill's exact hi/lo split of p in [0, 2^14]:
//     p = 128 hi + lo, sum p v = 128 (sum (hi - 64) v + 64 colsum v) + sum lo v;
//     A rows hh < G hold hi - 64 (resp. lo) of 64 consecutive slots, and row G
//     of the hi product holds ones, so C_hi[G][d] = colsum v over exactly the
//     slots of the B fragments; B-fragment lane l = channel l % 16, slots
//     16 (l / 16) .. + 15 of V^T (slot-contiguous). Wave w owns channels
//     (128 / NW) w .. + 128 / NW - 1 (8 / NW 16-channel blocks).
// Slots past S read zero V fragments (16-slot chunks starting at or past S),
// so their A values do not matter; the p of slots S .. ceil16(S) are 0.
// |accumulators| <= 128 * 128 * S < 2^31 for S <= 131071.
// p in [0, 2^14] packed as (hi - 64) | lo << 8 (p = 128 hi + lo; p = 0 packs
// as hi - 64 = -64, lo = 0)
__device__ __forceinline__ int32_t pack_p(i64 p) {
  const int hi = (int)(p >> 7), lo = (int)(p & 127);
  return (int32_t)((uint32_t)(uint8_t)(int8_t)(hi - 64) | ((uint32_t)lo << 8));
}

// MFMA A fragments of 16 packed p words (16 consecutive slots of one head):
// bytes 0 of the words -> hi - 64 fragment, bytes 1 -> lo
__device__ __forceinline__ void p_frags(const int32_t* pp, v4i& ahi, v4i& alo) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const v4i w = *(const v4i*)(pp + 4 * q);
    const uint32_t h01 = __builtin_amdgcn_perm((uint32_t)w[1], (uint32_t)w[0], 0x0c0c0400u);
    const uint32_t h23 = __builtin_amdgcn_perm((uint32_t)w[3], (uint32_t)w[2], 0x04000c0cu);
    const uint32_t l01 = __builtin_amdgcn_perm((uint32_t)w[1], (uint32_t)w[0], 0x0c0c0501u);
    const uint32_t l23 = __builtin_amdgcn_perm((uint32_t)w[3], (uint32_t)w[2], 0x05010c0cu);
    ahi[q] = (int)(h01 | h23);
    alo[q] = (int)(l01 | l23);
  }
}

// sum_s p_s v_s of the wave's channels from the hi/lo accumulators: lane
// (grp, l16), element r holds head 4 grp + r, channel 16 (NB wave + nb) + l16;
// the colsum of that channel sits in row G (lane 16 (G / 4) + l16, element
// G % 4). out_heads: the block's first head row of [.][128] int64.
// each(nb, r, value) sees every stored value.
template <int G, int NB = 2, class Each>
__device__ __forceinline__ void store_pv(const v4i (&chi)[NB], const v4i (&clo)[NB],
                                         int64_t* out_heads, Each&& each) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, grp = lane >> 4;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int cs_src = (G / 4) * 16 + l16;
    const int32_t cs = __shfl(chi[nb][G % 4], cs_src, 64);
    const int d = wave * 16 * NB + nb * 16 + l16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hh = grp * 4 + r;
      if (hh < G) {
        const i64 o = ((i64)chi[nb][r] + 64 * (i64)cs) * 128 + (i64)clo[nb][r];
        out_heads[hh * 128 + d] = o;
        each(nb, r, o);
      }
    }
  }
}
template <int G, int NB = 2>
__device__ __forceinline__ void store_pv(const v4i (&chi)[NB], const v4i (&clo)[NB],
                                         int64_t* out_heads) {
  store_pv<G, NB>(chi, clo, out_heads, [](int, int, i64) {});
}

// The slots a decode block scans: a.S, bounded by the device count when one
// is given. Without one the load reads `always` (a pointer every launch
// has) and the value is selected after it: no branch around the load, whose
// merge would make every earlier load complete first. *over: the device
// count exceeds a.S; the reference would scan those slots, so the result
// would differ, and report_slots raises DI_ERR_SLOTS (after the kernel's
// last load: a pending atomic among loads makes every wait a full one).
__device__ __forceinline__ int scanned_slots(const DecodeArgs& a, const int64_t* always,
                                             bool* over) {
  const int64_t* p = a.s_dev ? a.s_dev : always;
  const i64 sd = p[0];
  *over = a.s_dev != nullptr && sd > (i64)a.S;
  return a.s_dev ? (int)imax(0, imin((i64)a.S, sd)) : a.S;
}
__device__ __forceinline__ void report_slots(const DecodeArgs& a, bool over, bool who) {
  if (over && who && a.err && threadIdx.x == 0) atomicOr(a.err, DI_ERR_SLOTS);
}

// K rows and validity flags of the first KPRE_SLOTS slots of the row, loaded
// before the fused kernel's Q/K/V epilogue so that their latency hides behind
// it; the slot the epilogue writes is taken from LDS instead. With NW waves a
// wave holds IT = KPRE_SLOTS / (64 NW) iterations of four 16-slot blocks.
constexpr int KPRE_SLOTS = 512;
template <int IT>
struct KPre {
  v4i kb[IT][4][2];
  int vf[IT][4];                 // 0 for slots of pages that are not mapped
  int pg[KPRE_SLOTS / DI_PAGE];  // the pages of those slots (-1: not mapped or past S)
  const int8_t* k_new;           // LDS, 128 bytes
  i64 new_slot;                  // -1: none
};

// S: the slots to scan (scanned_slots). pg_lds: the row's page ids for
// slots [0, S) (filled by the caller, before a barrier). Slots whose page is
// not mapped are masked and read page 0. VP: 64-slot steps of V loaded ahead.
// SCR: the scores live in the global scratch (a.scratch) instead of LDS (a
// compile-time choice: LDS-only code never issues flat accesses, which would
// wait on every outstanding load). NW: waves of the block (4 or 8): a wave
// takes every NW-th 16-slot block of the scores and 128 / NW channels of P.V.
// The merge factors of a lane's outputs (store_pv's layout: head 4 grp + r,
// channel 16 (NB wave + nb) + l16; heads past G read entry 0), loaded where
// the caller's first loads issue.
template <int G, int NB>
struct OmPre {
  static constexpr int RG = G < 4 ? G : 4;
  i64 v[NB][RG];
  __device__ __forceinline__ void load(const DecodeArgs& a, int kvh) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, grp = lane >> 4;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        const int hh = grp * 4 + r;
        const int d = wave * 16 * NB + nb * 16 + l16;
        v[nb][r] = a.om[hh < G ? (kvh * G + hh) * 128 + d : 0];
      }
  }
};

// OMP: omp holds the merge factors (else decode_body loads them when a.ext
// is set).
template <int G, int VP, bool SCR, bool PRE = false, int NW = 4, bool OMP = false>
__device__ __forceinline__ void decode_body(const DecodeArgs& a, int S, int kvh, int b,
                                            const int8_t* qsrc, const int64_t* tsrc,
                                            int32_t* sh_scores, const int32_t* pg_lds,
                                            const KPre<8 / NW>& pre = KPre<8 / NW>{},
                                            const OmPre<G, 8 / NW>& omp = OmPre<G, 8 / NW>{}) {
  static_assert(G <= 8, "query heads per kv head");
  static_assert(NW == 4 || NW == 8, "waves per block");
  constexpr int NT = NW * 64;  // threads
  constexpr int NB = 8 / NW;   // 16-channel blocks of P.V per wave
  constexpr int IT = 8 / NW;   // prefetched iterations per wave
  __shared__ i64 red_buf[32];
  BlockRedT<NT / 64> red{red_buf, 0, NT};
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, grp = lane >> 4;
  const int Spad = (a.S + 15) & ~15;
  int32_t* sc = SCR ? a.scratch + ((i64)b * a.n_q + kvh * G) * Spad : sh_scores;
  const uint8_t* vrow = a.valid + (i64)b * a.valid_stride;
  const int nstep = (S + 63) / 64;  // 64-slot steps of P.V
  auto pg_of = [&](int s) -> int {  // page of slot s < S, page 0 when not mapped
    const int pg = pg_lds[s >> 7];
    return pg < 0 ? 0 : pg;
  };

  // V fragments of 64-slot steps (a step lies in one page). Loads are
  // unconditional (no branch whose merge would make them complete early): a
  // 16-slot group at or past S reads slot 0's bytes, and every A row of such
  // a group, the colsum row included, is zero.
  auto vfrag = [&](int st, int nb) -> v4i {
    const int s0 = st * 64 + grp * 16;
    const int sl = s0 < S ? s0 : 0;
    const int8_t* vch = a.kv.vchan(pg_of(sl), kvh, wave * 16 * NB + nb * 16 + l16);
    return *(const v4i*)(vch + (sl & (DI_PAGE - 1)));
  };
  // the same for a step below KPRE_SLOTS with the pages in registers (no LDS
  // read before the load): slot st * 64 + 16 grp lies in page st / 2 (a group
  // at or past S reads offset 0 of that page, or of page 0 when it is not
  // mapped; its A rows are zero)
  auto vfrag_pre = [&](int st, int nb) -> v4i {
    const int s0 = st * 64 + grp * 16;
    const int sl = s0 < S ? s0 : 0;
    const int pg = pre.pg[st >> 1];
    const int8_t* vch = a.kv.vchan(pg < 0 ? 0 : pg, kvh, wave * 16 * NB + nb * 16 + l16);
    return *(const v4i*)(vch + (sl & (DI_PAGE - 1)));
  };

  // the merge factors of this lane's outputs, used after P.V
  constexpr int RG = OmPre<G, NB>::RG;
  OmPre<G, NB> oml;
  if (!OMP && a.ext != nullptr) oml.load(a, kvh);
  const OmPre<G, NB>& omv = OMP ? omp : oml;

  // query fragments (row l16 = head) and the heads' DI-Exp constants
  v4i qa0 = v4i{0, 0, 0, 0}, qa1 = v4i{0, 0, 0, 0};
  if (l16 < G) {
    qa0 = *(const v4i*)(qsrc + l16 * 128 + grp * 16);
    qa1 = *(const v4i*)(qsrc + l16 * 128 + 64 + grp * 16);
  }
  // per head: the fp64-estimate DI-Exp (intops.h dexp_est) when tpos < 2^23
  // (every score difference is below 2^22: |q8 . k8| <= 2^21), else the
  // integer form
  // (the fused kernel's constants are written during the score pass and
  // read after the maxima's barrier)
  i64 tph[G];
  if (!PRE) {
#pragma unroll
    for (int hh = 0; hh < G; ++hh) tph[hh] = tsrc[hh];
  }

  // ---- pass 1: scores on MFMA; masked slots marked; per-head row max.
  // Lane (grp, l16) holds C[4 grp + r][slot l16] in element r.
  int32_t mx[4] = {SCORE_MASKED, SCORE_MASKED, SCORE_MASKED, SCORE_MASKED};
  const int nblk = (S + 15) / 16;
  // blocks blk0 + NW u (u < 4) from K fragments kb and validity flags vf
  auto score4 = [&](int blk0, const v4i (&kb)[4][2], const int (&vf)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int blk = blk0 + u * NW;
      if (blk < nblk) {  // wave-uniform
        v4i c = mfma16(qa0, kb[u][0], v4i{0, 0, 0, 0});
        c = mfma16(qa1, kb[u][1], c);
        const int s = blk * 16 + l16;
        const bool vis = s < S && vf[u] != 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int hh = grp * 4 + r;
          if (hh < G) {
            if (s < S) sc[hh * Spad + s] = vis ? c[r] : SCORE_MASKED;
            if (vis) mx[r] = ::max(mx[r], c[r]);
          }
        }
      }
    }
  };
  int blk0 = wave;
  if (PRE) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int bb = wave + 4 * NW * it;
      if (bb >= nblk) continue;  // wave-uniform
      v4i kb[4][2];
      int vf[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        kb[u][0] = pre.kb[it][u][0];
        kb[u][1] = pre.kb[it][u][1];
        if ((bb + u * NW) * 16 + l16 == pre.new_slot) {
          kb[u][0] = *(const v4i*)(pre.k_new + grp * 16);
          kb[u][1] = *(const v4i*)(pre.k_new + 64 + grp * 16);
        }
        vf[u] = pre.vf[it][u];
      }
      score4(bb, kb, vf);
    }
    blk0 = wave + 4 * NW * IT;
  }
  for (; blk0 < nblk; blk0 += 4 * NW) {
    v4i kb[4][2];
    int vraw[4], vf[4];
    bool ok[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int s = (blk0 + u * NW) * 16 + l16;
      const int sc_ = s < S ? s : 0;
      const int8_t* kr = a.kv.krow(pg_of(sc_), kvh, sc_ & (DI_PAGE - 1));
      kb[u][0] = *(const v4i*)(kr + grp * 16);
      kb[u][1] = *(const v4i*)(kr + 64 + grp * 16);
      vraw[u] = vrow[sc_];  // loaded unconditionally, masked at use (no wait per block)
      ok[u] = pg_lds[sc_ >> 7] >= 0;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) vf[u] = ok[u] ? vraw[u] : 0;
    score4(blk0, kb, vf);
  }
  // the first VP steps of V, loaded now (the K fragments' registers are
  // free) to overlap the maxima, denominators and probabilities
  v4i vpre[VP][NB];
#pragma unroll
  for (int i = 0; i < VP; ++i)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      vpre[i][nb] = (PRE && i * 64 < KPRE_SLOTS) ? vfrag_pre(i, nb) : vfrag(i, nb);
  // per-head row maxima, two heads per block reduction (int32 scores biased
  // to order-preserving unsigned values)
  i64 hmax[G];
#pragma unroll
  for (int r = 0; r < 4; ++r) mx[r] = row16_max(mx[r]);
#pragma unroll
  for (int hh = 0; hh < G; hh += 2) {
    // head hh lives in lanes 16 (hh / 4) .. + 15, element hh % 4
    const int32_t m0 = grp == hh / 4 ? mx[hh % 4] : SCORE_MASKED;
    const int32_t m1 = hh + 1 < G && grp == (hh + 1) / 4 ? mx[(hh + 1) % 4] : SCORE_MASKED;
    uint32_t u0 = (uint32_t)m0 ^ 0x80000000u, u1 = (uint32_t)m1 ^ 0x80000000u;
    red.max2_u32(u0, u1);
    const int32_t r0 = (int32_t)(u0 ^ 0x80000000u), r1 = (int32_t)(u1 ^ 0x80000000u);
    hmax[hh] = r0 == SCORE_MASKED ? 0 : r0;  // no visible slot: max := 0, every p = 0
    if (hh + 1 < G) hmax[hh + 1] = r1 == SCORE_MASKED ? 0 : r1;
  }
  __syncthreads();
  if (PRE) {
#pragma unroll
    for (int hh = 0; hh < G; ++hh) tph[hh] = tsrc[hh];
  }
  // ---- pass 2: denominators (two heads per block reduction). When every
  // head takes the estimate path (the usual case), one loop serves all heads
  // and two slots per thread, the LDS reads of an iteration issued together.
  i64 den[G];
  bool allfast = true;
#pragma unroll
  for (int hh = 0; hh < G; ++hh) allfast = allfast && tph[hh] < ((i64)1 << 23);
  ExpEst Ef[G];
  if (DI_LIKELY(allfast)) {
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      Ef[hh] = make_expest(tph[hh]);
      den[hh] = 0;
    }
    for (int s0 = tid; s0 < S; s0 += 2 * NT) {
      const int s1 = s0 + NT;
      const int s1c = s1 < S ? s1 : s0;
      int32_t x0[G], x1[G];
#pragma unroll
      for (int hh = 0; hh < G; ++hh) {
        x0[hh] = sc[hh * Spad + s0];
        x1[hh] = sc[hh * Spad + s1c];
      }
#pragma unroll
      for (int hh = 0; hh < G; ++hh) {
        if (x0[hh] != SCORE_MASKED) den[hh] += dexp_est((uint32_t)(hmax[hh] - x0[hh]), Ef[hh]);
        if (s1 < S && x1[hh] != SCORE_MASKED)
          den[hh] += dexp_est((uint32_t)(hmax[hh] - x1[hh]), Ef[hh]);
      }
    }
  } else {
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    i64 acc = 0;
    if (tph[hh] < ((i64)1 << 23)) {
      const ExpEst Ee = make_expest(tph[hh]);
      for (int s = tid; s < S; s += NT) {
        const int32_t x = sc[hh * Spad + s];
        if (x != SCORE_MASKED) acc += dexp_est((uint32_t)(hmax[hh] - x), Ee);
      }
    } else {
      const ExpR E = make_exp(tph[hh]);
      for (int s = tid; s < S; s += NT) {
        const int32_t x = sc[hh * Spad + s];
        if (x != SCORE_MASKED) acc = wadd(acc, di_exp_neg((u64)wsub(hmax[hh], (i64)x), E));
      }
    }
    den[hh] = acc;
  }
  }
#pragma unroll
  for (int hh = 0; hh < G; hh += 2) {
    i64 d1 = hh + 1 < G ? den[hh + 1] : 0;
    red.sum2(den[hh], d1);
    den[hh] = imax(den[hh], 1);
    if (hh + 1 < G) den[hh + 1] = imax(d1, 1);
  }
  // ---- pass 3: p in [0, 2^14] as (hi - 64) | lo << 8 in place of the score
  // (0 for masked slots and the padding up to the next multiple of 16, i.e.
  // hi - 64 = -64, lo = 0)
  const int nchunk = (S + 15) / 16;
  bool pfast = allfast;
#pragma unroll
  for (int hh = 0; hh < G; ++hh) pfast = pfast && den[hh] < ((i64)1 << 34);
  if (DI_LIKELY(pfast)) {
    // as pass 2: every head, two slots per thread, reads first
    DivEst Df[G];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) Df[hh] = make_divest(den[hh], 16384.0);
    const int lim = nchunk * 16;
    for (int s0 = tid; s0 < lim; s0 += 2 * NT) {
      const int s1 = s0 + NT;
      const int s1c = s1 < lim ? s1 : s0;
      int32_t x0[G], x1[G];
#pragma unroll
      for (int hh = 0; hh < G; ++hh) {
        x0[hh] = sc[hh * Spad + s0];
        x1[hh] = sc[hh * Spad + s1c];
      }
#pragma unroll
      for (int hh = 0; hh < G; ++hh) {
        i64 p0 = 0, p1 = 0;
        if (s0 < S && x0[hh] != SCORE_MASKED)
          p0 = rhad_est((double)dexp_est((uint32_t)(hmax[hh] - x0[hh]), Ef[hh]), Df[hh]);
        if (s1 < S && x1[hh] != SCORE_MASKED)
          p1 = rhad_est((double)dexp_est((uint32_t)(hmax[hh] - x1[hh]), Ef[hh]), Df[hh]);
        sc[hh * Spad + s0] = pack_p(p0);
        if (s1 < lim) sc[hh * Spad + s1] = pack_p(p1);
      }
    }
  } else {
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    auto put = [&](int s, i64 p) { sc[hh * Spad + s] = pack_p(p); };
    if (tph[hh] < ((i64)1 << 23) && den[hh] < ((i64)1 << 34)) {
      // exps below 2^23, den < 2^34: p = rhad(ex 2^14, den) from rhad_est
      const ExpEst Ee = make_expest(tph[hh]);
      const DivEst D = make_divest(den[hh], 16384.0);
      for (int s = tid; s < nchunk * 16; s += NT) {
        i64 p = 0;
        if (s < S) {
          const int32_t x = sc[hh * Spad + s];
          if (x != SCORE_MASKED) p = rhad_est((double)dexp_est((uint32_t)(hmax[hh] - x), Ee), D);
        }
        put(s, p);
      }
    } else {
      const ExpR E = make_exp(tph[hh]);
      const Recip Rd = make_recip(den[hh]);
      for (int s = tid; s < nchunk * 16; s += NT) {
        i64 p = 0;
        if (s < S) {
          const int32_t x = sc[hh * Spad + s];
          if (x != SCORE_MASKED) {
            const i64 ex = di_exp_neg((u64)wsub(hmax[hh], (i64)x), E);
            p = to_i32(rhad_r(shl(ex, 14), Rd));
          }
        }
        put(s, p);
      }
    }
  }
  }
  __syncthreads();
  // ---- P.V on MFMA
  v4i chi[NB], clo[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) chi[nb] = clo[nb] = v4i{0, 0, 0, 0};
  auto pv_step = [&](int st, const v4i (&vb)[NB]) {
    v4i ahi = v4i{0, 0, 0, 0}, alo = v4i{0, 0, 0, 0};
    const int s0 = st * 64 + grp * 16;
    if (l16 < G && s0 < S) {
      p_frags(sc + l16 * Spad + s0, ahi, alo);  // 16 packed p of head l16
    } else if (l16 == G && s0 < S) {
      ahi = v4i{0x01010101, 0x01010101, 0x01010101, 0x01010101};  // colsum row
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      chi[nb] = mfma16(ahi, vb[nb], chi[nb]);
      clo[nb] = mfma16(alo, vb[nb], clo[nb]);
    }
  };
#pragma unroll
  for (int i = 0; i < VP; ++i)
    if (i < nstep) pv_step(i, vpre[i]);
  for (int st0 = VP; st0 < nstep; st0 += 4) {
    v4i vb[4][NB];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) vb[i][nb] = vfrag(st0 + i, nb);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (st0 + i < nstep) pv_step(st0 + i, vb[i]);
  }
  if (a.ext == nullptr) {
    store_pv<G, NB>(chi, clo, a.out + (i64)b * a.n_q * 128 + kvh * G * 128);
    return;
  }
  // with the merge's row statistics of the block's outputs (0 included, as
  // merge_rowcol_row starts its extremes from 0)
  i64 vmx = 0, nmn = -1;
  store_pv<G, NB>(chi, clo, a.out + (i64)b * a.n_q * 128 + kvh * G * 128,
                  [&](int nb, int r, i64 o) {
                    const i64 v = wmul(o, omv.v[nb][r < RG ? r : 0]);
                    vmx = imax(vmx, v);
                    nmn = imax(nmn, ~v);
                  });
  red.max2(vmx, nmn);
  if (tid == 0) {
    a.ext[((i64)b * a.n_kv + kvh) * 2] = vmx;
    a.ext[((i64)b * a.n_kv + kvh) * 2 + 1] = nmn;
  }
}

template <int G, bool SCR>
__global__ __launch_bounds__(256) void k_attn_decode(DecodeArgs a) {
  keep_hidden_args();
  extern __shared__ __attribute__((aligned(16))) int32_t sh_scores[];
  __shared__ int32_t pg_lds[DEC_MAX_PAGES];
  const int kvh = blockIdx.x, b = blockIdx.y;
  const i64 q0 = (i64)b * a.n_q + kvh * G;
  bool over;
  const int S = scanned_slots(a, a.tpos, &over);
  const int npages = (a.S + DI_PAGE - 1) / DI_PAGE;
  for (int i = threadIdx.x; i < npages; i += 256) pg_lds[i] = a.kv.page(b, (i64)i * DI_PAGE);
  if (npages == 0 && threadIdx.x == 0) pg_lds[0] = -1;  // S = 0: loads read page 0
  __syncthreads();
  decode_body<G, VPRE, SCR>(a, S, kvh, b, a.q8 + q0 * 128, a.tpos + q0, sh_scores, pg_lds);
  report_slots(a, over, kvh == 0);
}

// Decode step with the Q/K/V epilogue fused in (G <= 2): waves 0..G-1 finish
// the block's query heads into LDS, wave G writes the key head and wave G + 1
// the value head of this step's slot into the cache (the other waves only
// prefetch); after one barrier the block's QAD_WAVES waves attend over every
// slot, the new one included (two waves per SIMD, each with half the slots
// and channels of a four-wave block). NS1: the Q/K/V product has no K split
// (qa.nsplit == 1). SCR as in decode_body.
constexpr int QAD_WAVES = 8;
template <int G, bool NS1, bool SCR>
__global__ __launch_bounds__(QAD_WAVES * 64) void k_qkv_attn_decode(DecodeArgs a, QKVArgs qa) {
  keep_hidden_args();
  constexpr int NW = QAD_WAVES, NT = NW * 64, IT = 8 / NW;
  static_assert(G + 2 <= NW, "one wave per head slot");
  extern __shared__ __attribute__((aligned(16))) int32_t sh_scores[];
  __shared__ __attribute__((aligned(16))) int8_t q_lds[G][128];
  __shared__ int64_t t_lds[G];
  __shared__ int64_t am_lds[G];
  const int kvh = blockIdx.x, b = blockIdx.y;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // wave-uniform
  // (kernel arguments pass through opaque_* below: the optimizer would
  // otherwise fold selects between them into loads from selected argument
  // addresses, each behind its own wait)
  const int n_q = opaque_i32(qa.n_q), n_kv = opaque_i32(qa.n_kv);
  const int slotw = w < G ? kvh * G + w : w == G ? n_q + kvh : w == G + 1 ? n_q + n_kv + kvh : -1;
  __shared__ __attribute__((aligned(16))) int8_t k_new[128];
  __shared__ int32_t pg_lds[DEC_MAX_PAGES];
  const int lane = threadIdx.x & 63, l16 = lane & 15, grp = lane >> 4;
  constexpr int NPK = KPRE_SLOTS / DI_PAGE;
  // 1. loads whose addresses follow from the kernel arguments alone. The
  // block's scalars come from one vector load (lane i reads word i) and the
  // pages of the prefetched slots from another, instead of a chain of scalar
  // loads (a scalar-load wait covers every scalar load in flight).
  //   word 0 position, 1 xk, 2 xm, 3 the step's slot (device scalar), 4 the
  //   scanned-slot bound (device scalar), 5-8 vq_m, vq_k, ks_m, ks_k of the
  //   kv head; other lanes (and absent device scalars) read the position
  const int64_t* const pos_p = opaque_ptr(qa.positions) + b;
  const int64_t* const sb_p = opaque_ptr(qa.slot_base_dev);
  const int64_t* const sd_p = opaque_ptr(a.s_dev);
  const int64_t* const xk_p = opaque_ptr(qa.xk) + b;
  const int64_t* const xm_p = opaque_ptr(qa.xm) + b;
  const int64_t* const vqm_p = opaque_ptr(qa.vq_m) + kvh;
  const int64_t* const vqk_p = opaque_ptr(qa.vq_k) + kvh;
  const int64_t* const ksm_p = opaque_ptr(qa.ks_m) + kvh;
  const int64_t* const ksk_p = opaque_ptr(qa.ks_k) + kvh;
  const int64_t* wq = pos_p;
  wq = lane == 1 ? xk_p : wq;
  wq = lane == 2 ? xm_p : wq;
  wq = lane == 3 && sb_p ? sb_p : wq;
  wq = lane == 4 && sd_p ? sd_p : wq;
  wq = lane == 5 ? vqm_p : wq;
  wq = lane == 6 ? vqk_p : wq;
  wq = lane == 7 ? ksm_p : wq;
  wq = lane == 8 ? ksk_p : wq;
  const i64 word = ld_global(wq);
  // page j of the row for lanes j < NPK with slots below a.S (<= width * 128,
  // so j < width), else page 0's entry (masked below)
  const bool pk_ok = lane < NPK && lane * DI_PAGE < a.S;
  const int32_t pword = a.kv.table[(i64)b * a.kv.width + (pk_ok ? lane : 0)];
  // the row's page ids (stored to LDS after the epilogue)
  // (npages <= width: each load is in bounds, the ones past npages masked)
  const int npages = (a.S + DI_PAGE - 1) / DI_PAGE;
  int pgv[DEC_MAX_PAGES / NT];
#pragma unroll
  for (int q = 0; q < DEC_MAX_PAGES / NT; ++q) {
    const int i = (int)threadIdx.x + NT * q;
    pgv[q] = a.kv.table[(i64)b * a.kv.width + (i < npages ? i : 0)];
  }
  // the head slot's per-channel loads (unconditional: a wave without a head
  // slot loads slot 0's and ignores them, so no branch merge forces the loads
  // to complete early)
  const int slotl = slotw >= 0 ? slotw : 0;
  QKVHeadIn in = qkv_head_load<NS1>(qa, b, slotl, QKVScalars{});
  // the merge factors of this wave's outputs (for the row statistics)
  OmPre<G, 8 / NW> omp;
  if (a.ext != nullptr) omp.load(a, kvh);
  // (every load above is issued before the wait for the gathered scalars)
  __builtin_amdgcn_sched_barrier(0);
  in.pos_raw = readlane64(word, 0);
  in.xk = readlane64(word, 1);
  in.xm = readlane64(word, 2);
  in.base = sb_p ? readlane64(word, 3) : qa.slot_base;
  in.vqm = readlane64(word, 5);
  in.vqk = readlane64(word, 6);
  in.ksm = readlane64(word, 7);
  in.ksk = readlane64(word, 8);
  const i64 sdev = readlane64(word, 4);
  const bool over = sd_p != nullptr && sdev > (i64)a.S;
  const int S = sd_p ? (int)imax(0, imin((i64)a.S, sdev)) : a.S;
  const i64 base = in.base;
  qkv_head_rope_load(qa, slotl, in);  // waits for the position only
  // 2. the loads that depend on those: this wave's K rows of the scores
  // pass's first iterations (the pass masks slots at or past the scanned
  // count and slots of pages that are not mapped)
  int pgk[NPK];
#pragma unroll
  for (int j = 0; j < NPK; ++j)
    pgk[j] = j * DI_PAGE < a.S ? __builtin_amdgcn_readlane(pword, j) : -1;
  KPre<IT> pre;
  int vraw[IT][4];
  bool vok[IT][4];
  {
    const uint8_t* vrow = a.valid + (i64)b * a.valid_stride;
#pragma unroll
    for (int it = 0; it < IT; ++it)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int s = (w + 4 * NW * it + u * NW) * 16 + l16;  // < KPRE_SLOTS
        // slots at or past the scanned count read slot 0 (one cached line
        // instead of rows nobody scores; the pass masks them)
        const int sc_ = s < S ? s : 0;
        const int j = sc_ >> 7;
        int pg = pgk[0];
#pragma unroll
        for (int jj = 1; jj < NPK; ++jj) pg = j == jj ? pgk[jj] : pg;
        const int8_t* kr = a.kv.krow(pg < 0 ? 0 : pg, kvh, sc_ & (DI_PAGE - 1));
        pre.kb[it][u][0] = *(const v4i*)(kr + grp * 16);
        pre.kb[it][u][1] = *(const v4i*)(kr + 64 + grp * 16);
        vraw[it][u] = vrow[sc_];  // masked after the epilogue: no wait here
        vok[it][u] = pg >= 0;
      }
    pre.k_new = k_new;
#pragma unroll
    for (int j = 0; j < NPK; ++j) pre.pg[j] = pgk[j];
  }
  // 3. the epilogue
  if (slotw >= 0)
    qkv_head_compute(qa, b, slotw, in, w < G ? q_lds[w] : nullptr, nullptr,
                     w == G ? k_new : nullptr, w < G ? &am_lds[w] : nullptr);
  if (slotw >= 0) qkv_head_report(qa, slotw, in);
#pragma unroll
  for (int it = 0; it < IT; ++it)
#pragma unroll
    for (int u = 0; u < 4; ++u) pre.vf[it][u] = vok[it][u] ? vraw[it][u] : 0;
  // T = 1: the step's slot is base (when its page is not mapped nothing was
  // written, and the slot is masked: the substituted row is never a score)
  pre.new_slot = base;
#pragma unroll
  for (int q = 0; q < DEC_MAX_PAGES / NT; ++q) {
    const int i = (int)threadIdx.x + NT * q;
    if (i < npages) pg_lds[i] = pgv[q];  // (loaded unconditionally above)
  }
  __syncthreads();
  // the query heads' DI-Exp constants (one lane's serial chain per head) on
  // the last wave, while the others start the scores; decode_body reads
  // them after its maxima's barrier
  if (w == NW - 1 && lane < G)
    t_lds[lane] = q_head_tpos(qa, am_lds[lane], in.ksm, in.ksk, nullptr);
  decode_body<G, VPRE_FUSED, SCR, true, NW, true>(a, S, kvh, b, &q_lds[0][0], t_lds, sh_scores,
                                                  pg_lds, pre, omp);
  report_slots(a, over, kvh == 0);
}

// ---------------------------------------------------------------------------
// Split-S decode attention: the slots of a (row, kv head) are cut into chunks
// of `chunk` slots (a multiple of the page), one block per chunk, in two
// launches:
//   k_attn_split_scores: the chunk's scores (int32, to a global scratch) and
//     its per-head maximum over visible slots;
//   k_attn_split_pv: the row maximum (the maximum of the chunk maxima — the
//     TRUE row max, DI-Exp being not multiplicative), the denominator over
//     ALL the row's slots (every block sums the same integers, so every block
//     holds the same den), then p of the chunk's slots and their P.V into the
//     chunk's own int64 partial context.
// The context is the sum of the partials (exact integer addition, in any
// order); the attention-output merge sums them. Same integers as
// k_attn_decode for every chunking.

constexpr int SPLIT_MAX_CHUNK = 4096;                  // slots per chunk
constexpr int SPLIT_MAX_PAGES = SPLIT_MAX_CHUNK / DI_PAGE;

struct SplitArgs {
  DecodeArgs d;     // scratch: scores [B][n_q][spad]; out: partials [ns][B][n_q * 128]
  int32_t* cmax;    // [B][n_q][ns] chunk maxima (SCORE_MASKED: no visible slot)
  int chunk, ns;
  i64 spad;         // row stride of the scores (>= S)
  i64 out_stride;   // elements between partials (B * n_q * 128)
};

template <int G>
__global__ __launch_bounds__(256) void k_attn_split_scores(SplitArgs sa) {
  keep_hidden_args();
  const DecodeArgs& a = sa.d;
  __shared__ i64 red_buf[32];
  __shared__ int32_t pg_lds[SPLIT_MAX_PAGES];
  BlockRedT<4> red{red_buf, 0, 256};
  const int kvh = blockIdx.x, b = blockIdx.y, c = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l16 = lane & 15, grp = lane >> 4;
  bool over;
  const int S = scanned_slots(a, a.tpos, &over);
  report_slots(a, over, kvh == 0 && c == 0);  // every later load depends on S anyway
  const int lo = c * sa.chunk, hi = ::min(lo + sa.chunk, S);
  const i64 q0 = (i64)b * a.n_q + kvh * G;
  int32_t* cm = sa.cmax + q0 * sa.ns + c;  // head hh at cm[hh * ns]
  if (lo >= hi) {  // block-uniform: a chunk past the scanned slots
    if (tid < G) cm[tid * sa.ns] = SCORE_MASKED;
    return;
  }
  const int npg = (hi - lo + DI_PAGE - 1) / DI_PAGE;
  if (tid < npg) pg_lds[tid] = a.kv.page(b, (i64)lo + (i64)tid * DI_PAGE);
  v4i qa0 = v4i{0, 0, 0, 0}, qa1 = v4i{0, 0, 0, 0};
  if (l16 < G) {
    const int8_t* qsrc = a.q8 + q0 * 128;
    qa0 = *(const v4i*)(qsrc + l16 * 128 + grp * 16);
    qa1 = *(const v4i*)(qsrc + l16 * 128 + 64 + grp * 16);
  }
  __syncthreads();
  int32_t* sc = a.scratch + q0 * sa.spad;
  const uint8_t* vrow = a.valid + (i64)b * a.valid_stride;
  int32_t mx[4] = {SCORE_MASKED, SCORE_MASKED, SCORE_MASKED, SCORE_MASKED};
  const int blo = lo / 16, bhi = (hi + 15) / 16;
  for (int blk0 = blo + wave; blk0 < bhi; blk0 += 16) {
    v4i kb[4][2];
    int vraw[4], vf[4];
    bool ok[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int s = (blk0 + u * 4) * 16 + l16;
      const int sc_ = s < hi ? s : lo;
      const int pg = pg_lds[(sc_ - lo) / DI_PAGE];
      const int8_t* kr = a.kv.krow(pg < 0 ? 0 : pg, kvh, sc_ & (DI_PAGE - 1));
      kb[u][0] = *(const v4i*)(kr + grp * 16);
      kb[u][1] = *(const v4i*)(kr + 64 + grp * 16);
      vraw[u] = vrow[sc_];  // masked at use (no wait per block)
      ok[u] = pg >= 0;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) vf[u] = ok[u] ? vraw[u] : 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int blk = blk0 + u * 4;
      if (blk < bhi) {  // wave-uniform
        v4i cc = mfma16(qa0, kb[u][0], v4i{0, 0, 0, 0});
        cc = mfma16(qa1, kb[u][1], cc);
        const int s = blk * 16 + l16;
        const bool vis = s < hi && vf[u] != 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int hh = grp * 4 + r;
          if (hh < G) {
            if (s < hi) sc[hh * sa.spad + s] = vis ? cc[r] : SCORE_MASKED;
            if (vis) mx[r] = ::max(mx[r], cc[r]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) mx[r] = row16_max(mx[r]);
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    const int32_t mine = grp == hh / 4 ? mx[hh % 4] : SCORE_MASKED;
    const i64 m = red.max((i64)mine);
    if (tid == 0) cm[hh * sa.ns] = (int32_t)m;
  }
}

template <int G>
__global__ __launch_bounds__(256) void k_attn_split_pv(SplitArgs sa) {
  keep_hidden_args();
  const DecodeArgs& a = sa.d;
  extern __shared__ __attribute__((aligned(16))) int32_t p_lds[];  // [G][chunk] packed p
  __shared__ i64 red_buf[32];
  __shared__ int32_t pg_lds[SPLIT_MAX_PAGES];
  BlockRedT<4> red{red_buf, 0, 256};
  const int kvh = blockIdx.x, b = blockIdx.y, c = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l16 = lane & 15, grp = lane >> 4;
  bool over;
  const int S = scanned_slots(a, a.tpos, &over);
  const int lo = c * sa.chunk, hi = ::min(lo + sa.chunk, S);
  const i64 q0 = (i64)b * a.n_q + kvh * G;
  int64_t* outp = a.out + c * sa.out_stride + q0 * 128;
  if (lo >= hi) {  // block-uniform: this chunk contributes nothing
    for (int i = tid; i < G * 128; i += 256) outp[i] = 0;
    return;
  }
  const int npg = (hi - lo + DI_PAGE - 1) / DI_PAGE;
  if (tid < npg) pg_lds[tid] = a.kv.page(b, (i64)lo + (i64)tid * DI_PAGE);
  i64 tph[G], hmax[G];
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    tph[hh] = a.tpos[q0 + hh];
    i64 m = SCORE_MASKED;
    const int32_t* cmh = sa.cmax + (q0 + hh) * sa.ns;
    for (int k = 0; k < sa.ns; ++k) m = imax(m, (i64)cmh[k]);
    hmax[hh] = m == (i64)SCORE_MASKED ? 0 : m;  // no visible slot: max := 0, every p = 0
  }
  __syncthreads();
  // V fragments of the chunk's first VPRE 64-slot steps (a step lies in one
  // page), loaded before the denominator pass
  auto vfrag = [&](int st, int nb) -> v4i {  // unconditional, as in decode_body
    const int s0 = st * 64 + grp * 16;
    const int sl = s0 < hi ? s0 : lo;
    const int pg = pg_lds[(sl - lo) / DI_PAGE];
    const int8_t* vch = a.kv.vchan(pg < 0 ? 0 : pg, kvh, wave * 32 + nb * 16 + l16);
    return *(const v4i*)(vch + (sl & (DI_PAGE - 1)));
  };
  const int st_lo = lo / 64, st_hi = (hi + 63) / 64;
  v4i vpre[VPRE][2];
#pragma unroll
  for (int i = 0; i < VPRE; ++i)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) vpre[i][nb] = vfrag(st_lo + i, nb);
  const int32_t* sc = a.scratch + q0 * sa.spad;
  // denominators over every scanned slot of the row
  i64 den[G];
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    i64 acc = 0;
    if (tph[hh] < ((i64)1 << 23)) {
      const ExpEst Ee = make_expest(tph[hh]);
      for (int s = tid; s < S; s += 256) {
        const int32_t x = sc[hh * sa.spad + s];
        if (x != SCORE_MASKED) acc += dexp_est((uint32_t)(hmax[hh] - x), Ee);
      }
    } else {
      const ExpR E = make_exp(tph[hh]);
      for (int s = tid; s < S; s += 256) {
        const int32_t x = sc[hh * sa.spad + s];
        if (x != SCORE_MASKED) acc = wadd(acc, di_exp_neg((u64)wsub(hmax[hh], (i64)x), E));
      }
    }
    den[hh] = imax(red.sum(acc), 1);
  }
  // p of the chunk's slots, packed into LDS (0 for masked slots and the
  // padding to the next multiple of 16)
  const int n16 = (hi - lo + 15) / 16 * 16;
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    int32_t* ph = p_lds + hh * sa.chunk;
    if (tph[hh] < ((i64)1 << 23) && den[hh] < ((i64)1 << 34)) {
      const ExpEst Ee = make_expest(tph[hh]);
      const DivEst D = make_divest(den[hh], 16384.0);
      for (int i = tid; i < n16; i += 256) {
        i64 p = 0;
        if (lo + i < hi) {
          const int32_t x = sc[hh * sa.spad + lo + i];
          if (x != SCORE_MASKED) p = rhad_est((double)dexp_est((uint32_t)(hmax[hh] - x), Ee), D);
        }
        ph[i] = pack_p(p);
      }
    } else {
      const ExpR E = make_exp(tph[hh]);
      const Recip Rd = make_recip(den[hh]);
      for (int i = tid; i < n16; i += 256) {
        i64 p = 0;
        if (lo + i < hi) {
          const int32_t x = sc[hh * sa.spad + lo + i];
          if (x != SCORE_MASKED) {
            const i64 ex = di_exp_neg((u64)wsub(hmax[hh], (i64)x), E);
            p = to_i32(rhad_r(shl(ex, 14), Rd));
          }
        }
        ph[i] = pack_p(p);
      }
    }
  }
  __syncthreads();
  // P.V of the chunk
  v4i chi[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}}, clo[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
  auto pv_step = [&](int st, const v4i (&vb)[2]) {
    v4i ahi = v4i{0, 0, 0, 0}, alo = v4i{0, 0, 0, 0};
    const int s0 = st * 64 + grp * 16;
    if (l16 < G && s0 < hi) {
      p_frags(p_lds + l16 * sa.chunk + (s0 - lo), ahi, alo);
    } else if (l16 == G && s0 < hi) {
      ahi = v4i{0x01010101, 0x01010101, 0x01010101, 0x01010101};  // colsum row
    }
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      chi[nb] = mfma16(ahi, vb[nb], chi[nb]);
      clo[nb] = mfma16(alo, vb[nb], clo[nb]);
    }
  };
#pragma unroll
  for (int i = 0; i < VPRE; ++i)
    if (st_lo + i < st_hi) pv_step(st_lo + i, vpre[i]);
  for (int st0 = st_lo + VPRE; st0 < st_hi; st0 += 4) {
    v4i vb[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) vb[i][nb] = vfrag(st0 + i, nb);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (st0 + i < st_hi) pv_step(st0 + i, vb[i]);
  }
  store_pv<G>(chi, clo, outp);
}

}  // namespace

extern "C" {

// The paged cache arguments of every entry below: kpool / vpool the layer's
// page pools (common.h KVPages), table [B][width] int32 page ids (-1: not
// mapped); a row holds width * 128 slots.
static bool kv_ok(const int8_t* kpool, const int8_t* vpool, const int32_t* table, int width) {
  return kpool && vpool && table && width > 0 && width <= (1 << 24);
}

int detllm_attn_prefill(const int8_t* q8, const int64_t* tpos, const int8_t* kpool,
                        const int8_t* vpool, const int32_t* table, int width,
                        const uint8_t* valid, int64_t valid_stride, int B, int T, int S_past,
                        int n_q, int n_kv, int64_t* out, hipStream_t s) {
  if (B <= 0 || T <= 0) return DI_OK;
  const i64 S = (i64)S_past + T;
  if (n_q <= 0 || n_kv <= 0 || n_q % n_kv || S_past < 0 || !kv_ok(kpool, vpool, table, width) ||
      S > (i64)width * DI_PAGE || valid_stride < S || !q8 || !tpos || !valid || !out)
    return DI_EINVAL;
  if (S > 131071) return DI_ERANGE;  // int32 MFMA accumulators of P.V
  PrefillArgs a{q8, tpos, KVPages{(int8_t*)kpool, (int8_t*)vpool, table, width, n_kv}, valid, out,
                T, (int)S, S_past, n_q, n_kv, B, valid_stride};
  const i64 pairs = (i64)(((T + 63) / 64 + 1) / 2) * n_q * B;
  if (2 * pairs > 0x7fffffff) return DI_ERANGE;
  // column sums, tile masks, page ids
  const size_t lds = PF_CSUM + 8 * (size_t)((S + 63) / 64) + 4 * (size_t)((S + 127) / 128);
  hipLaunchKernelGGL(k_attn_prefill, dim3((unsigned)(2 * pairs)), dim3(256), lds, s, a);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

// Decode (one query per batch row). S: slots to scan (<= width * 128);
// s_dev: optional device scalar that further bounds it (graph replay).
// scratch may be null when n_q/n_kv * ceil16(S) * 4 bytes fit in 48 KiB of LDS.
int detllm_attn_decode(const int8_t* q8, const int64_t* tpos, const int8_t* kpool,
                       const int8_t* vpool, const int32_t* table, int width,
                       const uint8_t* valid, int64_t valid_stride, int B, int S, int n_q, int n_kv,
                       const int64_t* s_dev, int32_t* scratch, int64_t* out, int32_t* err,
                       hipStream_t s) {
  if (B <= 0) return DI_OK;
  if (n_q <= 0 || n_kv <= 0 || n_q % n_kv || S < 0 || !kv_ok(kpool, vpool, table, width) ||
      S > (i64)width * DI_PAGE || valid_stride < S || !q8 || !tpos || !valid || !out)
    return DI_EINVAL;
  const int G = n_q / n_kv;
  if (G > MAXG) return DI_ENOSYS;
  if (S > DEC_MAX_S) return DI_ERANGE;  // int32 MFMA accumulators of P.V
  const i64 Spad = ((i64)S + 15) & ~15;
  const i64 lds = (i64)G * Spad * 4;
  size_t dyn = 0;
  if (lds <= DECODE_LDS_BYTES) {
    dyn = (size_t)lds;
    scratch = nullptr;
  } else if (!scratch) {
    return DI_ERANGE;
  }
  DecodeArgs a{q8, tpos, KVPages{(int8_t*)kpool, (int8_t*)vpool, table, width, n_kv}, valid, out,
               scratch, s_dev, S, n_q, n_kv, valid_stride, err};
  const dim3 grid(n_kv, B);
  switch (G) {
#define DI_DEC_LAUNCH(G_)                                                                      \
  if (scratch) hipLaunchKernelGGL((k_attn_decode<G_, true>), grid, dim3(256), dyn, s, a);    \
  else hipLaunchKernelGGL((k_attn_decode<G_, false>), grid, dim3(256), dyn, s, a)
    case 1: DI_DEC_LAUNCH(1); break;
    case 2: DI_DEC_LAUNCH(2); break;
    case 4: DI_DEC_LAUNCH(4); break;
    case 8: DI_DEC_LAUNCH(8); break;
#undef DI_DEC_LAUNCH
    default: return DI_ENOSYS;
  }
  DI_LAUNCH_CHECK();
  return DI_OK;
}

// Fused decode step for one query token per row: the Q/K/V epilogue of
// detllm_qkv_epilogue (T = 1) followed by detllm_attn_decode, one launch.
static int qkv_attn_decode_launch(const int32_t* P, int nsplit, int64_t split_stride, int B, int n_q,
                           int n_kv, const int64_t* xm, const int64_t* xk,
                           const int64_t* positions, const int64_t* q_m, int64_t q_k,
                           const int64_t* k_m, int64_t k_k, const int64_t* v_m, int64_t v_k,
                           const int64_t* q_norm_m, int64_t q_norm_k, const int64_t* k_norm_m,
                           int64_t k_norm_k, const int64_t* qs_m, int64_t qs_k,
                           const int64_t* kq_m, const int64_t* kq_k, const int64_t* ks_m,
                           const int64_t* ks_k, const int64_t* vq_m, const int64_t* vq_k,
                           const int16_t* cos_t, const int16_t* sin_t, int64_t max_pos,
                           int8_t* kpool, int8_t* vpool, const int32_t* table, int width,
                           const int64_t* slot_base_dev, int64_t slot_base,
                           const uint8_t* valid, int64_t valid_stride, int S,
                           const int64_t* s_dev, int32_t* scratch, int64_t* out, int32_t* err,
                           const int64_t* om, int64_t* ext, hipStream_t s) {
  if (B <= 0) return DI_OK;
  if (n_q <= 0 || n_kv <= 0 || n_q % n_kv || nsplit < 1 || S < 1 ||
      !kv_ok(kpool, vpool, table, width) || S > (i64)width * DI_PAGE || valid_stride < S ||
      max_pos <= 0 || !P || !positions || !out || !valid)
    return DI_EINVAL;
  if (S > DEC_MAX_S) return DI_ERANGE;  // int32 MFMA accumulators of P.V
  if (!slot_base_dev && (slot_base < 0 || slot_base + 1 > (i64)width * DI_PAGE)) return DI_ERANGE;
  const int G = n_q / n_kv;
  if (G > 2) return DI_ENOSYS;  // one wave per head slot of the block
  const i64 Spad = ((i64)S + 15) & ~15;
  const i64 lds = (i64)G * Spad * 4;
  size_t dyn = 0;
  if (lds <= DECODE_LDS_BYTES) {
    dyn = (size_t)lds;
    scratch = nullptr;
  } else if (!scratch) {
    return DI_ERANGE;
  }
  const KVPages kv{kpool, vpool, table, width, n_kv};
  QKVArgs qa{};
  qa.T = 1; qa.n_q = n_q; qa.n_kv = n_kv; qa.P = P; qa.nsplit = nsplit;
  qa.split_stride = split_stride; qa.xm = xm; qa.xk = xk; qa.positions = positions;
  qa.q_m = q_m; qa.k_m = k_m; qa.v_m = v_m; qa.q_k = q_k; qa.k_k = k_k; qa.v_k = v_k;
  qa.q_norm_m = q_norm_m; qa.k_norm_m = k_norm_m; qa.q_norm_k = q_norm_k;
  qa.k_norm_k = k_norm_k; qa.qs_m = qs_m; qa.qs_k = qs_k; qa.kq_m = kq_m; qa.kq_k = kq_k;
  qa.ks_m = ks_m; qa.ks_k = ks_k; qa.vq_m = vq_m; qa.vq_k = vq_k; qa.cos_t = cos_t;
  qa.sin_t = sin_t; qa.max_pos = max_pos; qa.q8 = nullptr; qa.tpos = nullptr; qa.dbg = nullptr;
  qa.kv = kv; qa.slot_base_dev = slot_base_dev; qa.slot_base = slot_base; qa.err = err;
  if ((om == nullptr) != (ext == nullptr)) return DI_EINVAL;
  DecodeArgs a{nullptr, nullptr, kv, valid, out, scratch, s_dev, S, n_q, n_kv, valid_stride, err,
               om, ext};
  const dim3 grid(n_kv, B);
#define DI_QAD_LAUNCH(G_, NS1_)                                                                 \
  if (scratch) hipLaunchKernelGGL((k_qkv_attn_decode<G_, NS1_, true>), grid, dim3(QAD_WAVES * 64), dyn, s, a, qa); \
  else hipLaunchKernelGGL((k_qkv_attn_decode<G_, NS1_, false>), grid, dim3(QAD_WAVES * 64), dyn, s, a, qa)
  if (G == 1) {
    if (nsplit == 1) { DI_QAD_LAUNCH(1, true); }
    else { DI_QAD_LAUNCH(1, false); }
  } else {
    if (nsplit == 1) { DI_QAD_LAUNCH(2, true); }
    else { DI_QAD_LAUNCH(2, false); }
  }
#undef DI_QAD_LAUNCH
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_qkv_attn_decode(const int32_t* P, int nsplit, int64_t split_stride, int B, int n_q,
                           int n_kv, const int64_t* xm, const int64_t* xk,
                           const int64_t* positions, const int64_t* q_m, int64_t q_k,
                           const int64_t* k_m, int64_t k_k, const int64_t* v_m, int64_t v_k,
                           const int64_t* q_norm_m, int64_t q_norm_k, const int64_t* k_norm_m,
                           int64_t k_norm_k, const int64_t* qs_m, int64_t qs_k,
                           const int64_t* kq_m, const int64_t* kq_k, const int64_t* ks_m,
                           const int64_t* ks_k, const int64_t* vq_m, const int64_t* vq_k,
                           const int16_t* cos_t, const int16_t* sin_t, int64_t max_pos,
                           int8_t* kpool, int8_t* vpool, const int32_t* table, int width,
                           const int64_t* slot_base_dev, int64_t slot_base,
                           const uint8_t* valid, int64_t valid_stride, int S,
                           const int64_t* s_dev, int32_t* scratch, int64_t* out, int32_t* err,
                           hipStream_t s) {
  return qkv_attn_decode_launch(
      P, nsplit, split_stride, B, n_q, n_kv, xm, xk, positions, q_m, q_k, k_m, k_k, v_m, v_k,
      q_norm_m, q_norm_k, k_norm_m, k_norm_k, qs_m, qs_k, kq_m, kq_k, ks_m, ks_k, vq_m, vq_k,
      cos_t, sin_t, max_pos, kpool, vpool, table, width, slot_base_dev, slot_base, valid,
      valid_stride, S, s_dev, scratch, out, err, nullptr, nullptr, s);
}

int detllm_qkv_attn_decode_ext(const int32_t* P, int nsplit, int64_t split_stride, int B, int n_q,
                           int n_kv, const int64_t* xm, const int64_t* xk,
                           const int64_t* positions, const int64_t* q_m, int64_t q_k,
                           const int64_t* k_m, int64_t k_k, const int64_t* v_m, int64_t v_k,
                           const int64_t* q_norm_m, int64_t q_norm_k, const int64_t* k_norm_m,
                           int64_t k_norm_k, const int64_t* qs_m, int64_t qs_k,
                           const int64_t* kq_m, const int64_t* kq_k, const int64_t* ks_m,
                           const int64_t* ks_k, const int64_t* vq_m, const int64_t* vq_k,
                           const int16_t* cos_t, const int16_t* sin_t, int64_t max_pos,
                           int8_t* kpool, int8_t* vpool, const int32_t* table, int width,
                           const int64_t* slot_base_dev, int64_t slot_base,
                           const uint8_t* valid, int64_t valid_stride, int S,
                           const int64_t* s_dev, int32_t* scratch, int64_t* out, int32_t* err,
                               const int64_t* om, int64_t* ext, hipStream_t s) {
  if (!om || !ext) return DI_EINVAL;
  return qkv_attn_decode_launch(
      P, nsplit, split_stride, B, n_q, n_kv, xm, xk, positions, q_m, q_k, k_m, k_k, v_m, v_k,
      q_norm_m, q_norm_k, k_norm_m, k_norm_k, qs_m, qs_k, kq_m, kq_k, ks_m, ks_k, vq_m, vq_k,
      cos_t, sin_t, max_pos, kpool, vpool, table, width, slot_base_dev, slot_base, valid,
      valid_stride, S, s_dev, scratch, out, err, om, ext, s);
}

// Chunking of the split-S decode attention: enough chunks that the launch has
// about 1024 blocks (four per CU; c4, 32 rows x 8 kv heads at 4096 slots:
// 3.88 ms per step at 1024-slot chunks against 4.41 at 512, 4.20 at 2048 —
// every block sums the whole row's denominator, so more chunks cost more),
// chunks of at least 256 slots, a multiple of the page, within the LDS of
// the packed p (G * chunk * 4 bytes <= 48 KiB) and SPLIT_MAX_CHUNK.
int detllm_attn_split_plan(int B, int S, int n_q, int n_kv, int* chunk, int* nsplit) {
  if (!chunk || !nsplit || B <= 0 || S <= 0 || n_q <= 0 || n_kv <= 0 || n_q % n_kv) return DI_EINVAL;
  const int G = n_q / n_kv;
  if (G > MAXG) return DI_ENOSYS;
  const i64 blocks = (i64)B * n_kv;
  const i64 want = blocks >= 1024 ? 1 : (1024 + blocks - 1) / blocks;
  i64 ch = ((i64)S + want - 1) / want;
  ch = (ch + DI_PAGE - 1) / DI_PAGE * DI_PAGE;
  i64 cmax = DECODE_LDS_BYTES / (4 * G) / DI_PAGE * DI_PAGE;
  if (cmax > SPLIT_MAX_CHUNK) cmax = SPLIT_MAX_CHUNK;
  ch = imax(imin(ch, cmax), (i64)2 * DI_PAGE);
  *chunk = (int)ch;
  *nsplit = (int)(((i64)S + ch - 1) / ch);
  return DI_OK;
}

// Split-S decode attention (one query token per row; q8, tpos as written by
// detllm_qkv_epilogue with T = 1). scores: int32 [B][n_q][nsplit * chunk];
// cmax: int32 [B][n_q][nsplit]; out: int64 partial contexts
// [nsplit][B][n_q * 128] whose sum is detllm_attn_decode's out.
int detllm_attn_decode_split(const int8_t* q8, const int64_t* tpos, const int8_t* kpool,
                             const int8_t* vpool, const int32_t* table, int width,
                             const uint8_t* valid, int64_t valid_stride, int B, int S, int n_q,
                             int n_kv, const int64_t* s_dev, int chunk, int32_t* scores,
                             int32_t* cmax, int64_t* out, int32_t* err, hipStream_t s) {
  if (B <= 0) return DI_OK;
  if (n_q <= 0 || n_kv <= 0 || n_q % n_kv || S < 1 || !kv_ok(kpool, vpool, table, width) ||
      S > (i64)width * DI_PAGE || valid_stride < S || !q8 || !tpos || !valid || !out || !scores ||
      !cmax || chunk < DI_PAGE || chunk % DI_PAGE || chunk > SPLIT_MAX_CHUNK)
    return DI_EINVAL;
  const int G = n_q / n_kv;
  if (G > MAXG) return DI_ENOSYS;
  if (S > DEC_MAX_S) return DI_ERANGE;  // int32 MFMA accumulators of P.V
  const i64 dyn = (i64)G * chunk * 4;
  if (dyn > DECODE_LDS_BYTES) return DI_ERANGE;
  const int ns = (S + chunk - 1) / chunk;
  SplitArgs sa{};
  sa.d = DecodeArgs{q8, tpos, KVPages{(int8_t*)kpool, (int8_t*)vpool, table, width, n_kv}, valid,
                    out, scores, s_dev, S, n_q, n_kv, valid_stride, err};
  sa.cmax = cmax;
  sa.chunk = chunk;
  sa.ns = ns;
  sa.spad = (i64)ns * chunk;
  sa.out_stride = (i64)B * n_q * 128;
  const dim3 grid(n_kv, B, ns);
#define DI_SPLIT_LAUNCH(G_)                                                                   \
  hipLaunchKernelGGL(k_attn_split_scores<G_>, grid, dim3(256), 0, s, sa);                     \
  hipLaunchKernelGGL(k_attn_split_pv<G_>, grid, dim3(256), (size_t)dyn, s, sa)
  switch (G) {
    case 1: DI_SPLIT_LAUNCH(1); break;
    case 2: DI_SPLIT_LAUNCH(2); break;
    case 4: DI_SPLIT_LAUNCH(4); break;
    case 8: DI_SPLIT_LAUNCH(8); break;
    default: return DI_ENOSYS;
  }
#undef DI_SPLIT_LAUNCH
  DI_LAUNCH_CHECK();
  return DI_OK;
}

}  // extern "C"
