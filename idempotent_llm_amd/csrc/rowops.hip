// Row kernels of the integer forward pass: per-row (per-token) reductions
// fused with the dyadic requantisations around them.
//
// A row of C <= 4096 values is held in registers by one 256-thread block:
// thread t owns columns t, t+256, ... (coalesced loads/stores); columns past C
// hold 0, which is neutral for every max|x| and sum. All arithmetic goes
// through intops.h, which reproduces the reference's torch-CPU semantics.
//
// Fused model kernels (one launch per edge of the layer graph):
//   k_residual_normq  — [embedding gather | GEMM requant_i32_common(tb)] +
//                       residual_add/renorm + DI-RMSNorm + smoothing + int8 quant
//                       (dyadic.py:108-120, :174-206; di_rmsnorm.py:33-52;
//                        model.py:187-198, :246-249, :410-415, :424-427)
//   k_swiglu_quant    — requant_i32_common(14) x2 + DI-SwiGLU + quant_i8
//                       (model.py:416-423; di_swiglu.py:39-58)
//   k_merge_rowcol    — attention-output merge: requant_i8_rowcol
//                       (model.py:404-409; dyadic.py:123-139)
//   k_qkv_epilogue    — per (token, head): requant_i32_common(16) + QK-norm +
//                       RoPE + QK-smoothing + Q int8 quant + score-scale /
//                       DI-Exp constant; K/V static int8 quant into the cache
//                       (model.py:200-216, :303-340, :351-358)
// Op-level kernels (the same device functions, one reference function each)
// back the op API used by the parity tests.

#include <type_traits>

#include "common.h"
#include "gemv.h"
#include "qkv_epilogue.h"

using namespace di;

namespace {

constexpr int RT = DI_ROW_THREADS;
// The fused model kernels run one row per block with up to RT_WIDE threads
// (at most 4 columns per thread), shortening the per-element part of the
// serial per-row chain that bounds them at decode.
constexpr int RT_WIDE = 1024;
// The block reducer of a row kernel launched with NT threads: launches at
// NT < RT_WIDE run exactly NT threads (prefill rows at 256, decode rows at
// the width their shape picks), so the reducer knows its wave count; the
// RT_WIDE instantiation runs the thread count in the args' nt.
template <int NT>
using RowRed = BlockRedT<NT < RT_WIDE ? NT / 64 : 0>;

template <int VPT, class Red>
__device__ __forceinline__ i64 row_absmax(const i64 (&v)[VPT], Red& red) {
  i64 g = 0;
#pragma unroll
  for (int j = 0; j < VPT; ++j) g = imax(g, wabs(v[j]));
  return red.max(g);
}

// max_j |v_j| over the row as an unsigned value: the same maximum as
// row_absmax, except that a row holding INT64_MIN (whose wrapped |v| is
// negative and counts for nothing in dyadic.py's row maximum) returns 2^63.
// The fp64 quotient estimates need |v| <= max, so such a row takes the
// exact path, which recomputes the maximum with row_absmax. The unsigned
// maximum reduces as signed values g - 2^63 (g ^ 2^63 for g <= 2^63).
template <int VPT, class Red>
__device__ __forceinline__ u64 row_absmax_u(const i64 (&v)[VPT], Red& red) {
  u64 g = 0;
#pragma unroll
  for (int j = 0; j < VPT; ++j) g = ::max(g, (u64)wabs(v[j]));
  constexpr u64 top = (u64)1 << 63;
  return (u64)red.max((i64)(g ^ top)) ^ top;
}

// ilog2(max(max_j |v_j|, 1)) over the row, from a 32-bit bit-length maximum
template <int VPT, class Red>
__device__ __forceinline__ i64 row_ilog2_absmax(const i64 (&v)[VPT], Red& red) {
  uint32_t L = 0;
#pragma unroll
  for (int j = 0; j < VPT; ++j) L = ::max(L, bitlen_abs(v[j]));
  return ilog2_from_bitlen(red.max_u32(L));
}

// ops/di_rmsnorm.py:33-52: v (<= C valid columns, 0 elsewhere) -> y (int32
// values). lg: ilog2(max(max |v|, 1)) when the caller already knows it, else
// -1 (one more block reduction).
template <int VPT, class Red>
__device__ __forceinline__ void rmsnorm_row(i64 (&v)[VPT], int C, Red& red, i64 lg = -1) {
  const i64 sh = 25 - (lg >= 0 ? lg : row_ilog2_absmax(v, red));
  const i64 up = imax(sh, 0), down = imax(-sh, 0);
  i64 ss = 0;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const i64 xp = shl(rshift_round(v[j], down), up);
    v[j] = xp;
    ss = wadd(ss, wmul(xp, xp));
  }
  ss = red.sum(ss);
  const i64 mean = (C & (C - 1)) == 0 ? rhad_pow2(ss, (int)ilog2(C)) : rhad(ss, (i64)C);
  const i64 rms = imax(isqrt_wave(mean), 1);
  if (DI_LIKELY(rms > ((i64)1 << 16))) {
    // the shift leaves |xp| <= 2^26, so 2 |xp| 2^20 + rms < 2^51 and the
    // quotient is below 2^31: rhad_est, and to_i32 keeps it
    const DivEst D = make_divest(rms, 1048576.0);
#pragma unroll
    for (int j = 0; j < VPT; ++j) v[j] = rhad_est_signed(v[j], D);
  } else {
    const Recip R = make_recip(rms);
#pragma unroll
    for (int j = 0; j < VPT; ++j) v[j] = to_i32(rhad_r(shl(v[j], 20), R));
  }
}

// dyadic.py:93-105. The quotients rhad(127 x, a) with |x| <= a come from the
// fp64 estimate (intops.h rhad_est) when a < 2^43 (then 2 * 127 |x| + a <
// 2^51 and no 127 x wraps), from the estimate corrected by its exact
// remainder (rhad_est_corr_signed) when a < 2^53, else from the 64-bit
// reciprocal.
template <int VPT, class Red>
__device__ __forceinline__ void quant_row(const i64 (&v)[VPT], i64 m_in, i64 k_in, int C,
                                          Red& red, int8_t* out, i64* m_out, i64* k_out,
                                          bool defer_fit = false) {
  i64 m, k;
  norm_scale(m_in, k_in, &m, &k);
  const u64 au = row_absmax_u(v, red);
  i64 a;
  if (DI_LIKELY(au < ((u64)1 << 43))) {
    a = imax((i64)au, 1);
    const DivEst D = make_divest(a, 127.0);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int c = red.tid() + j * red.nt();
      if (c < C) out[c] = (int8_t)rhad_est_signed(v[j], D);
    }
  } else if (DI_LIKELY(au < ((u64)1 << 53))) {
    a = (i64)au;
    const DivEst D = make_divest(a, 127.0);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int c = red.tid() + j * red.nt();
      if (c < C) out[c] = (int8_t)rhad_est_corr_signed(v[j], 127, a, D);
    }
  } else {
    a = DI_UNLIKELY(au >> 63) ? imax(row_absmax(v, red), 1) : (i64)au;
    const Recip R = make_recip(a);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int c = red.tid() + j * red.nt();
      if (c < C) out[c] = (int8_t)clamp_i8(rhad_r(wmul(v[j], 127), R));
    }
  }
  if (red.tid() == 0 && m_out) {
    if (defer_fit) {  // the consumer fits: (a m, k) stand for (m, k) = (fit(a m), k + e)
      *m_out = wmul(a, m);
      *k_out = k;
    } else {
      i64 mo, e;
      fit_dyadic_ratio_127(wmul(a, m), &mo, &e);
      *m_out = mo;
      *k_out = wadd(k, e);
    }
  }
}

// quant_row on exact integer values carried as doubles (|v| < 2^53), for a
// row whose every element this thread holds is exact (ok): the row maximum
// reduces the doubles' bit patterns (non-negative doubles order like their
// bits), and a thread whose values are not exact enters +inf, which sends
// the whole row back to the caller (returns false: the caller recomputes
// the values as int64 and runs quant_row). With a = max(max |v|, 1) below
// 2^43 the quotients rhad(127 |v|, a) come from the fp64 estimate, exactly
// as quant_row's (2 * 127 |v| + a < 2^51); a maximum in [2^43, 2^53) takes
// the same estimate corrected by its exact int64 remainder
// (rhad_est_corr_signed). Same integers and (m, k) as quant_row.
template <int VPT, class Red>
__device__ __forceinline__ bool quant_row_f64(const double (&v)[VPT], bool ok, i64 m_in, i64 k_in,
                                              int C, Red& red, int8_t* out, i64* m_out,
                                              i64* k_out, bool defer_fit = false) {
  double g = 0.0;
#pragma unroll
  for (int j = 0; j < VPT; ++j) g = fmax(g, fabs(v[j]));
  const i64 bits = red.max(ok ? f64_bits(g) : f64_bits(__builtin_inf()));
  if (DI_UNLIKELY(bits >= f64_bits(__builtin_inf()))) return false;
  const double au = f64_from_bits(bits);
  if (DI_UNLIKELY(au >= 0x1p53)) {  // (exact values stay below 2^53)
    i64 w[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) w[j] = (i64)v[j];
    quant_row(w, m_in, k_in, C, red, out, m_out, k_out, defer_fit);
    return true;
  }
  i64 m, k;
  norm_scale(m_in, k_in, &m, &k);
  const i64 a = imax((i64)au, 1);
  const DivEst D = make_divest(a, 127.0);
  if (DI_LIKELY(au < 0x1p43)) {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int c = red.tid() + j * red.nt();
      const uint32_t q = rhad_est(fabs(v[j]), D);
      if (c < C) out[c] = (int8_t)(v[j] < 0 ? -(int32_t)q : (int32_t)q);
    }
  } else {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int c = red.tid() + j * red.nt();
      const int32_t q = rhad_est_corr_signed((i64)v[j], 127, a, D);
      if (c < C) out[c] = (int8_t)q;
    }
  }
  if (red.tid() == 0 && m_out) {
    if (defer_fit) {
      *m_out = wmul(a, m);
      *k_out = k;
    } else {
      i64 mo, e;
      fit_dyadic_ratio_127(wmul(a, m), &mo, &e);
      *m_out = mo;
      *k_out = wadd(k, e);
    }
  }
  return true;
}

// rmsnorm_row, the smoothing product (sm: the row's smoothing mantissas when
// smooth) and quant_row(., 1, kq) of an int32-valued row h, on exact fp64
// values: the normalisation shift is a power-of-two scaling plus
// rshift_round_f64, the shifted values (|x| <= 2^26) square in int64 exactly
// as rmsnorm_row's (wrapping) sum does, and with rms > 2^16 the quotients
// rhad(x 2^20, rms) come from the same fp64 estimate, below 2^30 in
// magnitude; a smoothing mantissa below 2^21 keeps each product an exact
// double below 2^51 for quant_row_f64. Returns false (block-uniform, h
// untouched, nothing stored) when rms <= 2^16 (a zero row, or a sum of
// squares that wrapped): the caller runs the integer routines. A smoothing
// mantissa out of range makes the quantiser run on int64 products.
template <int VPT, class Red>
__device__ __forceinline__ bool norm_quant_row_f64(const i64 (&h)[VPT], int C, Red& red, i64 lg,
                                                   const i64 (&sm)[VPT], bool smooth, i64 kq,
                                                   int8_t* out, i64* m_out, i64* k_out) {
  if (lg < 0) lg = row_ilog2_absmax(h, red);
  const i64 sh = 25 - lg;
  const int up = (int)imax(sh, 0), down = (int)imax(-sh, 0);
  const double su = ldexp(1.0, up);
  double x[VPT];
  i64 ss = 0;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    x[j] = rshift_round_f64((double)(int32_t)h[j], down) * su;
    const int32_t xi = (int32_t)x[j];
    ss = wadd(ss, (i64)xi * xi);
  }
  ss = red.sum(ss);
  const i64 mean = (C & (C - 1)) == 0 ? rhad_pow2(ss, (int)ilog2(C)) : rhad(ss, (i64)C);
  const i64 rms = imax(isqrt_wave(mean), 1);
  if (DI_UNLIKELY(rms <= ((i64)1 << 16))) return false;
  const DivEst D = make_divest(rms, 1048576.0);
  constexpr i64 SM_LIM = (i64)1 << 21;
  bool ok = true;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    x[j] = (double)rhad_est_signed_f64(x[j], D);
    if (smooth) {
      ok = ok & in_range(sm[j], SM_LIM);
      x[j] *= (double)(int32_t)sm[j];
    }
  }
  if (DI_LIKELY(quant_row_f64(x, ok, 1, kq, C, red, out, m_out, k_out))) return true;
  i64 y[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) y[j] = wmul((i64)rhad_est_signed_f64(
      rshift_round_f64((double)(int32_t)h[j], down) * su, D), sm[j]);
  quant_row(y, 1, kq, C, red, out, m_out, k_out);
  return true;
}

// dyadic.py:108-120: v holds P on entry, y (int32 values) on exit; cm holds
// col_m of this thread's columns (0 past C); returns k_out
template <int VPT, class Red>
__device__ __forceinline__ i64 requant_common_row(i64 (&v)[VPT], const i64 (&cm)[VPT], i64 row_k,
                                                  i64 col_k, int tb, Red& red) {
#pragma unroll
  for (int j = 0; j < VPT; ++j) v[j] = wmul(v[j], cm[j]);
  const i64 sh = imax(row_ilog2_absmax(v, red) - (tb - 1), 0);
#pragma unroll
  for (int j = 0; j < VPT; ++j) v[j] = to_i32(rshift_round(v[j], sh));
  return wsub(wadd(row_k, col_k), sh);
}

// requant_common_row on two rows at once (gate and up of the same token):
// both bit-length maxima share one barrier. Returns the two k_out.
template <int VPT, class Red>
__device__ __forceinline__ void requant_common_row2(i64 (&v0)[VPT], const i64 (&cm0)[VPT],
                                                    i64 col_k0, i64 (&v1)[VPT],
                                                    const i64 (&cm1)[VPT], i64 col_k1, i64 row_k,
                                                    int tb, Red& red, i64* k0, i64* k1) {
  uint32_t L0 = 0, L1 = 0;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    v0[j] = wmul(v0[j], cm0[j]);
    v1[j] = wmul(v1[j], cm1[j]);
    L0 = ::max(L0, bitlen_abs(v0[j]));
    L1 = ::max(L1, bitlen_abs(v1[j]));
  }
  red.max2_u32(L0, L1);
  const i64 sh0 = imax(ilog2_from_bitlen(L0) - (tb - 1), 0);
  const i64 sh1 = imax(ilog2_from_bitlen(L1) - (tb - 1), 0);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    v0[j] = to_i32(rshift_round(v0[j], sh0));
    v1[j] = to_i32(rshift_round(v1[j], sh1));
  }
  *k0 = wsub(wadd(row_k, col_k0), sh0);
  *k1 = wsub(wadd(row_k, col_k1), sh1);
}

// dyadic.py:174-184. *lg_out: ilog2(max(max |h|, 1)) of the renormalised
// row when it follows from the reduction already done, else -1. Without a
// down-shift it does: an exact up-shift by u adds u to every bit length (and
// no shift leaves them), while rounding a down-shift may carry into the next
// bit.
template <int VPT, class Red>
__device__ __forceinline__ i64 residual_renorm_row(i64 (&h)[VPT], i64 k_res, Red& red,
                                                   i64* lg_out) {
  uint32_t L = 0;
#pragma unroll
  for (int j = 0; j < VPT; ++j) L = ::max(L, bitlen_abs(h[j]));
  L = red.max_u32(L);                       // g = max |h| > 0  <=>  L > 0
  const i64 lg = ilog2_from_bitlen(L);      // ilog2(max(g, 1))
  const i64 sh_down = imax(lg - 29, 0);
  i64 sh_up = L > 0 ? imax(26 - lg, 0) : 0;
  if (sh_down > 0) sh_up = 0;
#pragma unroll
  for (int j = 0; j < VPT; ++j) h[j] = to_i32(shl(rshift_round(h[j], sh_down), sh_up));
  *lg_out = sh_down > 0 ? -1 : ilog2_from_bitlen(L > 0 ? L + (uint32_t)sh_up : 0u);
  return wadd(wsub(k_res, sh_down), sh_up);
}

// dyadic.py:193-206
template <int VPT, class Red>
__device__ __forceinline__ i64 residual_add_row(i64 (&h)[VPT], i64 k_res, const i64 (&d)[VPT],
                                                i64 dm, i64 dk, Red& red, i64* lg_out) {
  const i64 rel = wsub(dk, k_res);
  const i64 down = imax(rel, 0), up = imax(wneg(rel), 0);
#pragma unroll
  for (int j = 0; j < VPT; ++j) h[j] = wadd(h[j], shl(rshift_round(wmul(d[j], dm), down), up));
  return residual_renorm_row(h, k_res, red, lg_out);
}

// requant_i32_common(tb) of a GEMM product, residual_add and the renorm
// (dyadic.py:108-120, :193-206, :174-184) on exact fp64 values. P holds the
// product sums (int32 values), cm the column mantissas, h the residual (int32
// values); on success h holds the renormalised residual, *kr its k and *lg
// what residual_renorm_row reports. Bounds, each making every intermediate an
// exact double and matching the int64 steps (no wrap anywhere):
//  * tb <= 20, |row_m| < 2^31, |col_m| < 2^21: P col_m is below 2^52, the
//    requantised d below 2^20 + 1, d row_m below 2^52 (rshift_round_f64);
//  * the alignment shift down <= 63 (rshift_round of |x| < 2^52 by 53..63
//    gives 0 both ways; from 64 on the int64 form differs) and up <= 52,
//    with the aligned delta below 2^51, so h + delta is below 2^52 and its
//    renormalisation is rshift_round_f64 and an exact power-of-two scaling.
// A row outside them returns false with h untouched (every test is
// block-uniform: row scalars, or a flag folded into a reduction), and the
// caller runs the integer routines.
template <int VPT, class Red>
__device__ __forceinline__ bool requant_residual_f64(i64 (&h)[VPT], const i64 (&P)[VPT],
                                                     const i64 (&cm)[VPT], i64 row_m, i64 row_k,
                                                     i64 col_k, int tb, i64 k_res, Red& red,
                                                     i64* kr, i64* lg_out) {
  if (tb > 20 || row_m <= -((i64)1 << 31) || row_m >= ((i64)1 << 31)) return false;
  constexpr i64 CM_LIM = (i64)1 << 21;
  double vd[VPT];
  uint32_t am = 0u;
  bool ok = true;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    ok = ok & in_range(cm[j], CM_LIM);
    vd[j] = (double)(int32_t)P[j] * (double)(int32_t)cm[j];
    am = ::max(am, f64_hiword_abs(vd[j]));
  }
  const uint32_t L = bitlen_from_hiword(red.max_u32(ok ? am : 0x7FF00000u));
  if (DI_UNLIKELY(L >= 64u)) return false;
  const i64 sh = imax(ilog2_from_bitlen(L) - (tb - 1), 0);
  const i64 dk = wsub(wadd(row_k, col_k), sh);
  const i64 rel = wsub(dk, k_res);
  const i64 down = imax(rel, 0), up = imax(wneg(rel), 0);
  if (down > 63 || up > 52) return false;
  const double rmd = (double)(int32_t)row_m, upf = ldexp(1.0, (int)up);
  double hn[VPT];
  uint32_t hm = 0u;
  ok = true;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const double d = rshift_round_f64(vd[j], (int)sh);
    const double al = rshift_round_f64(d * rmd, (int)down) * upf;
    ok = ok & (fabs(al) < 0x1p51);
    hn[j] = (double)(int32_t)h[j] + al;
    hm = ::max(hm, f64_hiword_abs(hn[j]));
  }
  const uint32_t L2 = bitlen_from_hiword(red.max_u32(ok ? hm : 0x7FF00000u));
  if (DI_UNLIKELY(L2 >= 64u)) return false;
  const i64 lg = ilog2_from_bitlen(L2);
  const i64 sh_down = imax(lg - 29, 0);
  const i64 sh_up = sh_down > 0 ? 0 : (L2 > 0 ? imax(26 - lg, 0) : 0);
  const double upf2 = ldexp(1.0, (int)sh_up);
#pragma unroll
  for (int j = 0; j < VPT; ++j) h[j] = (i64)(int32_t)(rshift_round_f64(hn[j], (int)sh_down) * upf2);
  *kr = wadd(wsub(k_res, sh_down), sh_up);
  *lg_out = sh_down > 0 ? -1 : ilog2_from_bitlen(L2 > 0 ? L2 + (uint32_t)sh_up : 0u);
  return true;
}

// Latency, not bandwidth, bounds these kernels at decode (one block per
// token row): every helper below issues all of its global loads before the
// first use, so a kernel waits for one memory round trip instead of one per
// load. The loads go through buffer views of the row (buf_view): a column
// past C reads 0, so each load is unconditional, needs no index clamp and no
// select after it, and its address is one 32-bit offset.

// Byte offset of this thread's column j (c = tid + j * nt) for elements of E bytes
template <int E, class Red>
__device__ __forceinline__ uint32_t col_off(const Red& red, int j) {
  return (uint32_t)(red.tid() + j * red.nt()) * (uint32_t)E;
}

// x[c] for the columns c = threadIdx.x + j * blockDim.x this thread owns (0 past C or
// when x is null).
template <int VPT, class Red>
__device__ __forceinline__ void prefetch_cols(i64 (&v)[VPT], const int64_t* x, int C,
                                              const Red& red) {
  const bufv_t xb = buf_view(x, x ? (i64)C * 8 : 0);
#pragma unroll
  for (int j = 0; j < VPT; ++j) v[j] = buf_ld_i64(xb, col_off<8>(red, j));
}

// x[c] for this thread's columns, 0 past C or when x is null (alt: unused,
// kept for the callers that name a stand-in vector).
template <int VPT, class Red>
__device__ __forceinline__ void load_cols_or0(i64 (&v)[VPT], const int64_t* x, const int64_t* alt,
                                              int C, const Red& red) {
  (void)alt;
  prefetch_cols(v, x, C, red);
}

// Row q of int32 partial k: P[k * stride + off[q] + c] for c < C
__device__ __forceinline__ bufv_t part_view(const int32_t* P, int k, i64 stride, i64 off, int C) {
  return buf_view(P + (i64)k * stride + off, (i64)C * 4);
}

// The first KF of the nsplit int32 partials P[k * stride + off + c], issued
// unconditionally (k clamped to nsplit - 1, nsplit >= 1); rows_i32_sum adds
// them, and the partials past KF, in a fixed order.
template <int KF, int NR, int VPT, class Red>
__device__ __forceinline__ void load_rows_i32_first(int32_t (&t)[KF][NR][VPT], const int32_t* P,
                                                    int nsplit, i64 stride, const i64 (&off)[NR],
                                                    int C, const Red& red) {
#pragma unroll
  for (int kk = 0; kk < KF; ++kk) {
    const int k = kk < nsplit ? kk : nsplit - 1;
#pragma unroll
    for (int q = 0; q < NR; ++q) {
      const bufv_t pb = part_view(P, k, stride, off[q], C);
#pragma unroll
      for (int j = 0; j < VPT; ++j) t[kk][q][j] = buf_ld_i32(pb, col_off<4>(red, j));
    }
  }
}
template <int KF, int NR, int VPT, class Red>
__device__ __forceinline__ void rows_i32_sum(i64 (&v)[NR][VPT], const int32_t (&t)[KF][NR][VPT],
                                             const int32_t* P, int nsplit, i64 stride,
                                             const i64 (&off)[NR], int C, const Red& red) {
  uint32_t s[NR][VPT];
#pragma unroll
  for (int q = 0; q < NR; ++q)
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      uint32_t a = 0;
#pragma unroll
      for (int kk = 0; kk < KF; ++kk)
        if (kk < nsplit) a += (uint32_t)t[kk][q][j];
      s[q][j] = a;
    }
  for (int k = KF; k < nsplit; ++k)  // more partials than KF: one at a time
#pragma unroll
    for (int q = 0; q < NR; ++q) {
      const bufv_t pb = part_view(P, k, stride, off[q], C);
#pragma unroll
      for (int j = 0; j < VPT; ++j) s[q][j] += (uint32_t)buf_ld_i32(pb, col_off<4>(red, j));
    }
#pragma unroll
  for (int q = 0; q < NR; ++q)
#pragma unroll
    for (int j = 0; j < VPT; ++j) v[q][j] = (i64)(int32_t)s[q][j];
}

// Sum of nsplit int32 partials P[k * stride + off + c] (the K-split of the
// skinny GEMM) in a fixed order, for NR rows at offsets off[0..NR).
template <int NR, int VPT, class Red>
__device__ __forceinline__ void load_rows_i32_sum(i64 (&v)[NR][VPT], const int32_t* P,
                                                  int nsplit, i64 stride, const i64 (&off)[NR],
                                                  int C, const Red& red) {
  if (nsplit == 1) {  // no K split (block-uniform): one load per element
#pragma unroll
    for (int q = 0; q < NR; ++q) {
      const bufv_t pb = part_view(P, 0, 0, off[q], C);
#pragma unroll
      for (int j = 0; j < VPT; ++j) v[q][j] = buf_ld_i32(pb, col_off<4>(red, j));
    }
    return;
  }
  constexpr int KU = NR * VPT > 8 ? 2 : 4;  // partials per batch of loads
  uint32_t s[NR][VPT];
#pragma unroll
  for (int q = 0; q < NR; ++q)
#pragma unroll
    for (int j = 0; j < VPT; ++j) s[q][j] = 0;
  for (int k0 = 0; k0 < nsplit; k0 += KU) {
    int32_t t[KU][NR][VPT];
#pragma unroll
    for (int kk = 0; kk < KU; ++kk) {
      const int k = k0 + kk < nsplit ? k0 + kk : nsplit - 1;
#pragma unroll
      for (int q = 0; q < NR; ++q) {
        const bufv_t pb = part_view(P, k, stride, off[q], C);
#pragma unroll
        for (int j = 0; j < VPT; ++j) t[kk][q][j] = buf_ld_i32(pb, col_off<4>(red, j));
      }
    }
#pragma unroll
    for (int kk = 0; kk < KU; ++kk)
      if (k0 + kk < nsplit)
#pragma unroll
        for (int q = 0; q < NR; ++q)
#pragma unroll
          for (int j = 0; j < VPT; ++j) s[q][j] += (uint32_t)t[kk][q][j];
  }
#pragma unroll
  for (int q = 0; q < NR; ++q)
#pragma unroll
    for (int j = 0; j < VPT; ++j) v[q][j] = (i64)(int32_t)s[q][j];
}

// =====================================================================
// Fused model kernels
// =====================================================================

struct ResNormArgs {
  int C;
  int nt;    // threads per block (set by the launch)
  int mode;  // 0: embedding gather (residual_from_delta); 1: GEMM residual add;
             // 2: norm-quant of the given rows only
  i64 vocab;
  const int64_t* ids;
  const int8_t* e8;
  const int64_t* em;
  const int64_t* ek;
  const int32_t* P;
  int nsplit;
  i64 split_stride;
  const int64_t* row_m;
  const int64_t* row_k;
  int row_fit;  // mode 1: (row_m, row_k) hold a deferred scale fit (fit_dyadic_ratio_127)
  const int64_t* col_m;
  i64 col_k;
  int tb;
  const int32_t* h_in;     // residual read (mode 1, 2); h when null
  const int64_t* k_res_in; // its k (mode 1); k_res when null
  int32_t* h;              // residual written (modes 0, 1); null: not stored
  int64_t* k_res;
  const int64_t* sm_m;  // null: no smoothing multiply
  i64 sm_k;
  int8_t* x8;  // null: no norm-quant
  i64 x8_stride;  // row stride of x8 (0: C)
  int64_t* xm;    // null: (m, k) of x8 not stored
  int64_t* xk;
  int32_t* err;  // optional device error word (DI_ERR_TOKEN)
  L2Warm warm;   // the next skinny GEMM's weights (extra blocks after the rows)
};

// MODE: the row's mode when the launch fixes it (the kernel then holds that
// path only: less code to fetch per launch), else -1 (a.mode decides).
template <int VPT, class Red, int MODE = -1>
__device__ __forceinline__ void residual_normq_row(const ResNormArgs& a, int r, Red& red) {
  const int mode = MODE >= 0 ? MODE : a.mode;
  const int C = a.C;
  const i64 off = (i64)r * C;
  i64 h[VPT], d[VPT], smv[VPT];
  i64 kr, lg = -1;
  const int32_t* h_in = a.h_in ? a.h_in : a.h;
  if (mode == 1) {
    // the GEMM residual add: every load of the row issued before any is used
    // (no branch between them; col_m is required in this mode, so it stands
    // in for a missing sm_m)
    i64 cm[VPT];
    load_cols_or0(smv, a.sm_m, a.col_m, C, red);
    load_cols_or0(cm, a.col_m, a.col_m, C, red);
    {
      const bufv_t hb = buf_view(h_in + off, (i64)C * 4);
#pragma unroll
      for (int j = 0; j < VPT; ++j) h[j] = buf_ld_i32(hb, col_off<4>(red, j));
    }
    i64 row_k = a.row_k[r], row_m = a.row_m[r];
    const i64 k_res = (a.k_res_in ? a.k_res_in : a.k_res)[r];
    constexpr int KF = 4;
    int32_t t[KF][1][VPT];
    const i64 offs[1] = {off};
    load_rows_i32_first<KF, 1, VPT>(t, a.P, a.nsplit, a.split_stride, offs, C, red);
    __builtin_amdgcn_sched_barrier(0);
    if (a.row_fit) {
      // the producer of the GEMM's operand left its scale fit to this launch:
      // every lane fits while the partials are in flight
      i64 fm, fe;
      fit_dyadic_ratio_127(row_m, &fm, &fe);
      row_m = fm;
      row_k = wadd(row_k, fe);
    }
    i64 dd[1][VPT];
    rows_i32_sum<KF, 1, VPT>(dd, t, a.P, a.nsplit, a.split_stride, offs, C, red);
#pragma unroll
    for (int j = 0; j < VPT; ++j) d[j] = dd[0][j];
    if (DI_UNLIKELY(!requant_residual_f64(h, d, cm, row_m, row_k, a.col_k, a.tb, k_res, red,
                                          &kr, &lg))) {
      const i64 dk = requant_common_row(d, cm, row_k, a.col_k, a.tb, red);
      kr = residual_add_row(h, k_res, d, row_m, dk, red, &lg);
    }
  } else {
  prefetch_cols(smv, a.sm_m, C, red);
  if (mode == 2) {
    // _norm_quant of a given residual row: h is read, not written
    const bufv_t hb = buf_view(h_in + off, (i64)C * 4);
#pragma unroll
    for (int j = 0; j < VPT; ++j) h[j] = buf_ld_i32(hb, col_off<4>(red, j));
    kr = 0;
  } else if (mode == 0) {
    const i64 id = torch_index(a.ids[r], a.vocab, red.tid() ? nullptr : a.err, DI_ERR_TOKEN);
    const i64 dm = a.em[id], ek = a.ek[id];
    const bufv_t eb = buf_view(a.e8 + id * C, C);
#pragma unroll
    for (int j = 0; j < VPT; ++j) h[j] = wmul((i64)buf_ld_i8(eb, col_off<1>(red, j)), dm);
    kr = residual_renorm_row(h, ek, red, &lg);
  } else {
    i64 cm[VPT];
    prefetch_cols(cm, a.col_m, C, red);
    {
      const bufv_t hb = buf_view(h_in + off, (i64)C * 4);
#pragma unroll
      for (int j = 0; j < VPT; ++j) h[j] = buf_ld_i32(hb, col_off<4>(red, j));
    }
    const i64 row_k = a.row_k[r], row_m = a.row_m[r];
    const i64 k_res = (a.k_res_in ? a.k_res_in : a.k_res)[r];
    i64 dd[1][VPT];
    const i64 offs[1] = {off};
    load_rows_i32_sum<1, VPT>(dd, a.P, a.nsplit, a.split_stride, offs, C, red);
#pragma unroll
    for (int j = 0; j < VPT; ++j) d[j] = dd[0][j];
    const i64 dk = requant_common_row(d, cm, row_k, a.col_k, a.tb, red);
    kr = residual_add_row(h, k_res, d, row_m, dk, red, &lg);
  }
  }
  if (mode != 2 && a.h) {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int c = red.tid() + j * red.nt();
      if (c < C) a.h[off + c] = (int32_t)h[j];
    }
    if (red.tid() == 0) a.k_res[r] = kr;
  }
  if (a.x8 == nullptr) return;
  const i64 kq = a.sm_m != nullptr ? wadd(20, a.sm_k) : 20;
  int8_t* const x8 = a.x8 + (i64)r * (a.x8_stride ? a.x8_stride : C);
  if (DI_LIKELY(norm_quant_row_f64(h, C, red, lg, smv, a.sm_m != nullptr, kq, x8,
                                   a.xm ? a.xm + r : nullptr, a.xk ? a.xk + r : nullptr)))
    return;
  rmsnorm_row(h, C, red, lg);
  if (a.sm_m != nullptr) {
#pragma unroll
    for (int j = 0; j < VPT; ++j) h[j] = wmul(h[j], smv[j]);
  }
  quant_row(h, 1, kq, C, red, x8, a.xm ? a.xm + r : nullptr, a.xk ? a.xk + r : nullptr);
}

template <int VPT, int NT = RT_WIDE, bool WARM = false, int MODE = -1>
__global__ __launch_bounds__(NT) void k_residual_normq(ResNormArgs a) {
  keep_hidden_args();
  __shared__ i64 red_buf[32];
  if (WARM && (int)blockIdx.x < L2WARM_BLOCKS) {  // no kernel argument needed to decide
    l2_warm(a.warm, blockIdx.x, a.nt, red_buf);
    return;
  }
  RowRed<NT> red{red_buf, 0, a.nt};
  residual_normq_row<VPT, decltype(red), MODE>(a, (int)blockIdx.x - (WARM ? L2WARM_BLOCKS : 0), red);
}

// The GEMM residual add (mode 1) only.
template <int VPT, int NT = RT_WIDE, bool WARM = false>
__global__ __launch_bounds__(NT) void k_residual_add_normq(ResNormArgs a) {
  keep_hidden_args();
  __shared__ i64 red_buf[32];
  if (WARM && (int)blockIdx.x < L2WARM_BLOCKS) {  // no kernel argument needed to decide
    l2_warm(a.warm, blockIdx.x, a.nt, red_buf);
    return;
  }
  RowRed<NT> red{red_buf, 0, a.nt};
  residual_normq_row<VPT, decltype(red), 1>(a, (int)blockIdx.x - (WARM ? L2WARM_BLOCKS : 0), red);
}

// Many rows (prefill): one wave per row, four rows per block, every
// reduction a DPP reduction within the wave (no LDS round trip, no barrier),
// so more rows are in flight per CU than with a block per row.
template <int VPT, int MODE>
__global__ __launch_bounds__(256) void k_residual_normq_w(ResNormArgs a, int R) {
  keep_hidden_args();
  // (wave-uniform: the row's buffer views live in scalar registers)
  const int r = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
  if (r >= R) return;  // whole waves
  WaveRed red;
  residual_normq_row<VPT, WaveRed, MODE>(a, r, red);
}

struct SwigluArgs {
  int I;
  int nt;    // threads per block (set by the launch)
  const int32_t* P;  // [nsplit][R][2I]: gate | up
  int nsplit;
  i64 split_stride;
  const int64_t* xm;
  const int64_t* xk;
  const int64_t* gate_m;
  i64 gate_k;
  const int64_t* up_m;
  i64 up_k;
  const int64_t* ds_m;
  i64 ds_k;
  int8_t* y8;
  int64_t* ym;
  int64_t* yk;
  int defer_fit;  // (ym, yk) left for the consumer to fit (quant_row)
  L2Warm warm;  // the next skinny GEMM's weights (extra blocks after the rows)
};

template <int VPT, class Red>
__device__ __forceinline__ void swiglu_quant_row(const SwigluArgs& a, int r, Red& red) {
  const int I = a.I;
  // Many rows (prefill, more than 4 columns per thread): the down-smoothing
  // scales load after the requantisation, when the gate/up scales are dead,
  // and g, u live as int32 — fewer registers, more rows resident per CU (other
  // rows hide the extra load). Decode rows load everything up front.
  constexpr bool kLate = VPT > 4;
  i64 gm[VPT], um[VPT], dsm[VPT];
  i64 gu[2][VPT];
  const i64 offs[2] = {(i64)r * 2 * I, (i64)r * 2 * I + I};
  i64 xm, xk;
  if (!kLate) {
    // decode rows: every load issued before any is used, no branch between
    // them (the scale vectors are required: the entry point checks them)
    load_cols_or0(gm, a.gate_m, a.gate_m, I, red);
    load_cols_or0(um, a.up_m, a.up_m, I, red);
    load_cols_or0(dsm, a.ds_m, a.ds_m, I, red);
    xm = a.xm[r];
    xk = a.xk[r];
    constexpr int KF = 2;  // decode gate|up products: at most two K splits
    int32_t t[KF][2][VPT];
    load_rows_i32_first<KF, 2, VPT>(t, a.P, a.nsplit, a.split_stride, offs, I, red);
    __builtin_amdgcn_sched_barrier(0);
    rows_i32_sum<KF, 2, VPT>(gu, t, a.P, a.nsplit, a.split_stride, offs, I, red);
  } else {
    prefetch_cols(gm, a.gate_m, I, red);
    prefetch_cols(um, a.up_m, I, red);
    xm = a.xm[r];
    xk = a.xk[r];
    load_rows_i32_sum<2, VPT>(gu, a.P, a.nsplit, a.split_stride, offs, I, red);
  }
  // requant_i32_common(14) of gate and up (dyadic.py:108-120) on fp64: with
  // |col_m| < 2^21 every product P col_m (|P| < 2^31) is an exact double
  // below 2^52, its bit length is the fp64 exponent and rshift_round_f64
  // applies. A thread holding a larger col_m enters bit length 64, which no
  // exact product reaches, and the row takes the integer routine. Only the
  // doubles stay live across the reduction: the integer routines reload
  // their operands (a rare path), which keeps the registers of the common
  // one free.
  constexpr i64 CM_LIM = (i64)1 << 21;
  double vg[VPT], vu[VPT];
  uint32_t L0, L1;
  {
    bool ok = true;
    L0 = L1 = 0u;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      ok = ok & in_range(gm[j], CM_LIM) & in_range(um[j], CM_LIM);
      vg[j] = (double)(int32_t)gu[0][j] * (double)(int32_t)gm[j];
      vu[j] = (double)(int32_t)gu[1][j] * (double)(int32_t)um[j];
      L0 = ::max(L0, f64_hiword_abs(vg[j]));
      L1 = ::max(L1, f64_hiword_abs(vu[j]));
    }
    // the bit lengths of the row maxima from the high words
    if (!ok) L0 = L1 = 0x7FF00000u;
  }
  red.max2_u32(L0, L1);
  L0 = bitlen_from_hiword(L0);
  L1 = bitlen_from_hiword(L1);
  i64 gk, uk;
  int32_t g32[VPT], u32[VPT];
  if (DI_LIKELY(L0 < 64u && L1 < 64u)) {
    const i64 sh0 = imax(ilog2_from_bitlen(L0) - 13, 0);
    const i64 sh1 = imax(ilog2_from_bitlen(L1) - 13, 0);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      g32[j] = (int32_t)rshift_round_f64(vg[j], (int)sh0);
      u32[j] = (int32_t)rshift_round_f64(vu[j], (int)sh1);
    }
    gk = wsub(wadd(xk, a.gate_k), sh0);
    uk = wsub(wadd(xk, a.up_k), sh1);
  } else {
    i64 cg[VPT], cu[VPT], v[2][VPT];
    prefetch_cols(cg, a.gate_m, I, red);
    prefetch_cols(cu, a.up_m, I, red);
    load_rows_i32_sum<2, VPT>(v, a.P, a.nsplit, a.split_stride, offs, I, red);
    requant_common_row2(v[0], cg, a.gate_k, v[1], cu, a.up_k, xk, 14, red, &gk, &uk);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      g32[j] = (int32_t)v[0][j];
      u32[j] = (int32_t)v[1][j];
    }
  }
  // requant_i32_common(14) leaves |g|, |u| <= 2^14 (the shift brings the
  // row's largest magnitude to at most 2^14)
  if (kLate) prefetch_cols(dsm, a.ds_m, I, red);
  const i64 tp = di_exp_tpos_fast(xm, gk);
  const i64 ym = wmul(xm, xm);
  const i64 yk = wadd(wadd(wadd(gk, uk), 7), a.ds_k);
  int8_t* const y8 = a.y8 + (i64)r * I;
  if (DI_LIKELY(tp < ((i64)1 << 23))) {
    // y = g sig u ds_m on fp64: |g sig| <= 2^21 (an int32 product), |g sig u|
    // <= 2^35, and with |ds_m| < 2^18 the last product is an exact double
    // below 2^53 (no int64 step wraps); otherwise the thread reports its
    // values inexact and the row quantises int64 values (ds_m reloaded)
    constexpr i64 DS_LIM = (i64)1 << 18;
    const ExpEst Ee = make_expest(tp);
    double yd[VPT];
    bool ok = true;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      ok = ok & in_range(dsm[j], DS_LIM);
      yd[j] = (double)(int32_t)swiglu_gsig_est(g32[j], Ee) * (double)u32[j] *
              (double)(int32_t)dsm[j];
    }
    if (DI_LIKELY(quant_row_f64(yd, ok, ym, yk, I, red, y8, a.ym + r, a.yk + r,
                                a.defer_fit != 0)))
      return;
    i64 ds[VPT], y[VPT];
    prefetch_cols(ds, a.ds_m, I, red);
#pragma unroll
    for (int j = 0; j < VPT; ++j) y[j] = wmul(swiglu_elem_est(g32[j], u32[j], Ee), ds[j]);
    quant_row(y, ym, yk, I, red, y8, a.ym + r, a.yk + r, a.defer_fit != 0);
  } else {
    const ExpR E = make_exp(tp);
    i64 y[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) y[j] = wmul(swiglu_elem_e(g32[j], u32[j], E), dsm[j]);
    quant_row(y, ym, yk, I, red, y8, a.ym + r, a.yk + r, a.defer_fit != 0);
  }
}

#ifndef SWIGLU_MINB
#define SWIGLU_MINB 4
#endif

// Prefill (256-thread blocks, 8-12 columns per thread): at least four blocks
// per CU (128 VGPRs; 12 columns spill some registers to scratch) — measured
// on the 2048-token MLP block: 80.7 us against 82.2 at three blocks (168
// VGPRs) and 86.7 at two.
template <int VPT, int NT = RT_WIDE, bool WARM = false>
__global__ __launch_bounds__(NT, (NT == 256 && VPT >= 8 && VPT <= 12) ? SWIGLU_MINB : 1) void k_swiglu_quant(
    SwigluArgs a) {
  keep_hidden_args();
  __shared__ i64 red_buf[32];
  if (WARM && (int)blockIdx.x < L2WARM_BLOCKS) {  // no kernel argument needed to decide
    l2_warm(a.warm, blockIdx.x, a.nt, red_buf);
    return;
  }
  RowRed<NT> red{red_buf, 0, a.nt};
  swiglu_quant_row<VPT>(a, (int)blockIdx.x - (WARM ? L2WARM_BLOCKS : 0), red);
}

struct MergeArgs {
  int C;
  int nt;    // threads per block (set by the launch)
  const int64_t* attn;  // [nsplit][R][C]
  int nsplit;
  i64 split_stride;
  const int64_t* os_m;
  i64 os_k;
  const int64_t* col_m;
  i64 col_k;
  int8_t* a8;
  i64 a8_stride;  // row stride of a8 (0: C)
  int64_t* am;    // null: (m, k) of a8 not stored
  int64_t* ak;
  int defer_fit;  // (am, ak) left for the consumer to fit (quant_row)
  L2Warm warm;    // the next skinny GEMM's weights (extra blocks after the rows)
  // k_gemv_pro PRO 4: the rows' statistics [R][n_ext][2] (per part of a row
  // the largest v and the largest ~v, v = attn * os_m * col_m; the parts
  // cover the row)
  const int64_t* ext;
  int n_ext;
};

// The merge's pre-shift sh and quantisation maximum a2 of a row from its
// largest and smallest value (each taken together with 0), valid when every
// |v| < 2^62: rshift_round(., sh) then cannot wrap and does not decrease, so
// max |rshift_round(v, sh)| sits at an extreme, and so does the bit length
// of max |v|. False (sh, a2 unset) outside that range.
__device__ __forceinline__ bool merge_shift_ext(i64 vmax, i64 vmin, i64* sh, i64* a2) {
  const i64 lim = (i64)1 << 62;
  if (!(vmax < lim && vmin > -lim)) return false;
  const uint32_t L = ::max(bitlen_abs(vmax), bitlen_abs(vmin));
  *sh = imax(ilog2_from_bitlen(L) - 45, 0);
  *a2 = imax(imax(wabs(rshift_round(vmax, *sh)), wabs(rshift_round(vmin, *sh))), 1);
  return true;
}

// (am, ak) of a merged row: the fit of a2 / 127 (dyadic.py:137-139), or a2
// itself for the consumer to fit (defer)
__device__ __forceinline__ void merge_row_scale(const MergeArgs& a, int r, i64 a2, i64 sh) {
  if (a.defer_fit) {
    a.am[r] = a2;
    a.ak[r] = wsub(wadd(a.os_k, a.col_k), sh);
  } else {
    i64 mo, e;
    fit_dyadic_ratio_127(a2, &mo, &e);
    a.am[r] = mo;
    a.ak[r] = wsub(wadd(wadd(a.os_k, a.col_k), e), sh);
  }
}

template <int VPT, class Red>
__device__ __forceinline__ void merge_rowcol_row(const MergeArgs& a, int r, Red& red) {
  const int C = a.C;
  const i64 off = (i64)r * C;
  int8_t* const a8 = a.a8 + (i64)r * (a.a8_stride ? a.a8_stride : C);
  i64 v[VPT], om[VPT];
  // per-column factor os_m * col_m (col_m null: os_m already holds the
  // product; int64 multiplication wraps modulo 2^64, so the order of the
  // two factors does not change a bit)
  // every load of the first partial issued before any is used, no branch
  // between them (os_m stands in for a missing col_m)
  i64 cm[VPT];
  load_cols_or0(om, a.os_m, a.os_m, C, red);
  load_cols_or0(cm, a.col_m, a.os_m, C, red);
  {
    const bufv_t ab = buf_view(a.attn + off, (i64)C * 8);
#pragma unroll
    for (int j = 0; j < VPT; ++j) v[j] = buf_ld_i64(ab, col_off<8>(red, j));  // partial 0
  }
  __builtin_amdgcn_sched_barrier(0);
  if (a.col_m) {
#pragma unroll
    for (int j = 0; j < VPT; ++j) om[j] = wmul(om[j], cm[j]);
  }
  constexpr int KB = VPT > 16 ? 1 : 2;  // partials per batch of loads (registers)
  for (int k0 = 1; k0 < a.nsplit; k0 += KB) {
    i64 t[KB][VPT];
#pragma unroll
    for (int kk = 0; kk < KB; ++kk) {
      const int k = k0 + kk < a.nsplit ? k0 + kk : a.nsplit - 1;
      const bufv_t ab = buf_view(a.attn + (i64)k * a.split_stride + off, (i64)C * 8);
#pragma unroll
      for (int j = 0; j < VPT; ++j) t[kk][j] = buf_ld_i64(ab, col_off<8>(red, j));
    }
#pragma unroll
    for (int kk = 0; kk < KB; ++kk)
      if (k0 + kk < a.nsplit)
#pragma unroll
        for (int j = 0; j < VPT; ++j) v[j] = wadd(v[j], t[kk][j]);
  }
#pragma unroll
  for (int j = 0; j < VPT; ++j) v[j] = wmul(v[j], om[j]);  // 0 past C
  // Blocks: the pre-shift and the quantisation maximum from one reduction
  // of the row's largest and smallest value. Both follow from them when
  // every |v| < 2^62 (then rshift_round(., sh) cannot wrap and does not
  // decrease, so max_j |rshift_round(v_j, sh)| sits at an extreme, and so
  // does the bit length of max |v|); else (INT64_MIN or near-overflow
  // values), and in a single wave, where two reductions cost less than the
  // extra work, the two reductions of dyadic.py:133-136 run as written.
  i64 sh, a2;
  bool exact = false;      // a row holding INT64_MIN after the shift
  i64 vmax = INT64_MAX, vmin = 0;
  if constexpr (Red::kBlock) {
    vmax = 0;  // columns past C hold 0
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      vmax = imax(vmax, v[j]);
      vmin = imin(vmin, v[j]);
    }
    i64 nmin = ~vmin;  // ~ reverses the order without overflow
    if (red.nt() <= 512) {
      red.max2(vmax, nmin);
    } else {
      vmax = red.max(vmax);
      nmin = red.max(nmin);
    }
    vmin = ~nmin;
  }
  if (DI_LIKELY(merge_shift_ext(vmax, vmin, &sh, &a2))) {
#pragma unroll
    for (int j = 0; j < VPT; ++j) v[j] = rshift_round(v[j], sh);
  } else {
    sh = imax(row_ilog2_absmax(v, red) - 45, 0);
#pragma unroll
    for (int j = 0; j < VPT; ++j) v[j] = rshift_round(v[j], sh);
    const u64 au = row_absmax_u(v, red);
    exact = au >> 63;
    a2 = DI_UNLIKELY(exact) ? imax(row_absmax(v, red), 1) : imax((i64)au, 1);
  }
  if (DI_LIKELY(a2 < ((i64)1 << 46) && !exact)) {
    // |v| <= a2 < 2^46 (the pre-shift leaves at most 46 bits): 127 |v| does
    // not wrap and 127 |v| + a2 < 2^53; the plain estimate is exact below
    // 2^43, the corrected one above
    const DivEst D = make_divest(a2, 127.0);
    if (DI_LIKELY(a2 < ((i64)1 << 43))) {
#pragma unroll
      for (int j = 0; j < VPT; ++j) {
        const int c = red.tid() + j * red.nt();
        if (c < C) a8[c] = (int8_t)rhad_est_signed(v[j], D);
      }
    } else {
#pragma unroll
      for (int j = 0; j < VPT; ++j) {
        const int c = red.tid() + j * red.nt();
        if (c < C) a8[c] = (int8_t)rhad_est_corr_signed(v[j], 127, a2, D);
      }
    }
  } else {
    const Recip R = make_recip(a2);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int c = red.tid() + j * red.nt();
      if (c < C) a8[c] = (int8_t)clamp_i8(rhad_r(wmul(v[j], 127), R));
    }
  }
  if (red.tid() == 0 && a.am) merge_row_scale(a, r, a2, sh);
}

// The merge of decode rows from the attention's row statistics (a.ext,
// a.n_ext <= 8 entries per row): every value is elementwise once the row's
// pre-shift and maximum are known, so each row is cut into 256-column
// pieces, one block each (one column per thread, no reduction), after the
// L2-warming blocks of the next GEMV. A row outside the estimate tiers is
// merged in full by each of its piece blocks (the same bytes; piece 0 stores
// the scale). C <= 2048.
constexpr int MEXT_MAX = 8;  // statistics entries per row
template <bool WARM>
__global__ __launch_bounds__(256) void k_merge_ext(MergeArgs a, int pieces) {
  keep_hidden_args();
  __shared__ i64 red_buf[32];
  if (WARM && (int)blockIdx.x < L2WARM_BLOCKS) {  // no kernel argument needed to decide
    l2_warm(a.warm, blockIdx.x, 256, red_buf);
    return;
  }
  const int bid = (int)blockIdx.x - (WARM ? L2WARM_BLOCKS : 0);
  const int r = bid / pieces, piece = bid - r * pieces;
  const int C = a.C;
  const int c = piece * 256 + (int)threadIdx.x;
  // the value, its factor and the row's statistics (the same entries on
  // every lane), all issued before any is used
  const i64 x = buf_ld_i64(buf_view(a.attn + (i64)r * C, (i64)C * 8), c < C ? (uint32_t)c * 8 : BUF_OOB);
  const i64 om = buf_ld_i64(buf_view(a.os_m, (i64)C * 8), c < C ? (uint32_t)c * 8 : BUF_OOB);
  v4i q[MEXT_MAX];
  {
    const bufv_t ev = buf_view(a.ext + (i64)r * a.n_ext * 2, (i64)a.n_ext * 16);
#pragma unroll
    for (int e = 0; e < MEXT_MAX; ++e) q[e] = buf_ld_16<v4i>(ev, e < a.n_ext ? (uint32_t)e * 16 : BUF_OOB);
  }
  __builtin_amdgcn_sched_barrier(0);
  i64 vmax = 0, nmin = -1;
#pragma unroll
  for (int e = 0; e < MEXT_MAX; ++e) {
    const i64 hi = (i64)(((u64)(uint32_t)q[e][1] << 32) | (uint32_t)q[e][0]);
    const i64 nm = (i64)(((u64)(uint32_t)q[e][3] << 32) | (uint32_t)q[e][2]);
    vmax = imax(vmax, hi);
    nmin = imax(nmin, e < a.n_ext ? nm : (i64)-1);
  }
  i64 sh = 0, a2 = 1;
  const bool fast = merge_shift_ext(vmax, ~nmin, &sh, &a2) && a2 < ((i64)1 << 46);
  int8_t* const a8 = a.a8 + (i64)r * (a.a8_stride ? a.a8_stride : C);
  if (DI_LIKELY(fast)) {  // uniform: the row's statistics
    const DivEst D = make_divest(a2, 127.0);
    const i64 v = rshift_round(wmul(x, om), sh);
    const int qv = a2 < ((i64)1 << 43) ? rhad_est_signed(v, D) : rhad_est_corr_signed(v, 127, a2, D);
    if (c < C) a8[c] = (int8_t)qv;
    if (piece == 0 && threadIdx.x == 0 && a.am) merge_row_scale(a, r, a2, sh);
    return;
  }
  MergeArgs m = a;
  if (piece != 0) {
    m.am = nullptr;
    m.ak = nullptr;
  }
  BlockRedT<4> red{red_buf, 0, 256};
  merge_rowcol_row<8>(m, r, red);
}

template <int VPT, int NT = RT_WIDE, bool WARM = false>
__global__ __launch_bounds__(NT) void k_merge_rowcol(MergeArgs a) {
  keep_hidden_args();
  __shared__ i64 red_buf[32];
  if (WARM && (int)blockIdx.x < L2WARM_BLOCKS) {  // no kernel argument needed to decide
    l2_warm(a.warm, blockIdx.x, a.nt, red_buf);
    return;
  }
  RowRed<NT> red{red_buf, 0, a.nt};
  merge_rowcol_row<VPT>(a, (int)blockIdx.x - (WARM ? L2WARM_BLOCKS : 0), red);
}

__global__ __launch_bounds__(RT) void k_qkv_epilogue(QKVArgs a) {
  keep_hidden_args();
  const int slotw = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (slotw >= a.n_q + 2 * a.n_kv) return;
  const int r = blockIdx.x;  // token row = b * T + t
  const int b = r / a.T, t = r - b * a.T;
  const i64 qrow = ((i64)b * a.n_q + (slotw < a.n_q ? slotw : 0)) * a.T + t;
  qkv_head(a, r, slotw, a.q8 + qrow * 128, a.tpos + qrow);
}

// Many token rows (prefill): one wave per (head slot, 4 rows), head-major so
// a block's waves share a head's scale vectors.
#ifndef QKV_ROWS_MINW
#define QKV_ROWS_MINW 1
#endif
__global__ __launch_bounds__(RT, QKV_ROWS_MINW) void k_qkv_epilogue_rows(QKVArgs a, int R, int ngroups) {
  keep_hidden_args();
  const int heads = a.n_q + 2 * a.n_kv;
  // (wave-uniform, so the head slot's pointer and scale selects stay scalar)
  const int wg = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + (threadIdx.x >> 6)));
  if (wg >= heads * ngroups) return;  // whole waves only
  const int slotw = wg / ngroups, grp = wg - slotw * ngroups;
  qkv_rows4(a, R, grp * 4, slotw);
}

// Bookkeeping of one graphed decode step before its replay (graphed.py:112-131
// semantics): slot `slot` becomes valid in every row, the step's K/V write
// slot and scanned-slot count go to the device scalars the captured kernels
// read, and each row's position is its prompt length plus the steps taken.
__global__ __launch_bounds__(256) void k_decode_prologue(uint8_t* valid, i64 stride, int B, i64 slot,
                                                         int64_t* len_idx, int64_t* nslots,
                                                         int64_t* pos, const int64_t* pos0,
                                                         i64 step) {
  keep_hidden_args();
  for (int b = threadIdx.x; b < B; b += blockDim.x) {
    valid[(i64)b * stride + slot] = 1;
    pos[b] = pos0[b] + step;
  }
  if (threadIdx.x == 0) {
    len_idx[0] = slot;
    nslots[0] = slot + 1;
  }
}

// kq_channel of every channel: est[i] = {den, up, bits of D.r, bits of D.k}
__global__ __launch_bounds__(256) void k_kq_est(const int64_t* kq_m, const int64_t* kq_k, i64 n,
                                                i64 rowk, int64_t* est) {
  keep_hidden_args();
  const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
  if (i >= n) return;
  const KqChan q = kq_channel(kq_m[i], kq_k[i], rowk);
  est[i * 4 + 0] = q.den;
  est[i * 4 + 1] = q.up;
  est[i * 4 + 2] = __double_as_longlong(q.D.r);
  est[i * 4 + 3] = __double_as_longlong(q.D.k);
}

// =====================================================================
// Op-level row kernels (one reference function each)
// =====================================================================

template <int VPT>
__device__ __forceinline__ void load_row64(i64 (&v)[VPT], const int64_t* x, i64 off, int C) {
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int c = threadIdx.x + j * (int)blockDim.x;
    v[j] = c < C ? x[off + c] : 0;
  }
}

template <int VPT>
__global__ __launch_bounds__(RT) void k_op_quant(const int64_t* x, const int64_t* m,
                                                 const int64_t* k, int C, int8_t* x8,
                                                 int64_t* mo, int64_t* ko) {
  keep_hidden_args();
  __shared__ i64 red_buf[32];
  BlockRedT<RT / 64> red{red_buf, 0, RT};
  const int r = blockIdx.x;
  i64 v[VPT];
  load_row64(v, x, (i64)r * C, C);
  quant_row(v, m[r], k[r], C, red, x8 + (i64)r * C, mo + r, ko + r);
}

template <int VPT>
__global__ __launch_bounds__(RT) void k_op_requant_common(const int64_t* P, const int64_t* row_k,
                                                          const int64_t* col_m, int G, i64 col_k,
                                                          int tb, int C, int32_t* y,
                                                          int64_t* ko) {
  keep_hidden_args();
  __shared__ i64 red_buf[32];
  BlockRedT<RT / 64> red{red_buf, 0, RT};
  const int r = blockIdx.x;
  i64 v[VPT];
  load_row64(v, P, (i64)r * C, C);
  i64 cm[VPT];
  prefetch_cols(cm, col_m + (i64)(r % G) * C, C, red);
  const i64 k = requant_common_row(v, cm, row_k[r], col_k, tb, red);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int c = threadIdx.x + j * (int)blockDim.x;
    if (c < C) y[(i64)r * C + c] = (int32_t)v[j];
  }
  if (threadIdx.x == 0) ko[r] = k;
}

template <int VPT>
__global__ __launch_bounds__(RT) void k_op_rowcol(const int64_t* P, const int64_t* row_m,
                                                  const int64_t* row_k, const int64_t* col_m,
                                                  i64 col_k, int C, int8_t* y8, int64_t* mo,
                                                  int64_t* ko) {
  keep_hidden_args();
  __shared__ i64 red_buf[32];
  BlockRedT<RT / 64> red{red_buf, 0, RT};
  const int r = blockIdx.x;
  i64 v[VPT];
  load_row64(v, P, (i64)r * C, C);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int c = threadIdx.x + j * (int)blockDim.x;
    v[j] = c < C ? wmul(v[j], col_m[c]) : 0;
  }
  const i64 sh = imax(row_ilog2_absmax(v, red) - 45, 0);
#pragma unroll
  for (int j = 0; j < VPT; ++j) v[j] = rshift_round(v[j], sh);
  const i64 a2 = imax(row_absmax(v, red), 1);
  const Recip R = make_recip(a2);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int c = threadIdx.x + j * (int)blockDim.x;
    if (c < C) y8[(i64)r * C + c] = (int8_t)clamp_i8(rhad_r(wmul(v[j], 127), R));
  }
  if (threadIdx.x == 0) {
    i64 m, e;
    fit_dyadic_ratio_127(wmul(a2, row_m[r]), &m, &e);
    mo[r] = m;
    ko[r] = wsub(wadd(wadd(row_k[r], col_k), e), sh);
  }
}

// mode 0: residual_renorm(h64, k); 1: residual_add(h, k, d, dm, dk)
template <int VPT>
__global__ __launch_bounds__(RT) void k_op_residual(int mode, const int64_t* h_in,
                                                    const int64_t* k_res, const int64_t* d,
                                                    const int64_t* dm, const int64_t* dk, int C,
                                                    int32_t* h_out, int64_t* k_out) {
  keep_hidden_args();
  __shared__ i64 red_buf[32];
  BlockRedT<RT / 64> red{red_buf, 0, RT};
  const int r = blockIdx.x;
  i64 h[VPT];
  load_row64(h, h_in, (i64)r * C, C);
  i64 k, lg;
  if (mode == 0) {
    k = residual_renorm_row(h, k_res[r], red, &lg);
  } else {
    i64 dv[VPT];
    load_row64(dv, d, (i64)r * C, C);
    k = residual_add_row(h, k_res[r], dv, dm[r], dk[r], red, &lg);
  }
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int c = threadIdx.x + j * (int)blockDim.x;
    if (c < C) h_out[(i64)r * C + c] = (int32_t)h[j];
  }
  if (threadIdx.x == 0) k_out[r] = k;
}

template <int VPT>
__global__ __launch_bounds__(RT) void k_op_rmsnorm(const int64_t* x, const int64_t* gamma_m,
                                                   int C, int32_t* y32, int64_t* y64) {
  keep_hidden_args();
  __shared__ i64 red_buf[32];
  BlockRedT<RT / 64> red{red_buf, 0, RT};
  const int r = blockIdx.x;
  i64 v[VPT];
  load_row64(v, x, (i64)r * C, C);
  rmsnorm_row(v, C, red);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int c = threadIdx.x + j * (int)blockDim.x;
    if (c < C) {
      if (gamma_m) y64[(i64)r * C + c] = wmul(v[j], gamma_m[c]);
      else y32[(i64)r * C + c] = (int32_t)v[j];
    }
  }
}

template <int VPT>
__global__ __launch_bounds__(RT) void k_op_softmax(const int64_t* x, const int64_t* m,
                                                   const int64_t* k, const uint8_t* valid,
                                                   int has_clip, i64 clip_c, int p_out_bits,
                                                   int C, int32_t* probs) {
  keep_hidden_args();
  // ops/di_softmax.py:33-61
  __shared__ i64 red_buf[32];
  BlockRedT<RT / 64> red{red_buf, 0, RT};
  const int r = blockIdx.x;
  const i64 off = (i64)r * C;
  const i64 NEG = INT64_MIN + 1;
  i64 v[VPT];
  bool ok[VPT];
  i64 mx = NEG;
  bool anyv = false;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int c = threadIdx.x + j * (int)blockDim.x;
    ok[j] = c < C && valid[off + c] != 0;
    v[j] = c < C ? x[off + c] : 0;
    if (ok[j]) {
      mx = imax(mx, v[j]);
      anyv = true;
    }
  }
  mx = red.max(mx);
  const i64 any = red.max(anyv ? 1 : 0);
  if (!any) mx = 0;
  const i64 mm = m[r], kk = k[r];
  const ExpR Et = make_exp(di_exp_tpos(mm, kk));
  i64 cint = 0;
  if (has_clip) cint = rhad(wmul(clip_c, shl(1, kk)), mm);
  i64 den = 0;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    i64 xd = ok[j] ? wsub(v[j], mx) : 0;
    if (has_clip) xd = imax(xd, wneg(cint));
    // xd <= 0 for every visible slot (x <= row max, clip only raises it)
    const i64 e = !ok[j] ? 0 : (xd <= 0 ? di_exp_neg((u64)wneg(xd), Et)
                                        : di_exp_r(xd, Et.tpos, Et.R));
    v[j] = e;
    den = wadd(den, e);
  }
  den = imax(red.sum(den), 1);
  const Recip Rd = make_recip(den);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int c = threadIdx.x + j * (int)blockDim.x;
    if (c < C) probs[off + c] = (int32_t)to_i32(rhad_r(shl(v[j], p_out_bits - 1), Rd));
  }
}

__global__ void k_op_di_exp(const int64_t* x, const int64_t* m, const int64_t* k, int C,
                            i64 n, int64_t* res, int64_t* tpos_out) {
  keep_hidden_args();
  // ops/di_exp.py:21-37, row constants recomputed per element
  for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n;
       i += (i64)gridDim.x * blockDim.x) {
    const i64 r = i / C;
    const ExpR E = make_exp(di_exp_tpos(m[r], k[r]));
    res[i] = x[i] <= 0 ? di_exp_neg((u64)wneg(x[i]), E) : di_exp_r(x[i], E.tpos, E.R);
    if (i % C == 0) tpos_out[r] = E.tpos;
  }
}

__global__ void k_op_swiglu(const int64_t* gate, const int64_t* gm, const int64_t* gk,
                            const int64_t* up, const int64_t* um, const int64_t* uk, int C,
                            i64 n, int64_t* y, int64_t* ym, int64_t* yk) {
  keep_hidden_args();
  for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n;
       i += (i64)gridDim.x * blockDim.x) {
    const i64 r = i / C;
    y[i] = swiglu_elem_e(gate[i], up[i], make_exp(di_exp_tpos(gm[r], gk[r])));
    if (i % C == 0) {
      ym[r] = wmul(gm[r], um[r]);
      yk[r] = wadd(wadd(gk[r], uk[r]), 7);
    }
  }
}

__global__ void k_op_rope(const int64_t* x, const int64_t* pos, const int16_t* cos_t,
                          const int16_t* sin_t, i64 max_pos, i64 rows, int64_t* y,
                          int32_t* err) {
  keep_hidden_args();
  // ops/rope.py:38-55 on rows of 128 channels
  const i64 r = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const i64 p = torch_index(pos[r], max_pos, lane ? nullptr : err, DI_ERR_POSITION);
  const i64 x0 = x[r * 128 + lane], x1 = x[r * 128 + lane + 64];
  y[r * 128 + lane] = rshift_round(
      wadd(wmul(x0, (i64)cos_t[p * 128 + lane]), wmul(wneg(x1), (i64)sin_t[p * 128 + lane])), 14);
  y[r * 128 + lane + 64] = rshift_round(
      wadd(wmul(x1, (i64)cos_t[p * 128 + lane + 64]), wmul(x0, (i64)sin_t[p * 128 + lane + 64])),
      14);
}

__global__ void k_op_static(const int64_t* P, const int64_t* row_m, const int64_t* row_k,
                            const int64_t* col_m, const int64_t* col_k, const int64_t* s_m,
                            const int64_t* s_k, i64 n, int8_t* y8) {
  keep_hidden_args();
  // dyadic.py:142-163 with every operand materialised per element
  for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n;
       i += (i64)gridDim.x * blockDim.x) {
    const i64 num = wmul(wmul(P[i], col_m[i]), row_m[i]);
    const i64 shift = wsub(wadd(row_k[i], col_k[i]), s_k[i]);
    const i64 up = imax(wneg(shift), 0), down = imax(shift, 0);
    i64 den = shl(s_m[i], down);
    if (den == 0) den = 1;  // the reference's division raises there
    y8[i] = (int8_t)clamp_i8(rhad(shl(num, up), den));
  }
}

// requant_i8_static of a GEMM's int32 output with per-row (row_m, row_k)
// (null: (1, 0)), per-column col_m, scalar col_k and a scalar static target
// (s_m, s_k) — dyadic.py:142-163; config c0's canonical epilogue is
// (P, 1, 0, m, 20, 1, 0). P: nsplit int32 partials, summed in a fixed order.
// One thread per 4 consecutive columns of a row.
__global__ __launch_bounds__(256) void k_static_cols(const int32_t* __restrict__ P, int nsplit,
                                                     i64 split_stride, int R, int C,
                                                     const int64_t* row_m, const int64_t* row_k,
                                                     const int64_t* __restrict__ col_m, i64 col_k,
                                                     i64 s_m, i64 s_k, int8_t* __restrict__ y8) {
  keep_hidden_args();
  const int cq = (C + 3) / 4;
  const i64 t = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (i64)R * cq) return;
  const int r = (int)(t / cq), c0 = (int)(t - (i64)r * cq) * 4;
  const i64 rm = row_m ? row_m[r] : 1, rk = row_k ? row_k[r] : 0;
  const i64 shift = wsub(wadd(rk, col_k), s_k);
  const i64 up = imax(wneg(shift), 0), down = imax(shift, 0);
  i64 den = shl(s_m, down);
  if (den == 0) den = 1;  // the reference's division raises there
  const bool fast_den = den > 0 && den < ((i64)1 << 49);
  const DivEst D = make_divest(fast_den ? den : 1, 1.0);
  const i64 off = (i64)r * C + c0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (c0 + j >= C) break;
    uint32_t acc = 0;
    for (int k = 0; k < nsplit; ++k) acc += (uint32_t)P[(i64)k * split_stride + off + j];
    const i64 n = shl(wmul(wmul((i64)(int32_t)acc, col_m[c0 + j]), rm), up);
    const i64 lim = (i64)1 << 49;  // 2 |n| + den < 2^51 for rhad_est_i8
    y8[off + j] = (int8_t)((fast_den && n > -lim && n < lim) ? rhad_est_i8(n, D)
                                                             : clamp_i8(rhad(n, den)));
  }
}

// op: 0 isqrt, 1 ilog2, 2 norm_scale, 3 fit_dyadic_ratio, 4 scaled_round_div,
// 5 fit_dyadic_ratio(a, 127) through the constant-127 path the kernels use
// (6, the wave-parallel isqrt, runs in k_op_isqrt_wave)
__global__ void k_op_scalar(int op, const int64_t* a, const int64_t* b, const int64_t* c, i64 n,
                            int64_t* o1, int64_t* o2) {
  keep_hidden_args();
  for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n;
       i += (i64)gridDim.x * blockDim.x) {
    i64 x, y;
    switch (op) {
      case 0: o1[i] = isqrt(a[i]); break;
      case 1: o1[i] = ilog2(a[i]); break;
      case 2: norm_scale(a[i], b[i], &x, &y); o1[i] = x; o2[i] = y; break;
      case 3: fit_dyadic_ratio(a[i], b[i], &x, &y); o1[i] = x; o2[i] = y; break;
      case 5: fit_dyadic_ratio_127(a[i], &x, &y); o1[i] = x; o2[i] = y; break;
      case 7: o1[i] = sigmoid_est24((uint32_t)a[i], (uint32_t)b[i]); break;
      // the fp64-estimate forms of the fused kernels, element by element:
      // a = operand, b = divisor or tpos, c = scale s (8, 9, 11) or k (14)
      case 8: o1[i] = rhad_est((double)a[i], make_divest(b[i], (double)c[i])); break;
      case 9: o1[i] = rhad_est_signed(a[i], make_divest(b[i], (double)c[i])); break;
      case 10: o1[i] = rhad_est_i8(a[i], make_divest(b[i], 1.0)); break;
      case 11:
        o1[i] = rhad_est_corr_signed(a[i], (int)c[i], b[i], make_divest(b[i], (double)c[i]));
        break;
      case 12: o1[i] = dexp_est((uint32_t)a[i], make_expest(b[i])); break;
      case 13: {
        const ExpEst E = make_expest(b[i]);
        o1[i] = dexp_est_sp((int32_t)a[i], E, dexp_sp_const(E));
        break;
      }
      case 14: o1[i] = di_exp_tpos_fast(a[i], b[i]); break;
      case 15: o1[i] = isqrt_est(a[i]); break;
      default: o1[i] = scaled_round_div(a[i], b[i], c[i]); break;
    }
  }
}

// isqrt_wave on every element: each wave walks its 64 elements one at a time
// (the search needs the whole wave; indices are clamped so every lane stays
// active).
__global__ void k_op_isqrt_wave(const int64_t* a, i64 n, int64_t* o) {
  keep_hidden_args();
  const i64 lane = threadIdx.x & 63;
  const i64 wave0 = (blockIdx.x * (i64)blockDim.x + threadIdx.x) - lane;
  const i64 stride = (i64)gridDim.x * blockDim.x;
  for (i64 base = wave0; base < n; base += stride) {
    const i64 i = base + lane < n ? base + lane : n - 1;
    const i64 mine = a[i];
    i64 res = 0;
    for (int j = 0; j < 64; ++j) {
      const i64 nj = readlane64(mine, j);
      const i64 r = isqrt_wave(nj);
      if (lane == j) res = r;
    }
    if (base + lane < n) o[base + lane] = res;
  }
}

inline int pick_vpt(int C) {
  const int need = (C + RT - 1) / RT;
  if (need <= 1) return 1;
  if (need <= 2) return 2;
  if (need <= 4) return 4;
  if (need <= 8) return 8;
  if (need <= 12) return 12;
  if (need <= 16) return 16;
  return 0;
}

// threads and columns per thread of a fused row kernel over C columns
inline bool wide_shape(int C, int* threads, int* vpt) {
  int t = ((C + 3) / 4 + 63) / 64 * 64;
  t = t < 64 ? 64 : (t > RT_WIDE ? RT_WIDE : t);
  const int v = (C + t - 1) / t;
  if (v > 4) return false;
  *threads = t;
  *vpt = v;
  return true;
}

inline int grid_for(i64 n) {
  i64 g = (n + 255) / 256;
  return (int)(g < 65536 ? (g < 1 ? 1 : g) : 65536);
}

// =====================================================================
// Decode GEMV with its operand's row kernel fused in
// =====================================================================
//
// At decode (R <= 8 rows) a skinny GEMM waits for the row kernel that makes
// its int8 operand, and each of those launches is latency-bound: the row
// kernel by its chain of block reductions and divisions, the GEMM by the
// first loads of its weights. k_gemv_pro runs both in one launch: every block
// first issues the loads of its weight slice (registers), then computes the
// operand rows itself into LDS (the producing row kernel's body, the same
// integers: one wave per row, wave-wide reductions; one row uses the whole
// block), so the weight latency hides behind the row chain and the operand
// never goes through global memory. Every block recomputes the same rows;
// block (0, 0) alone stores the rows' other outputs (residual, row scales).
//
// Block: 512 threads, NB 16-column groups x one K split of the product; wave
// w covers K [kbeg + 64 NI w, + 64 NI) with NI MFMA steps (kchunk = 512 NI)
// for each group. The 8 waves' int32 accumulators are summed through LDS
// (exact).

constexpr int PRO_THREADS = 512;
constexpr int PRO_ROWS = 8;
constexpr int PRO_WAVES = PRO_THREADS / 64;

struct ProGemv {
  const int8_t* B;  // [N][K] weights
  int32_t* C;       // [ksplit][R][N] int32 partials, split_stride elements apart
  int R, N, K, kchunk;
  i64 split_stride;
};

template <int CMAX, int NB>
struct ProLds {
  int8_t a[16][CMAX + 16];  // operand rows (rows >= R unused), padded against bank conflicts
  int32_t red[PRO_WAVES - 1][NB][4][64];
  i64 red_buf[32];
};

constexpr int PRO_MAX_EXT = 8;  // statistics entries per row (MergeArgs::n_ext)

// PRO 4: the operand rows of the merge (merge_rowcol_row's integers, nsplit
// 1) over the block's K range [kbeg, kbeg + 512 NI) only, their row
// statistics taken from a.ext instead of row reductions, so every value is
// elementwise: lane r < R reduces row r's entries and fits its divisor once,
// each wave then quantises 64 NI columns of every row. A row outside the
// estimate tiers (extremes beyond merge_shift_ext's range, or a2 = 2^46) is
// merged in full by merge_rowcol_row over the whole block. Lead: (am, ak)
// stored.
template <int NI, bool ONE, int CMAX>
__device__ __forceinline__ void merge_rows_ext(const MergeArgs& a, int R, int kbeg, int8_t* a8,
                                               int stride, i64* red_buf) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int K = a.C;
  // this lane's columns and their factors; every row's values, loaded first
  // (buffer views: rows >= R and columns >= K read 0)
  constexpr int RMAX = ONE ? 1 : PRO_ROWS;  // rows the launch may hold
  int col[NI];
  i64 om[NI];
  i64 x[RMAX][NI];
  {
    const bufv_t ov = buf_view(a.os_m, (i64)K * 8);
    const bufv_t av = buf_view(a.attn, (i64)R * K * 8);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      col[i] = kbeg + (wave * NI + i) * 64 + lane;
      om[i] = buf_ld_i64(ov, col[i] < K ? (uint32_t)col[i] * 8 : BUF_OOB);
#pragma unroll
      for (int r = 0; r < RMAX; ++r)
        x[r][i] = buf_ld_i64(av, (r < R && col[i] < K) ? (uint32_t)(r * K + col[i]) * 8 : BUF_OOB);
    }
  }
  // row statistics: lane r < R takes row r (other lanes row 0, unused);
  // one view of the whole array (a descriptor must be wave-uniform: a
  // per-lane base would make the compiler loop over the lanes' values)
  v4i q[PRO_MAX_EXT];
  {
    const int rr = lane < R ? lane : 0;
    const bufv_t ev = buf_view(a.ext, (i64)R * a.n_ext * 16);
    const uint32_t rowoff = (uint32_t)(rr * a.n_ext) * 16;
#pragma unroll
    for (int e = 0; e < PRO_MAX_EXT; ++e)
      q[e] = buf_ld_16<v4i>(ev, e < a.n_ext ? rowoff + (uint32_t)e * 16 : BUF_OOB);
  }
  // (every load above is issued before any is used)
  __builtin_amdgcn_sched_barrier(0);
  i64 vmax = 0, nmin = -1;
#pragma unroll
  for (int e = 0; e < PRO_MAX_EXT; ++e) {
    const i64 hi = (i64)(((u64)(uint32_t)q[e][1] << 32) | (uint32_t)q[e][0]);
    const i64 nm = (i64)(((u64)(uint32_t)q[e][3] << 32) | (uint32_t)q[e][2]);
    vmax = imax(vmax, hi);
    nmin = imax(nmin, e < a.n_ext ? nm : (i64)-1);
  }
  // the estimate tiers of merge_rowcol_row (a2 < 2^46: rhad_est, plain
  // below 2^43, corrected above); a row past them (a2 = 2^46 after rounding,
  // or extremes beyond 2^62) takes the fallback below
  i64 sh = 0, a2 = 1;
  const bool fast = merge_shift_ext(vmax, ~nmin, &sh, &a2) && a2 < ((i64)1 << 46);
  const uint32_t fastm = (uint32_t)__ballot(fast) & ((1u << R) - 1u);
  const DivEst D = make_divest(fast ? a2 : 1, 127.0);
  if (a.am && lane < R && fast) merge_row_scale(a, lane, a2, sh);
#pragma unroll
  for (int r = 0; r < RMAX; ++r) {
    if (r >= R || !((fastm >> r) & 1u)) continue;  // wave-uniform
    // one row: every lane computed row 0's values; else lane r's
    const i64 shr = ONE ? sh : readlane64(sh, r), a2r = ONE ? a2 : readlane64(a2, r);
    DivEst Dr = D;
    if (!ONE) {
      Dr.r = __longlong_as_double(readlane64(__double_as_longlong(D.r), r));
      Dr.k = __longlong_as_double(readlane64(__double_as_longlong(D.k), r));
    }
    int8_t* const row = a8 + r * stride;
    if (DI_LIKELY(a2r < ((i64)1 << 43))) {
#pragma unroll
      for (int i = 0; i < NI; ++i)
        if (col[i] < K) row[col[i]] = (int8_t)rhad_est_signed(rshift_round(wmul(x[r][i], om[i]), shr), Dr);
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i)
        if (col[i] < K)
          row[col[i]] = (int8_t)rhad_est_corr_signed(rshift_round(wmul(x[r][i], om[i]), shr), 127, a2r, Dr);
    }
  }
  if (DI_UNLIKELY(fastm != (1u << R) - 1u)) {
    // rows past the estimate tiers: the row kernel's own reductions, one row
    // at a time over the whole block (few registers per thread)
    MergeArgs m = a;
    m.a8 = a8;
    m.a8_stride = stride;
    BlockRedT<PRO_THREADS / 64> red{red_buf, 0, PRO_THREADS};
    for (int r = 0; r < R; ++r)
      if (!((fastm >> r) & 1u)) merge_rowcol_row<CMAX / PRO_THREADS>(m, r, red);  // uniform
  }
}

// PRO 1: residual_normq (ResNormArgs, mode 1, C = K <= CMAX); 2: merge_rowcol
// (MergeArgs, C = K <= CMAX); 3: swiglu_quant (SwigluArgs, I = K <= CMAX, one
// row only); 4: merge_rows_ext (MergeArgs with ext). ONE: a single row,
// computed by the whole block (else one wave per row); separate
// instantiations keep the one-row kernel free of the wave path's registers.
template <int PRO, int CMAX, int NI, int NB, bool ONE>
__global__ __launch_bounds__(PRO_THREADS) void k_gemv_pro(ProGemv g, ResNormArgs ra, MergeArgs ma,
                                                         SwigluArgs sa, Prefetch pf) {
  keep_hidden_args();
  __shared__ __attribute__((aligned(16))) ProLds<CMAX, NB> L;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int bx = blockIdx.x, by = blockIdx.y;
  const int kbeg = by * g.kchunk;
  // 1. this wave's weight fragments, loaded before anything else: a buffer
  // view of the block's weight rows below N (a row past N reads 0, a slice
  // past K gets an offset beyond the view), so the loads are unconditional
  v4i b[NB][NI];
  {
    const int c0 = bx * NB * 16;
    const bufv_t bv = buf_view(g.B + (i64)c0 * g.K, (i64)min(NB * 16, g.N - c0) * g.K);
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      const uint32_t rowoff = (uint32_t)((n * 16 + (lane & 15)) * g.K);
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int k = kbeg + (wave * NI + i) * 64 + (lane >> 4) * 16;
        b[n][i] = buf_ld_16<v4i>(bv, k < g.K ? rowoff + (uint32_t)k : BUF_OOB);
      }
    }
  }
  const PrefetchHold ph = prefetch_issue(pf, by == 0 ? (i64)bx * PRO_THREADS + tid : (i64)-1);
  // 2. the operand rows into LDS
  const bool lead = bx == 0 && by == 0;  // the block that stores the row outputs
  if (PRO == 1) {
    ResNormArgs a = ra;
    a.x8 = &L.a[0][0];
    a.x8_stride = CMAX + 16;
    if (!lead) {
      a.h = nullptr;
      a.k_res = nullptr;
      a.xm = nullptr;
      a.xk = nullptr;
    }
    if (ONE) {
      BlockRedT<PRO_THREADS / 64> red{L.red_buf, 0, PRO_THREADS};
      residual_normq_row<CMAX / PRO_THREADS, decltype(red), 1>(a, 0, red);
    } else if (wave < g.R) {
      WaveRed red;
      residual_normq_row<CMAX / 64, WaveRed, 1>(a, wave, red);
    }
  } else if (PRO == 3) {
    SwigluArgs a = sa;
    a.y8 = &L.a[0][0];  // row 0 (the entry point takes one row)
    if (!lead) {
      a.ym = nullptr;
      a.yk = nullptr;
    }
    if (ONE) {
      BlockRedT<PRO_THREADS / 64> red{L.red_buf, 0, PRO_THREADS};
      swiglu_quant_row<CMAX / PRO_THREADS>(a, 0, red);
    }
  } else if constexpr (PRO == 4) {
    MergeArgs a = ma;
    if (!lead) {
      a.am = nullptr;
      a.ak = nullptr;
    }
    merge_rows_ext<NI, ONE, CMAX>(a, g.R, kbeg, &L.a[0][0], CMAX + 16, L.red_buf);
  } else {
    MergeArgs a = ma;
    a.a8 = &L.a[0][0];
    a.a8_stride = CMAX + 16;
    if (!lead) {
      a.am = nullptr;
      a.ak = nullptr;
    }
    if (ONE) {
      BlockRedT<PRO_THREADS / 64> red{L.red_buf, 0, PRO_THREADS};
      merge_rowcol_row<CMAX / PRO_THREADS>(a, 0, red);
    } else if (wave < g.R) {
      WaveRed red;
      merge_rowcol_row<CMAX / 64>(a, wave, red);
    }
  }
  __syncthreads();
  // 3. MFMAs: A rows from LDS (row lane % 16), B from registers
  v4i acc[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n) acc[n] = zero4();
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int k = kbeg + (wave * NI + i) * 64 + (lane >> 4) * 16;
    const v4i a = k < g.K ? *(const v4i*)(&L.a[lane & 15][k]) : zero4();
#pragma unroll
    for (int n = 0; n < NB; ++n) acc[n] = mfma16(a, b[n][i], acc[n]);
  }
  if (wave > 0) {
#pragma unroll
    for (int n = 0; n < NB; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) L.red[wave - 1][n][r][lane] = acc[n][r];
  }
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    const int col = (bx * NB + n) * 16 + (lane & 15);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int32_t s = acc[n][r];
#pragma unroll
      for (int w = 0; w < PRO_WAVES - 1; ++w) s += L.red[w][n][r][lane];
      const int row = (lane >> 4) * 4 + r;
      if (row < g.R && col < g.N) g.C[by * g.split_stride + (i64)row * g.N + col] = s;
    }
  }
  prefetch_keep(pf, ph);
}

// One launch of k_gemv_pro.
template <int PRO, int CMAX, bool ONE>
void launch_pro1(const ProGemv& g, int ni, int nb, dim3 grid, const ResNormArgs& ra,
                 const MergeArgs& ma, const SwigluArgs& sa, const Prefetch& pf, hipStream_t s) {
  const dim3 block(PRO_THREADS);
#define DI_PRO_LAUNCH(NI_, NB_) \
  hipLaunchKernelGGL((k_gemv_pro<PRO, CMAX, NI_, NB_, ONE>), grid, block, 0, s, g, ra, ma, sa, pf)
  if (nb == 1) {
    if (ni == 1) DI_PRO_LAUNCH(1, 1);
    else DI_PRO_LAUNCH(2, 1);
  } else {
    if (ni == 1) DI_PRO_LAUNCH(1, 2);
    else DI_PRO_LAUNCH(2, 2);
  }
#undef DI_PRO_LAUNCH
}

template <int PRO, int CMAX>
void launch_pro(const ProGemv& g, int ni, int ksplit, const ResNormArgs& ra, const MergeArgs& ma,
                const SwigluArgs& sa, const Prefetch& pf, hipStream_t s) {
  // NB = 2 when one column group per block would need more blocks than the
  // chip has CUs (measured at one row, c3 b1: 1.635 ms per step against
  // 1.670 with one group per block and 1.677 with up to four)
  const int groups = (g.N + 15) / 16;
  const int nb = (long)groups * ksplit > 256 ? 2 : 1;
  const dim3 grid((groups + nb - 1) / nb, ksplit);
  if (g.R == 1) {
    launch_pro1<PRO, CMAX, true>(g, ni, nb, grid, ra, ma, sa, pf, s);
  } else {
    if constexpr (PRO != 3) launch_pro1<PRO, CMAX, false>(g, ni, nb, grid, ra, ma, sa, pf, s);
  }
}

}  // namespace

#define DI_VPT_DISPATCH(vpt, KERNEL, GRID, STREAM, ...)                                  \
  switch (vpt) {                                                                         \
    case 1: hipLaunchKernelGGL(KERNEL<1>, GRID, dim3(RT), 0, STREAM, __VA_ARGS__); break;   \
    case 2: hipLaunchKernelGGL(KERNEL<2>, GRID, dim3(RT), 0, STREAM, __VA_ARGS__); break;   \
    case 4: hipLaunchKernelGGL(KERNEL<4>, GRID, dim3(RT), 0, STREAM, __VA_ARGS__); break;   \
    case 8: hipLaunchKernelGGL(KERNEL<8>, GRID, dim3(RT), 0, STREAM, __VA_ARGS__); break;   \
    case 12: hipLaunchKernelGGL(KERNEL<12>, GRID, dim3(RT), 0, STREAM, __VA_ARGS__); break; \
    case 16: hipLaunchKernelGGL(KERNEL<16>, GRID, dim3(RT), 0, STREAM, __VA_ARGS__); break; \
    default: return DI_ERANGE;                                                            \
  }

#define DI_WIDE_DISPATCH(C, KERNEL, GRID, STREAM, ARGS)                                      \
  do {                                                                                       \
    int thr_, vpt_;                                                                          \
    if (!wide_shape((C), &thr_, &vpt_)) return DI_ENOSYS;                                    \
    (ARGS).nt = thr_;                                                                        \
    switch (vpt_) {                                                                          \
      case 1: hipLaunchKernelGGL(KERNEL<1>, GRID, dim3(thr_), 0, STREAM, ARGS); break;      \
      case 2: hipLaunchKernelGGL(KERNEL<2>, GRID, dim3(thr_), 0, STREAM, ARGS); break;      \
      case 3: hipLaunchKernelGGL(KERNEL<3>, GRID, dim3(thr_), 0, STREAM, ARGS); break;      \
      default: hipLaunchKernelGGL(KERNEL<4>, GRID, dim3(thr_), 0, STREAM, ARGS); break;     \
    }                                                                                        \
  } while (0)

// Row kernels over many rows (prefill, R > 64) run 256-thread blocks with up
// to 16 columns per thread: the per-row work (reductions, scale fits,
// divisors) is then shared by 4 waves instead of up to 16, and more rows fit
// on a CU at once. Decode-sized calls keep the wide blocks, which shorten
// the per-row serial chain. ARGS.nt tells the kernel its block size.
#define DI_ROWS_DISPATCH(R, C, KERNEL, GRID, STREAM, ARGS)                                      \
  do {                                                                                          \
    if ((R) > 64) {                                                                             \
      const int v_ = ((C) + 255) / 256;                                                         \
      (ARGS).nt = 256;                                                                          \
      if (v_ <= 4) hipLaunchKernelGGL((KERNEL<4, 256>), GRID, dim3(256), 0, STREAM, ARGS);      \
      else if (v_ <= 8) hipLaunchKernelGGL((KERNEL<8, 256>), GRID, dim3(256), 0, STREAM, ARGS); \
      else if (v_ <= 12) hipLaunchKernelGGL((KERNEL<12, 256>), GRID, dim3(256), 0, STREAM, ARGS); \
      else if (v_ <= 16) hipLaunchKernelGGL((KERNEL<16, 256>), GRID, dim3(256), 0, STREAM, ARGS); \
      else return DI_ENOSYS;                                                                    \
    } else {                                                                                    \
      DI_WIDE_DISPATCH(C, KERNEL, GRID, STREAM, ARGS);                                          \
    }                                                                                           \
  } while (0)

// A decode row launch with the next GEMM's warming blocks in front of the
// rows (block ids 0 .. L2WARM_BLOCKS - 1: the kernel tells them apart by the
// block id alone, so the rows' argument loads are not held up by a test on
// an argument) when ARGS.warm asks for them and the shape takes four columns
// per thread (every model shape); else the plain row launch.
#define DI_WARM_OR_ROWS(R, C, KERNEL, STREAM, ARGS)                                          \
  do {                                                                                       \
    int thr_, vpt_;                                                                          \
    if ((ARGS).warm.nwarm > 0 && (R) <= 64 && wide_shape((C), &thr_, &vpt_) && vpt_ == 4) { \
      (ARGS).nt = thr_;                                                                      \
      const dim3 g_(L2WARM_BLOCKS + (R));                                                    \
      switch (thr_) { /* the model's widths at their exact thread count */                   \
        case 256: hipLaunchKernelGGL((KERNEL<4, 256, true>), g_, dim3(256), 0, STREAM, ARGS); break; \
        case 512: hipLaunchKernelGGL((KERNEL<4, 512, true>), g_, dim3(512), 0, STREAM, ARGS); break; \
        case 768: hipLaunchKernelGGL((KERNEL<4, 768, true>), g_, dim3(768), 0, STREAM, ARGS); break; \
        default:                                                                             \
          hipLaunchKernelGGL((KERNEL<4, RT_WIDE, true>), g_, dim3(thr_), 0, STREAM, ARGS);   \
      }                                                                                      \
    } else {                                                                                 \
      DI_ROWS_DISPATCH(R, C, KERNEL, dim3(R), STREAM, ARGS);                                 \
    }                                                                                        \
  } while (0)

// The wave-per-row launch of a prefill-sized residual / norm-quant call
// (R > 64 rows of C = 512 or 1024 columns); false: the caller launches the
// block-per-row kernel.
template <int MODE>
static bool rows_wave_launch(int R, int C, hipStream_t s, ResNormArgs& a) {
#ifdef ROWS_BLOCK
  return false;
#endif
  if (R <= 64 || (C != 512 && C != 1024)) return false;
  a.nt = 64;
  const dim3 grid((unsigned)((R + 3) / 4));
  if (C == 1024) hipLaunchKernelGGL((k_residual_normq_w<16, MODE>), grid, dim3(256), 0, s, a, R);
  else hipLaunchKernelGGL((k_residual_normq_w<8, MODE>), grid, dim3(256), 0, s, a, R);
  return true;
}

extern "C" {

// ---------------------------------------------------------------- model path

// Warming blocks for the skinny GEMM that follows a decode row launch of R
// rows (none for prefill-sized launches or without a next weight matrix).
static L2Warm warm_for(int R, const int8_t* next_w, int next_n, int next_k, int next_ksplit) {
  if (R > 64) return L2Warm{};
  return make_l2warm(next_w, next_n, next_k, next_ksplit, 0);
}


int detllm_embed_normq(const int64_t* ids, int R, int C, int64_t vocab, const int8_t* e8,
                       const int64_t* em, const int64_t* ek, int32_t* h, int64_t* k_res,
                       const int64_t* sm_m, int64_t sm_k, int8_t* x8, int64_t* xm, int64_t* xk,
                       int32_t* err, hipStream_t s) {
  if (R <= 0) return DI_OK;
  if (C <= 0 || vocab <= 0 || !ids || !e8 || !em || !ek || !h || !k_res) return DI_EINVAL;
  ResNormArgs a{};
  a.C = C; a.mode = 0; a.vocab = vocab; a.ids = ids; a.e8 = e8; a.em = em; a.ek = ek;
  a.h = h; a.k_res = k_res; a.sm_m = sm_m; a.sm_k = sm_k; a.x8 = x8; a.xm = xm; a.xk = xk;
  a.err = err;
  DI_ROWS_DISPATCH(R, C, k_residual_normq, dim3(R), s, a);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_residual_normq(const int32_t* P, int nsplit, int64_t split_stride, int R, int C,
                          const int64_t* row_m, const int64_t* row_k, const int64_t* col_m,
                          int64_t col_k, int tb, int32_t* h, int64_t* k_res, const int64_t* sm_m,
                          int64_t sm_k, int8_t* x8, int64_t* xm, int64_t* xk,
                          const int8_t* next_w, int next_n, int next_k, int next_ksplit,
                          int row_fit, hipStream_t s) {
  if (R <= 0) return DI_OK;
  if (C <= 0 || nsplit < 1 || !P || !row_m || !row_k || !col_m || !h || !k_res ||
      (row_fit != 0 && row_fit != 1))
    return DI_EINVAL;
  ResNormArgs a{};
  a.C = C; a.mode = 1; a.P = P; a.nsplit = nsplit; a.split_stride = split_stride;
  a.row_m = row_m; a.row_k = row_k; a.row_fit = row_fit;
  a.col_m = col_m; a.col_k = col_k; a.tb = tb;
  a.h = h; a.k_res = k_res; a.sm_m = sm_m; a.sm_k = sm_k; a.x8 = x8; a.xm = xm; a.xk = xk;
  a.warm = warm_for(R, next_w, next_n, next_k, next_ksplit);
  if (!rows_wave_launch<1>(R, C, s, a)) DI_WARM_OR_ROWS(R, C, k_residual_add_normq, s, a);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

// Prefetch ranges of the fused GEMVs (n a multiple of 4, 0 = unused)
static bool pro_prefetch(const void* pf0, int64_t n0, const void* pf1, int64_t n1, Prefetch* pf) {
  *pf = Prefetch{};
  const void* ps[2] = {pf0, pf1};
  const int64_t ns[2] = {n0, n1};
  for (int i = 0; i < 2; ++i) {
    if (ns[i] < 0 || (ns[i] > 0 && (!ps[i] || (ns[i] & 3) != 0 || ((uintptr_t)ps[i] & 3) != 0)))
      return false;
    pf->p[i] = (const int8_t*)ps[i];
    pf->n[i] = ps[i] ? ns[i] : 0;
  }
  return true;
}

// The product's K split (detllm_igemv_plan) and the MFMA steps per wave it
// gives, or 0 when the fused kernel does not cover the shape.
static int pro_steps(int K, int ksplit, int* kchunk) {
  if (K <= 0 || K % 16 != 0 || ksplit < 1) return 0;
  *kchunk = gemv_kchunk(K, ksplit);
  if ((K + *kchunk - 1) / *kchunk != ksplit || *kchunk % (PRO_THREADS) != 0) return 0;
  const int ni = *kchunk / PRO_THREADS;
  return ni <= 2 ? ni : 0;
}

int detllm_igemv_resnormq(const int8_t* W, int32_t* C, int R, int N, int K, int ksplit,
                          int64_t split_stride, const int32_t* P, int nsplit,
                          int64_t p_split_stride, const int64_t* row_m, const int64_t* row_k,
                          const int64_t* col_m, int64_t col_k, int tb, const int32_t* h_in,
                          const int64_t* k_res_in, int32_t* h_out, int64_t* k_res_out,
                          const int64_t* sm_m, int64_t sm_k, int64_t* xm, int64_t* xk,
                          const void* pf0, int64_t n0, const void* pf1, int64_t n1,
                          hipStream_t s) {
  if (R <= 0 || N <= 0) return DI_OK;
  if (R > PRO_ROWS || K > 1024 || !W || !C || !P || nsplit < 1 || !row_m || !row_k || !col_m ||
      !h_in || !k_res_in || !h_out || !k_res_out || !xm || !xk || (void*)h_in == (void*)h_out ||
      (void*)k_res_in == (void*)k_res_out || (ksplit > 1 && split_stride < (int64_t)R * N))
    return DI_EINVAL;
  int kchunk = 0;
  const int ni = pro_steps(K, ksplit, &kchunk);
  if (ni == 0) return DI_ENOSYS;
  Prefetch pf;
  if (!pro_prefetch(pf0, n0, pf1, n1, &pf)) return DI_EINVAL;
  ResNormArgs a{};
  a.C = K; a.mode = 1; a.P = P; a.nsplit = nsplit; a.split_stride = p_split_stride;
  a.row_m = row_m; a.row_k = row_k; a.col_m = col_m; a.col_k = col_k; a.tb = tb;
  a.h_in = h_in; a.k_res_in = k_res_in; a.h = h_out; a.k_res = k_res_out; a.sm_m = sm_m;
  a.sm_k = sm_k; a.xm = xm; a.xk = xk;
  const ProGemv g{W, C, R, N, K, kchunk, (i64)split_stride};
  launch_pro<1, 1024>(g, ni, ksplit, a, MergeArgs{}, SwigluArgs{}, pf, s);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_igemv_merge(const int8_t* W, int32_t* C, int R, int N, int K, int ksplit,
                       int64_t split_stride, const int64_t* attn, int nsplit,
                       int64_t a_split_stride, const int64_t* os_m, int64_t os_k,
                       const int64_t* col_m, int64_t col_k, int64_t* am, int64_t* ak,
                       const void* pf0, int64_t n0, const void* pf1, int64_t n1, hipStream_t s) {
  if (R <= 0 || N <= 0) return DI_OK;
  if (R > PRO_ROWS || K > 2048 || !W || !C || !attn || nsplit < 1 || !os_m || !am || !ak ||
      (ksplit > 1 && split_stride < (int64_t)R * N))
    return DI_EINVAL;
  int kchunk = 0;
  const int ni = pro_steps(K, ksplit, &kchunk);
  if (ni == 0) return DI_ENOSYS;
  Prefetch pf;
  if (!pro_prefetch(pf0, n0, pf1, n1, &pf)) return DI_EINVAL;
  MergeArgs m{};
  m.C = K; m.attn = attn; m.nsplit = nsplit; m.split_stride = a_split_stride; m.os_m = os_m;
  m.os_k = os_k; m.col_m = col_m; m.col_k = col_k; m.am = am; m.ak = ak;
  const ProGemv g{W, C, R, N, K, kchunk, (i64)split_stride};
  launch_pro<2, 2048>(g, ni, ksplit, ResNormArgs{}, m, SwigluArgs{}, pf, s);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_igemv_merge_ext(const int8_t* W, int32_t* C, int R, int N, int K, int ksplit,
                           int64_t split_stride, const int64_t* attn, const int64_t* om,
                           int64_t os_k, int64_t col_k, const int64_t* ext, int n_ext,
                           int64_t* am, int64_t* ak, int defer_fit, const void* pf0, int64_t n0,
                           const void* pf1, int64_t n1, hipStream_t s) {
  if (R <= 0 || N <= 0) return DI_OK;
  if (R > PRO_ROWS || K > 2048 || !W || !C || !attn || !om || !ext || n_ext < 1 ||
      n_ext > PRO_MAX_EXT || !am || !ak || (defer_fit != 0 && defer_fit != 1) ||
      (ksplit > 1 && split_stride < (int64_t)R * N))
    return DI_EINVAL;
  int kchunk = 0;
  const int ni = pro_steps(K, ksplit, &kchunk);
  if (ni == 0) return DI_ENOSYS;
  Prefetch pf;
  if (!pro_prefetch(pf0, n0, pf1, n1, &pf)) return DI_EINVAL;
  MergeArgs m{};
  m.C = K; m.attn = attn; m.nsplit = 1; m.split_stride = 0; m.os_m = om; m.os_k = os_k;
  m.col_m = nullptr; m.col_k = col_k; m.am = am; m.ak = ak; m.defer_fit = defer_fit;
  m.ext = ext; m.n_ext = n_ext;
  const ProGemv g{W, C, R, N, K, kchunk, (i64)split_stride};
  launch_pro<4, 2048>(g, ni, ksplit, ResNormArgs{}, m, SwigluArgs{}, pf, s);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_igemv_swiglu(const int8_t* W, int32_t* C, int N, int K, int ksplit,
                        int64_t split_stride, const int32_t* P, int nsplit, int64_t p_split_stride,
                        const int64_t* xm, const int64_t* xk, const int64_t* gate_m,
                        int64_t gate_k, const int64_t* up_m, int64_t up_k, const int64_t* ds_m,
                        int64_t ds_k, int64_t* ym, int64_t* yk, int defer_fit, const void* pf0,
                        int64_t n0, const void* pf1, int64_t n1, hipStream_t s) {
  if (N <= 0) return DI_OK;
  if (K <= 0 || K > 3072 || K % 512 != 0 || !W || !C || !P || nsplit < 1 || !xm || !xk ||
      !gate_m || !up_m || !ds_m || !ym || !yk || (defer_fit != 0 && defer_fit != 1) ||
      (ksplit > 1 && split_stride < (int64_t)N))
    return DI_EINVAL;
  int kchunk = 0;
  const int ni = pro_steps(K, ksplit, &kchunk);
  if (ni == 0) return DI_ENOSYS;
  Prefetch pf;
  if (!pro_prefetch(pf0, n0, pf1, n1, &pf)) return DI_EINVAL;
  SwigluArgs a{};
  a.I = K; a.nt = PRO_THREADS; a.P = P; a.nsplit = nsplit; a.split_stride = p_split_stride;
  a.xm = xm; a.xk = xk; a.gate_m = gate_m; a.gate_k = gate_k; a.up_m = up_m; a.up_k = up_k;
  a.ds_m = ds_m; a.ds_k = ds_k; a.ym = ym; a.yk = yk; a.defer_fit = defer_fit;
  const ProGemv g{W, C, 1, N, K, kchunk, (i64)split_stride};
  launch_pro<3, 3072>(g, ni, ksplit, ResNormArgs{}, MergeArgs{}, a, pf, s);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_norm_quant(const int32_t* h, int R, int C, const int64_t* sm_m, int64_t sm_k,
                      int8_t* x8, int64_t* xm, int64_t* xk, hipStream_t s) {
  if (R <= 0) return DI_OK;
  if (C <= 0 || !h || !x8 || !xm || !xk) return DI_EINVAL;
  ResNormArgs a{};
  a.C = C; a.mode = 2; a.h = const_cast<int32_t*>(h); a.sm_m = sm_m; a.sm_k = sm_k;
  a.x8 = x8; a.xm = xm; a.xk = xk;
  if (!rows_wave_launch<2>(R, C, s, a)) DI_ROWS_DISPATCH(R, C, k_residual_normq, dim3(R), s, a);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_swiglu_quant(const int32_t* P, int nsplit, int64_t split_stride, int R, int I,
                        const int64_t* xm, const int64_t* xk, const int64_t* gate_m,
                        int64_t gate_k, const int64_t* up_m, int64_t up_k, const int64_t* ds_m,
                        int64_t ds_k, int8_t* y8, int64_t* ym, int64_t* yk,
                        const int8_t* next_w, int next_n, int next_k, int next_ksplit,
                        int defer_fit, hipStream_t s) {
  if (R <= 0) return DI_OK;
  if (I <= 0 || nsplit < 1 || !P || !xm || !xk || !gate_m || !up_m || !ds_m || !y8 || !ym ||
      !yk || (defer_fit != 0 && defer_fit != 1))
    return DI_EINVAL;
  SwigluArgs a{};
  a.I = I; a.P = P; a.nsplit = nsplit; a.split_stride = split_stride; a.xm = xm; a.xk = xk;
  a.gate_m = gate_m; a.gate_k = gate_k; a.up_m = up_m; a.up_k = up_k; a.ds_m = ds_m;
  a.ds_k = ds_k; a.y8 = y8; a.ym = ym; a.yk = yk; a.defer_fit = defer_fit;
  a.warm = warm_for(R, next_w, next_n, next_k, next_ksplit);
#ifdef SWIGLU_PREFILL_WIDE
  if (R > 64) {
    DI_WIDE_DISPATCH(I, k_swiglu_quant, dim3(R), s, a);
    DI_LAUNCH_CHECK();
    return DI_OK;
  }
#endif
  DI_WARM_OR_ROWS(R, I, k_swiglu_quant, s, a);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_merge_rowcol(const int64_t* attn, int nsplit, int64_t split_stride, int R, int C,
                        const int64_t* os_m, int64_t os_k, const int64_t* col_m, int64_t col_k,
                        int8_t* a8, int64_t* am, int64_t* ak, const int8_t* next_w,
                        int next_n, int next_k, int next_ksplit, int defer_fit, hipStream_t s) {
  if (R <= 0) return DI_OK;
  if (C <= 0 || nsplit < 1 || !attn || !os_m || !col_m || !a8 || !am || !ak ||
      (defer_fit != 0 && defer_fit != 1))
    return DI_EINVAL;
  MergeArgs a{};
  a.C = C; a.attn = attn; a.nsplit = nsplit; a.split_stride = split_stride; a.os_m = os_m;
  a.os_k = os_k; a.col_m = col_m; a.col_k = col_k; a.a8 = a8; a.am = am; a.ak = ak;
  a.defer_fit = defer_fit;
  a.warm = warm_for(R, next_w, next_n, next_k, next_ksplit);
  DI_WARM_OR_ROWS(R, C, k_merge_rowcol, s, a);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_merge_ext(const int64_t* attn, int R, int C, const int64_t* om, int64_t os_k,
                     int64_t col_k, const int64_t* ext, int n_ext, int8_t* a8, int64_t* am,
                     int64_t* ak, const int8_t* next_w, int next_n, int next_k, int next_ksplit,
                     int defer_fit, hipStream_t s) {
  if (R <= 0) return DI_OK;
  if (C <= 0 || C > 2048 || R > 64 || !attn || !om || !ext || n_ext < 1 || n_ext > MEXT_MAX ||
      !a8 || !am || !ak || (defer_fit != 0 && defer_fit != 1))
    return DI_EINVAL;
  MergeArgs a{};
  a.C = C; a.nt = 256; a.attn = attn; a.nsplit = 1; a.split_stride = 0; a.os_m = om;
  a.os_k = os_k; a.col_m = nullptr; a.col_k = col_k; a.a8 = a8; a.am = am; a.ak = ak;
  a.defer_fit = defer_fit; a.ext = ext; a.n_ext = n_ext;
  a.warm = warm_for(R, next_w, next_n, next_k, next_ksplit);
  const int pieces = (C + 255) / 256;
  if (a.warm.nwarm > 0)
    hipLaunchKernelGGL(k_merge_ext<true>, dim3(L2WARM_BLOCKS + R * pieces), dim3(256), 0, s, a,
                       pieces);
  else
    hipLaunchKernelGGL(k_merge_ext<false>, dim3(R * pieces), dim3(256), 0, s, a, pieces);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

// One kernel for the per-step bookkeeping of a graphed decode step (a few
// bytes per row): valid[b][slot] = 1, *len_idx = slot, *nslots = slot + 1,
// pos[b] = pos0[b] + step.
int detllm_decode_prologue(uint8_t* valid, int64_t valid_stride, int B, int64_t slot,
                           int64_t* len_idx, int64_t* nslots, int64_t* pos, const int64_t* pos0,
                           int64_t step, hipStream_t s) {
  if (B <= 0) return DI_OK;
  if (!valid || !len_idx || !nslots || !pos || !pos0 || slot < 0 || slot >= valid_stride ||
      step < 0)
    return DI_EINVAL;
  hipLaunchKernelGGL(k_decode_prologue, dim3(1), dim3(256), 0, s, valid, valid_stride, B, slot,
                     len_idx, nslots, pos, pos0, step);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

// Per-channel divisor estimates of the static K requantisation for one layer
// (model-load time): est [n][4] = {den, up, bits of 1/den, bits of
// (floor(den/2) + 1/2) / den} from kq_m, kq_k [n] and rowk = 20 + k_norm_k.
int detllm_kq_est(const int64_t* kq_m, const int64_t* kq_k, int64_t n, int64_t rowk,
                  int64_t* est, hipStream_t s) {
  if (n <= 0) return DI_OK;
  if (!kq_m || !kq_k || !est) return DI_EINVAL;
  hipLaunchKernelGGL(k_kq_est, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, kq_m, kq_k, n,
                     rowk, est);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_qkv_epilogue(const int32_t* P, int nsplit, int64_t split_stride, int B, int T,
                        int n_q, int n_kv, const int64_t* xm, const int64_t* xk,
                        const int64_t* positions, const int64_t* q_m, int64_t q_k,
                        const int64_t* k_m, int64_t k_k, const int64_t* v_m, int64_t v_k,
                        const int64_t* q_norm_m, int64_t q_norm_k, const int64_t* k_norm_m,
                        int64_t k_norm_k, const int64_t* qs_m, int64_t qs_k,
                        const int64_t* kq_m, const int64_t* kq_k, const int64_t* ks_m,
                        const int64_t* ks_k, const int64_t* vq_m, const int64_t* vq_k,
                        const int16_t* cos_t, const int16_t* sin_t, int64_t max_pos,
                        int8_t* q8, int64_t* tpos, int64_t* dbg, int8_t* kpool,
                        int8_t* vpool, const int32_t* table, int width,
                        const int64_t* slot_base_dev, int64_t slot_base, const int64_t* kq_est,
                        int32_t* err, hipStream_t s) {
  if (B <= 0 || T <= 0) return DI_OK;
  if (n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0 || nsplit < 1 || max_pos <= 0 || !kpool ||
      !vpool || !table || width <= 0 || width > (1 << 24) || !P || !positions)
    return DI_EINVAL;
  if (!slot_base_dev && (slot_base < 0 || slot_base + T > (i64)width * DI_PAGE)) return DI_ERANGE;
  QKVArgs a{};
  a.T = T; a.n_q = n_q; a.n_kv = n_kv; a.P = P; a.nsplit = nsplit; a.split_stride = split_stride;
  a.xm = xm; a.xk = xk; a.positions = positions; a.q_m = q_m; a.k_m = k_m; a.v_m = v_m;
  a.q_k = q_k; a.k_k = k_k; a.v_k = v_k; a.q_norm_m = q_norm_m; a.k_norm_m = k_norm_m;
  a.q_norm_k = q_norm_k; a.k_norm_k = k_norm_k; a.qs_m = qs_m; a.qs_k = qs_k; a.kq_m = kq_m;
  a.kq_k = kq_k; a.ks_m = ks_m; a.ks_k = ks_k; a.vq_m = vq_m; a.vq_k = vq_k; a.cos_t = cos_t;
  a.sin_t = sin_t; a.max_pos = max_pos; a.q8 = q8; a.tpos = tpos; a.dbg = dbg;
  a.kv = KVPages{kpool, vpool, table, width, n_kv}; a.slot_base_dev = slot_base_dev;
  a.slot_base = slot_base; a.kq_est = kq_est; a.err = err;
  const int heads = n_q + 2 * n_kv;
  const int R = B * T;
  // the rows layout reads P 16 bytes at a time
  if (R > 64 && (nsplit == 1 || split_stride % 4 == 0) && ((uintptr_t)P & 15) == 0) {
    const int ngroups = (R + 3) / 4;
    const i64 waves = (i64)ngroups * heads;
    if ((waves + 3) / 4 > 0x7fffffff) return DI_ERANGE;
    hipLaunchKernelGGL(k_qkv_epilogue_rows, dim3((unsigned)((waves + 3) / 4)), dim3(RT), 0, s, a,
                       R, ngroups);
  } else {
    hipLaunchKernelGGL(k_qkv_epilogue, dim3(R, (heads + 3) / 4), dim3(RT), 0, s, a);
  }
  DI_LAUNCH_CHECK();
  return DI_OK;
}

// ---------------------------------------------------------------- op level

int detllm_op_quant_i8_pertoken(const int64_t* x, const int64_t* m, const int64_t* k, int R,
                                int C, int8_t* x8, int64_t* mo, int64_t* ko, hipStream_t s) {
  if (R <= 0) return DI_OK;
  const int vpt = pick_vpt(C);
  DI_VPT_DISPATCH(vpt, k_op_quant, dim3(R), s, x, m, k, C, x8, mo, ko);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_op_requant_i32_common(const int64_t* P, const int64_t* row_k, const int64_t* col_m,
                                 int G, int64_t col_k, int tb, int R, int C, int32_t* y,
                                 int64_t* ko, hipStream_t s) {
  if (R <= 0) return DI_OK;
  if (G < 1) return DI_EINVAL;
  const int vpt = pick_vpt(C);
  DI_VPT_DISPATCH(vpt, k_op_requant_common, dim3(R), s, P, row_k, col_m, G, col_k, tb, C, y, ko);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_op_requant_i8_rowcol(const int64_t* P, const int64_t* row_m, const int64_t* row_k,
                                const int64_t* col_m, int64_t col_k, int R, int C, int8_t* y8,
                                int64_t* mo, int64_t* ko, hipStream_t s) {
  if (R <= 0) return DI_OK;
  const int vpt = pick_vpt(C);
  DI_VPT_DISPATCH(vpt, k_op_rowcol, dim3(R), s, P, row_m, row_k, col_m, col_k, C, y8, mo, ko);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_op_requant_i8_static(const int64_t* P, const int64_t* row_m, const int64_t* row_k,
                                const int64_t* col_m, const int64_t* col_k, const int64_t* s_m,
                                const int64_t* s_k, int64_t n, int8_t* y8, hipStream_t s) {
  if (n <= 0) return DI_OK;
  hipLaunchKernelGGL(k_op_static, dim3(grid_for(n)), dim3(256), 0, s, P, row_m, row_k, col_m,
                     col_k, s_m, s_k, n, y8);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_requant_static_cols(const int32_t* P, int nsplit, int64_t split_stride, int R, int C,
                               const int64_t* row_m, const int64_t* row_k, const int64_t* col_m,
                               int64_t col_k, int64_t s_m, int64_t s_k, int8_t* y8,
                               hipStream_t s) {
  if (R <= 0 || C <= 0) return DI_OK;
  if (nsplit < 1 || !P || !col_m || !y8) return DI_EINVAL;
  const i64 threads = (i64)R * ((C + 3) / 4);
  if ((threads + 255) / 256 > 0x7fffffff) return DI_ERANGE;
  hipLaunchKernelGGL(k_static_cols, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, P,
                     nsplit, (i64)split_stride, R, C, row_m, row_k, col_m, (i64)col_k, (i64)s_m,
                     (i64)s_k, y8);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_op_residual(int mode, const int64_t* h, const int64_t* k_res, const int64_t* d,
                       const int64_t* dm, const int64_t* dk, int R, int C, int32_t* h_out,
                       int64_t* k_out, hipStream_t s) {
  if (R <= 0) return DI_OK;
  if (mode != 0 && mode != 1) return DI_EINVAL;
  const int vpt = pick_vpt(C);
  DI_VPT_DISPATCH(vpt, k_op_residual, dim3(R), s, mode, h, k_res, d, dm, dk, C, h_out, k_out);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_op_rmsnorm(const int64_t* x, const int64_t* gamma_m, int R, int C, int32_t* y32,
                      int64_t* y64, hipStream_t s) {
  if (R <= 0) return DI_OK;
  const int vpt = pick_vpt(C);
  DI_VPT_DISPATCH(vpt, k_op_rmsnorm, dim3(R), s, x, gamma_m, C, y32, y64);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_op_softmax(const int64_t* x, const int64_t* m, const int64_t* k, const uint8_t* valid,
                      int has_clip, int64_t clip_c, int p_out_bits, int R, int C, int32_t* probs,
                      hipStream_t s) {
  if (R <= 0) return DI_OK;
  if (p_out_bits < 1 || p_out_bits > 62) return DI_EINVAL;
  const int vpt = pick_vpt(C);
  DI_VPT_DISPATCH(vpt, k_op_softmax, dim3(R), s, x, m, k, valid, has_clip, clip_c, p_out_bits, C,
                  probs);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_op_di_exp(const int64_t* x, const int64_t* m, const int64_t* k, int R, int C,
                     int64_t* res, int64_t* tpos, hipStream_t s) {
  const i64 n = (i64)R * C;
  if (n <= 0) return DI_OK;
  hipLaunchKernelGGL(k_op_di_exp, dim3(grid_for(n)), dim3(256), 0, s, x, m, k, C, n, res, tpos);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_op_swiglu(const int64_t* gate, const int64_t* gm, const int64_t* gk,
                     const int64_t* up, const int64_t* um, const int64_t* uk, int R, int C,
                     int64_t* y, int64_t* ym, int64_t* yk, hipStream_t s) {
  const i64 n = (i64)R * C;
  if (n <= 0) return DI_OK;
  hipLaunchKernelGGL(k_op_swiglu, dim3(grid_for(n)), dim3(256), 0, s, gate, gm, gk, up, um, uk,
                     C, n, y, ym, yk);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_op_rope(const int64_t* x, const int64_t* pos, const int16_t* cos_t,
                   const int16_t* sin_t, int64_t max_pos, int64_t rows, int64_t* y,
                   int32_t* err, hipStream_t s) {
  if (rows <= 0) return DI_OK;
  if (max_pos <= 0) return DI_EINVAL;
  hipLaunchKernelGGL(k_op_rope, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, x, pos, cos_t,
                     sin_t, max_pos, rows, y, err);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int detllm_op_scalar(int op, const int64_t* a, const int64_t* b, const int64_t* c, int64_t n,
                     int64_t* o1, int64_t* o2, hipStream_t s) {
  if (n <= 0) return DI_OK;
  if (op < 0 || op > 15) return DI_EINVAL;
  if (op == 6)
    hipLaunchKernelGGL(k_op_isqrt_wave, dim3(grid_for(n)), dim3(256), 0, s, a, n, o1);
  else
    hipLaunchKernelGGL(k_op_scalar, dim3(grid_for(n)), dim3(256), 0, s, op, a, b, c, n, o1, o2);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

}  // extern "C"
