// Integer semantics of DetLLM's numerical path, for host and device code.
//
// Every helper reproduces torch's CPU integer kernels, which the reference's
// CPU backend runs on (src/detllm/intmath.py:7-17 fixes the rounding rules):
//   * int64 add / sub / mul wrap modulo 2^64 (done on uint64 here, so the
//     C++ code has no signed-overflow UB);
//   * a << k is the unsigned shift, 0 when k >= 64 or k < 0;
//   * a >> k is arithmetic, k clamped to 63 (sign fill) when k >= 63 or k < 0;
//   * floor division rounds toward -inf;
//   * int64 -> int32 truncates modulo 2^32.
//
// Division by a row-invariant divisor uses a precomputed reciprocal
// r = floor((2^64 - 1) / d): q0 = mulhi64(n, r) satisfies
// floor(n/d) - 1 <= q0 <= floor(n/d) for every n < 2^64, because
// n*r/2^64 = n/d - n*(1 + ((2^64-1) mod d))/(d*2^64) and the subtracted term
// is below 1; one compare-and-increment makes it exact. This is the
// reciprocal-with-correction family of Granlund & Montgomery, "Division by
// Invariant Integers using Multiplication" (PLDI 1994), in its simplest
// one-correction form. Tested exhaustively near multiples of d on the host.
#pragma once

#include <math.h>
#include <stdint.h>

// The exact-integer estimates below rely on IEEE-correct rounding of every
// fp64/fp32 operation as written: no reassociation, no reciprocal
// substitution, no contraction of a separate multiply and add into an fma.
#if defined(__FAST_MATH__) || defined(__FINITE_MATH_ONLY__) && __FINITE_MATH_ONLY__
#error "intops.h must not be built with -ffast-math or -ffinite-math-only"
#endif
#pragma clang fp contract(off)

#if defined(__HIPCC__) || defined(__HIP__)
#include <hip/hip_runtime.h>
#define DI_HD __host__ __device__ __forceinline__
#else
#define DI_HD static inline
#endif

// Branch hints for the exactness fallbacks (operands outside the ranges the
// fast forms are proven for): the compiler lays the unlikely side out of the
// hot instruction stream, so a launch fetches fewer instruction lines.
#define DI_LIKELY(x) __builtin_expect(!!(x), 1)
#define DI_UNLIKELY(x) __builtin_expect(!!(x), 0)

// Precondition checks of the fast forms, active in the CPU build that the
// tests run (intops_host.cpp): a violated bound aborts there. Device code
// and the host pass of the HIP library compile them away.
#if defined(__HIPCC__) || defined(__HIP__)
#define DI_HOST_CHECK(x) ((void)0)
#else
#include <stdlib.h>
#define DI_HOST_CHECK(x) ((x) ? (void)0 : abort())
#endif

typedef int64_t i64;
typedef uint64_t u64;

namespace di {

DI_HD i64 wadd(i64 a, i64 b) { return (i64)((u64)a + (u64)b); }
DI_HD i64 wsub(i64 a, i64 b) { return (i64)((u64)a - (u64)b); }
DI_HD i64 wmul(i64 a, i64 b) { return (i64)((u64)a * (u64)b); }
DI_HD i64 wneg(i64 a) { return (i64)(0ull - (u64)a); }
DI_HD i64 wabs(i64 a) { return a < 0 ? wneg(a) : a; }  // |INT64_MIN| stays INT64_MIN
DI_HD i64 imax(i64 a, i64 b) { return a > b ? a : b; }
DI_HD i64 imin(i64 a, i64 b) { return a < b ? a : b; }
// -lim < x < lim (lim >= 1) as one unsigned comparison (x + lim - 1 taken
// modulo 2^64), so a chain of operand bounds combines with & into one
// branch-free mask instead of a short-circuit branch per operand
DI_HD bool in_range(i64 x, i64 lim) { return (u64)x + (u64)(lim - 1) < (u64)(2 * lim - 1); }

// torch.bitwise_left_shift / bitwise_right_shift on int64
DI_HD i64 shl(i64 a, i64 k) { return (k < 0 || k >= 64) ? 0 : (i64)((u64)a << k); }
DI_HD i64 shr(i64 a, i64 k) { return a >> ((k < 0 || k >= 63) ? 63 : k); }

DI_HD int clz64(u64 a) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __clzll((long long)a);
#else
  return a ? __builtin_clzll(a) : 64;
#endif
}

DI_HD u64 mulhi64(u64 a, u64 b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __umul64hi(a, b);
#else
  return (u64)(((unsigned __int128)a * b) >> 64);
#endif
}

// int_prims.py:47-55 (_ilog2_loop): floor(log2 a) for a >= 2, else 0
DI_HD i64 ilog2(i64 a) { return a < 2 ? 0 : 63 - clz64((u64)a); }

// int_prims.py:31-44 (_isqrt_loop): 32 steps of the bitwise method from 2^62;
// negative inputs give 0
DI_HD i64 isqrt(i64 n) {
  i64 rem = n, c = 0, d = (i64)1 << 62;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    i64 t = wadd(c, d);
    bool ge = rem >= t;
    rem = ge ? wsub(rem, t) : rem;
    c = (c >> 1) + (ge ? d : 0);
    d >>= 2;
  }
  return c;
}

// c10::div_floor_integer semantics for b != 0
DI_HD i64 floor_div(i64 a, i64 b) {
  if (b == -1) return wneg(a);
  i64 q = a / b;
  i64 r = a - q * b;
  if (r != 0 && ((r < 0) != (b < 0))) q -= 1;
  return q;
}

// intmath.py:62-80 tensor branch: sign(a) * floor((|a| + floor(b/2)) / b)
DI_HD i64 rhad(i64 a, i64 b) {
  i64 mag = wabs(a);
  i64 q = floor_div(wadd(mag, floor_div(b, 2)), b);
  return a < 0 ? wneg(q) : q;
}

// intmath.py:120-147 — rshift_round / rshift_round_t: k == 0 is the identity
DI_HD i64 rshift_round(i64 a, i64 k) {
  if (k == 0) return a;
  i64 kp = k < 1 ? 1 : k;
  return shr(wadd(a, shl(1, kp - 1)), kp);
}

DI_HD i64 clamp_i8(i64 a) { return a < -128 ? -128 : (a > 127 ? 127 : a); }

// ---- division by a row-invariant positive divisor ----------------------
struct Recip {
  u64 d;
  u64 r;
};

DI_HD Recip make_recip(i64 d) {  // d >= 1
  Recip R;
  R.d = (u64)d;
  R.r = ~0ull / (u64)d;
  return R;
}

DI_HD u64 udiv(u64 n, const Recip& R) {
  u64 q = mulhi64(n, R.r);
  u64 rem = n - q * R.d;
  return q + (rem >= R.d ? 1 : 0);
}

// floor(a / d) for signed a and invariant d >= 1
DI_HD i64 floor_div_r(i64 a, const Recip& R) {
  if (a >= 0) return (i64)udiv((u64)a, R);
  u64 m = 0ull - (u64)a;  // |a| as unsigned (2^63 for INT64_MIN)
  return wneg((i64)(udiv(m - 1, R) + 1));
}

// rhad(a, d) for invariant d >= 1 (bit-identical to rhad above)
DI_HD i64 rhad_r(i64 a, const Recip& R) {
  i64 mag = wabs(a);
  i64 q = floor_div_r(wadd(mag, (i64)(R.d >> 1)), R);
  return a < 0 ? wneg(q) : q;
}

// rhad(a, 2^k) for k >= 0: the same integer as rhad(a, 1 << k) above (floor
// division by a positive power of two is an arithmetic shift, including the
// wrapped |INT64_MIN| case).
DI_HD i64 rhad_pow2(i64 a, int k) {
  if (k == 0) return a;
  const i64 mag = wabs(a);
  const i64 q = shr(wadd(mag, (i64)1 << (k - 1)), k);
  return a < 0 ? wneg(q) : q;
}

// ---- dyadic helpers (src/detllm/dyadic.py) -----------------------------

// dyadic.py:45-49
DI_HD i64 scaled_round_div(i64 num, i64 den, i64 e) {
  i64 d = shl(den, imax(-e, 0));
  if (d == 0) d = 1;  // unreachable on the model path (den = 127, |e| < 50)
  return rhad(shl(num, imax(e, 0)), d);
}

// dyadic.py:75-90 (bits = 16)
DI_HD void norm_scale(i64 m, i64 k, i64* m_out, i64* k_out) {
  i64 sh = 15 - ilog2(imax(m, 1));
  i64 m2 = rshift_round(shl(m, imax(sh, 0)), imax(-sh, 0));
  if (m2 >= 65536) {
    m2 = rshift_round(m2, 1);
    sh -= 1;
  }
  *m_out = m2;
  *k_out = wadd(k, sh);
}

// dyadic.py:52-72 (bits = 16)
DI_HD void fit_dyadic_ratio(i64 num, i64 den, i64* m_out, i64* e_out) {
  i64 L = ilog2(num) - ilog2(den);
  i64 e = 15 - L;
  i64 m = scaled_round_div(num, den, e);
  i64 adj = (m >= 65536 ? -1 : 0) + (m < 32768 ? 1 : 0);
  e += adj;
  if (adj != 0) m = scaled_round_div(num, den, e);
  if (m >= 65536) {
    m = rshift_round(m, 1);
    e -= 1;
  }
  *m_out = m;
  *e_out = e;
}

// fit_dyadic_ratio(num, 127): every requantisation to int8 fits its output
// scale against 127. Same integer as the generic routine. For 0 < num < 2^62
// the divisions by 127 * 2^s go through srd127 / floor_div127 below (one fp64
// fma each), whose dividends stay below 2^24 for the exponents this routine
// tries (e = 21 - ilog2(num), then one step of +-1); any other num takes the
// generic integer path.
// floor(y / 127) for 0 <= y < 2^32 from one fp64 fma: y / 127 has a
// fractional part that is a multiple of 1/127 (0, or between 1/127 and
// 126/127), and fma(y, fl(1/127), 2^-12) lies within 2^-19 of
// y / 127 + 2^-12 (fl(1/127) is within 2^-60 of 1/127, i.e. y 2^-60 < 2^-28
// absolute, and the one rounding of a result below 2^26 adds at most 2^-27),
// so its truncation is the integer quotient.
DI_HD uint32_t floor_div127(uint32_t y) {
  return (uint32_t)fma((double)y, 1.0 / 127.0, 0x1p-12);
}

DI_HD i64 srd127(i64 num, i64 e) {
  // scaled_round_div(num, 127, e), valid ONLY for the (num, e) pairs that
  // fit_dyadic_ratio_127 passes: 0 < num < 2^62 and e = 21 - ilog2(num) or
  // one step from it, so num * 2^e < 2^23. Then rhad(x, 127 * 2^s) =
  // floor(floor((x + h) / 2^s) / 127) with h = floor(127 * 2^s / 2) (s <= 42,
  // h < 2^48, so the generic routine's x + h stays below 2^63 and does not
  // wrap), and rhad(x, 127) = floor((x + 63) / 127); either dividend is below
  // 2^24 (the uint32_t cast below would truncate a larger one, and
  // floor_div127 is proven for dividends below 2^32 only).
  u64 y;
  if (e >= 0) {
    y = ((u64)num << e) + 63;
  } else {
    const int s = (int)(-e);
    const u64 h = (127ull << s) >> 1;
    y = ((u64)num + h) >> s;
  }
  DI_HOST_CHECK(y < (1ull << 24));
  return (i64)floor_div127((uint32_t)y);
}

DI_HD void fit_dyadic_ratio_127(i64 num, i64* m_out, i64* e_out) {
  const i64 lg = ilog2(num);
  if (DI_UNLIKELY(num <= 0 || lg >= 62)) {
    fit_dyadic_ratio(num, 127, m_out, e_out);
    return;
  }
  // e = 15 - (lg - 6) in [-40, 21]; num << e < 2^(lg + e + 1) <= 2^22: no wrap
  i64 e = 21 - lg;
  i64 m = srd127(num, e);
  const i64 adj = (m >= 65536 ? -1 : 0) + (m < 32768 ? 1 : 0);
  e += adj;
  if (adj != 0) m = srd127(num, e);
  if (m >= 65536) {
    m = rshift_round(m, 1);
    e -= 1;
  }
  *m_out = m;
  *e_out = e;
}

// DI-Exp per-row constant (ops/di_exp.py:29-31; model.py:355-358)
DI_HD i64 di_exp_tpos(i64 m, i64 k) {
  i64 m_f = wsub(wadd(m, shr(m, 1)), shr(m, 4));
  if (m_f == 0) m_f = 1;  // m is a normalised mantissa on the model path
  return imax(rhad(shl(1, k), m_f), 1);
}

// ops/di_exp.py:33-36 for x <= 0 in the positive domain (fused_attn.py:11-22):
// neg = -x; q = neg // tpos; rem = neg - q*tpos;
// result = (tpos - ((rem + 1) >> 1)) >> min(q, 62).
// For x > 0 (never on the path) the generic form below is used.
DI_HD i64 di_exp_generic(i64 x, i64 tpos) {
  i64 t = wneg(tpos);
  i64 q = floor_div(x, t);
  i64 r = wsub(x, wmul(q, t));
  i64 unshifted = wsub(shr(r, 1), t);
  return shr(unshifted, imin(q, 62));
}

DI_HD i64 di_exp_r(i64 x, i64 tpos, const Recip& R) {
  if (x > 0) return di_exp_generic(x, tpos);
  u64 neg = 0ull - (u64)x;
  u64 q = udiv(neg, R);
  u64 rem = neg - q * R.d;
  i64 unshifted = wsub(tpos, (i64)((rem + 1) >> 1));
  return shr(unshifted, q > 62 ? 62 : (i64)q);
}

DI_HD uint32_t mulhi32(uint32_t a, uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __umulhi(a, b);
#else
  return (uint32_t)(((u64)a * b) >> 32);
#endif
}

// DI-Exp with a row-invariant constant tpos, for non-positive arguments x =
// -neg (every argument on the model path: x = score - row max, or -|gate|).
// When tpos < 2^31 and neg < 2^32 the whole computation fits 32 bits: q =
// floor(neg / tpos) from the 32-bit reciprocal r = floor((2^32 - 1) / tpos)
// (mulhi32(neg, r) is floor(neg / tpos) or one less, by the argument given for
// the 64-bit reciprocal above, with 2^32 for 2^64), rem = neg - q tpos <
// tpos, unshifted = tpos - ((rem + 1) >> 1) in [tpos / 2, tpos], and the
// result unshifted >> min(q, 62) is 0 once q >= 31. Otherwise the 64-bit form
// runs. Bit-identical to di_exp_r(-neg, tpos, R).
struct ExpR {
  i64 tpos;
  Recip R;
  uint32_t t32, r32;
  bool fast;
};

DI_HD ExpR make_exp(i64 tpos) {  // tpos >= 1
  ExpR E;
  E.tpos = tpos;
  E.R = make_recip(tpos);
  E.fast = tpos < ((i64)1 << 31);
  E.t32 = (uint32_t)tpos;
  E.r32 = E.fast ? 0xFFFFFFFFu / E.t32 : 0u;
  return E;
}

DI_HD i64 di_exp_neg(u64 neg, const ExpR& E) {
  if (E.fast && neg <= 0xFFFFFFFFull) {
    const uint32_t n = (uint32_t)neg;
    uint32_t q = mulhi32(n, E.r32);
    uint32_t rem = n - q * E.t32;
    if (rem >= E.t32) {
      q += 1;
      rem -= E.t32;
    }
    const uint32_t unshifted = E.t32 - ((rem + 1) >> 1);
    return q >= 31 ? 0 : (i64)(unshifted >> q);
  }
  return di_exp_r(wneg((i64)neg), E.tpos, E.R);
}

// round_half_away_div(num << 7, den) for 0 <= num <= den < 2^31, in 32 bits:
// one step for the integer bit, seven doubling steps (t < den < 2^31, so 2t
// fits), then the half-divisor rounding term. Same integer as sigmoid_div.
DI_HD i64 sigmoid_div32(uint32_t num, uint32_t den) {
  uint32_t t = num, q = 0;
  if (t >= den) {
    t -= den;
    q = 1;
  }
#pragma unroll
  for (int b = 0; b < 7; ++b) {
    t <<= 1;
    q <<= 1;
    if (t >= den) {
      t -= den;
      q |= 1;
    }
  }
  if (t + (den >> 1) >= den) q += 1;
  return (i64)q;
}

// round_half_away_div(num << 7, den) for 0 <= num <= den, den >= 1: the
// quotient is at most 128, so 8 restoring steps are exact. Larger operands
// (never produced on the model path) take the generic form.
DI_HD i64 sigmoid_div(i64 num, i64 den) {
  if (num >= 0 && den >= num && den < ((i64)1 << 48)) {
    u64 n = ((u64)num << 7) + ((u64)den >> 1);
    const u64 d = (u64)den;
    i64 q = 0;
#pragma unroll
    for (int b = 7; b >= 0; --b) {
      const u64 db = d << b;
      if (n >= db) {
        n -= db;
        q |= (i64)1 << b;
      }
    }
    return q;
  }
  return rhad(shl(num, 7), den);
}

// ops/di_swiglu.py:39-58 on one element (tpos/R per row)
DI_HD i64 swiglu_elem(i64 g, i64 u, i64 tpos, const Recip& R) {
  const i64 E = di_exp_r(wneg(wabs(g)), tpos, R);
  const i64 den = imax(wadd(tpos, E), 1);
  const i64 num = g >= 0 ? tpos : E;
  const i64 sig = sigmoid_div(num, den);
  return wmul(wmul(g, sig), u);
}

// swiglu_elem with the row's DI-Exp context: 32-bit DI-Exp and sigmoid
// division when tpos < 2^30 (then E <= tpos and den = tpos + E < 2^31) and g
// is an int32 value; otherwise the 64-bit form. Same integer.
DI_HD i64 swiglu_elem_e(i64 g, i64 u, const ExpR& E) {
  if (E.tpos < ((i64)1 << 30) && g >= INT32_MIN && g <= INT32_MAX) {
    const u64 mag = (u64)(g < 0 ? -g : g);
    const i64 e = di_exp_neg(mag, E);
    const uint32_t den = (uint32_t)imax(E.tpos + e, 1);
    const uint32_t num = (uint32_t)(g >= 0 ? E.tpos : e);
    const i64 sig = sigmoid_div32(num, den);
    return wmul((i64)(int32_t)g * sig, u);
  }
  return swiglu_elem(g, u, E.tpos, E.R);
}

// ---- exact integers from biased fp64 estimates -------------------------
//
// fp64 runs at the full vector rate on gfx950, while a 64-bit integer
// division or reciprocal multiply costs tens of instructions. Each helper
// below computes an integer quotient as the truncation of one fp64 estimate
// that carries a bias large enough to cover every rounding error of the
// estimate and small enough to stay below the gap to the next integer, so
// the truncation is exact. Callers check the stated operand bounds (a
// wave-uniform test per row) and otherwise take the integer routines above.
// fma and the fp64 division are IEEE-correctly rounded on the device and on
// the host, so the host build of these helpers is the device arithmetic.

// v_mad_u32_u24: a b + c (mod 2^32) for a, b < 2^24, full rate on gfx950
// (the 32-bit multiplies issue at a quarter of it). Written out on the
// device because the compiler does not always see the operand bounds.
DI_HD uint32_t mad_u24(uint32_t a, uint32_t b, uint32_t c) {
#if defined(__HIP_DEVICE_COMPILE__)
  uint32_t d;
  asm("v_mad_u32_u24 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
#else
  return a * b + c;
#endif
}

// rhad(m s, d) = floor((m s + floor(d/2)) / d) for an exact integer m >= 0, a
// scale s (a power of two or 127) and a row-invariant d >= 1, from r = fl(s/d)
// and k = fl((floor(d/2) + 1/2) / d): fma(m, r, k) = v + 1/(2d) + err with
// v = (m s + floor(d/2)) / d and |err| <= (2 m s + d + 2) 2^-53 / d (one
// relative rounding each on r, k and the fma). When 2 m s + d < 2^51,
// |err| < 1/(2d); v is a multiple of 1/d, at most (d - 1)/d above floor(v),
// so the estimate lies in (v, floor(v) + 1) and truncates to floor(v).
// Quotients below 2^32.
struct DivEst {
  double r;
  double k;
};

DI_HD DivEst make_divest(i64 d, double s) {  // 1 <= d < 2^51
  DivEst D;
  D.r = s / (double)d;
  D.k = ((double)(d >> 1) + 0.5) / (double)d;
  return D;
}

DI_HD uint32_t rhad_est(double m, const DivEst& D) { return (uint32_t)fma(m, D.r, D.k); }

// sign(a) rhad(|a| s, d) for |a| s bounded as above, as a signed int32
DI_HD int32_t rhad_est_signed(i64 a, const DivEst& D) {
  const uint32_t q = rhad_est((double)(a < 0 ? -a : a), D);
  return a < 0 ? -(int32_t)q : (int32_t)q;
}

// clamp_i8(rhad(n, d)) for 2 |n| + d < 2^51: estimates at or above 255
// (quotients of 255 or more) saturate before the conversion and clamp like
// the integer quotient would.
DI_HD int rhad_est_i8(i64 n, const DivEst& D) {
  const double e = fmin(fma((double)(n < 0 ? -n : n), D.r, D.k), 255.0);
  const int q = (int)(uint32_t)e;
  const int sq = n < 0 ? -q : q;
  return sq < -128 ? -128 : (sq > 127 ? 127 : sq);
}

// rhad_est_signed and rhad_est_i8 of an integer-valued double (the same
// integers: the two helpers above convert their int64 operand's magnitude to
// this double, exactly under their bounds)
DI_HD int32_t rhad_est_signed_f64(double a, const DivEst& D) {
  const uint32_t q = rhad_est(fabs(a), D);
  return a < 0 ? -(int32_t)q : (int32_t)q;
}
DI_HD int rhad_est_i8_f64(double n, const DivEst& D) {
  const double e = fmin(fma(fabs(n), D.r, D.k), 255.0);
  const int q = (int)(uint32_t)e;
  const int sq = n < 0 ? -q : q;
  return sq < -128 ? -128 : (sq > 127 ? 127 : sq);
}

// rhad(s |a|, d) signed, for s |a| + d < 2^53 and quotients below 2^31, or
// for |a| <= d < 2^53 and 1 <= s <= 127: the estimate may be one off once
// 2 s |a| + d reaches 2^51, so its truncation q0 is corrected with the exact
// remainder n - q0 d, n = s |a| + floor(d/2). In the second case |a| is an
// exact double, the fma's value (below 128.5) lies within 2^-44 of
// (n + 1/2) / d, whose floor is floor(n / d), so q0 is within one of it, and
// n < 2^60, q0 d <= 2^60 as int64.
DI_HD int32_t rhad_est_corr_signed(i64 a, int s, i64 d, const DivEst& D) {
  const i64 n = (a < 0 ? -a : a) * (i64)s + (d >> 1);
  i64 q = (i64)(uint32_t)fma((double)(a < 0 ? -a : a), D.r, D.k);
  const i64 rem = n - q * d;
  q += (rem >= d ? 1 : 0) - (rem < 0 ? 1 : 0);
  return a < 0 ? -(int32_t)q : (int32_t)q;
}

// sigmoid division round_half_away_div(num << 7, den) (ops/di_swiglu.py:
// 52-55) for 0 <= num <= den < 2^31, den >= 1: the quotient v = (128 num +
// floor(den/2)) / den is at most 128.5; fl((128 num + floor(den/2) + 1/2) /
// den) = v + 1/(2 den) within 2^-53 129 < 1/(2 den) (the numerator is exact),
// so it truncates to floor(v) as above.
DI_HD uint32_t sigmoid_est(uint32_t num, uint32_t den) {
  return (uint32_t)(fma((double)num, 128.0, (double)(den >> 1) + 0.5) / (double)den);
}

// 1 / x in single precision: v_rcp_f32 (1 ulp) on the device, the correctly
// rounded quotient on the host
DI_HD float rcp_f32(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_rcpf(x);
#else
  return 1.0f / x;
#endif
}

// sigmoid_est for 0 <= num <= den < 2^24 without a double division:
// N = 128 num + floor(den/2) < 2^32 and v = N / den <= 128.5. fl(N), the
// reciprocal of the exactly represented den and the product are each within
// a relative 2^-23, so q = trunc(fl(fl(N) rcp(den))) is within 129 * 3 *
// 2^-23 < 1 of v: floor(v) - 1 <= q <= floor(v) + 1, and one remainder step
// (q den <= 129 * 2^24 < 2^32 by the exact 24-bit multiply; N - q den lies in
// (-den, 2 den)) gives floor(v), the same integer as sigmoid_est.
DI_HD uint32_t sigmoid_est24(uint32_t num, uint32_t den) {
  const uint32_t N = num * 128u + (den >> 1);
  uint32_t q = (uint32_t)((float)N * rcp_f32((float)den));
  const int32_t rem = (int32_t)(N - mad_u24(q, den, 0u));
  q += (rem >= (int32_t)den ? 1u : 0u) - (rem < 0 ? 1u : 0u);
  return q;
}

// DI-Exp of -n (ops/di_exp.py:27-37) for 0 <= n < 2^22 and a row-invariant
// 1 <= t < 2^23: e = fma(n, fl(1/t), 1 + 2^-26) is n/t + 1 + 2^-26 within
// 2^-30 (the rounding of 1/t and of the fma, on values below 2^23), and a
// non-integer n/t is at least 1/t > 2^-23 below the next integer, so e
// truncates to q1 = floor(n/t) + 1. With rem = n - q t, the result
// (t - ceil(rem/2)) >> q is (2t - rem) >> (q + 1) = (q1 t + t - n) >> q1,
// where q1 t + t - n = (q + 2) t - n lies in (0, 2t] below 2^24, so any shift
// of 24 or more (clamped to 31) gives the 0 that min(q, 62) gives for
// q >= 23.
struct ExpEst {
  double rt;   // fl(1 / t)
  uint32_t t;  // tpos
};

DI_HD ExpEst make_expest(i64 tpos) {  // 1 <= tpos < 2^23
  ExpEst E;
  E.t = (uint32_t)tpos;
  E.rt = 1.0 / (double)tpos;
  return E;
}

// di_exp_tpos with the division rhad(2^k, m_f) from the estimate when
// 0 <= k <= 46 and 1 <= m_f < 2^31 (2 * 2^k + m_f < 2^51, quotient < 2^32
// for m_f >= 2^15; smaller m_f takes the integer path); same integer.
DI_HD i64 di_exp_tpos_fast(i64 m, i64 k) {
  const i64 m_f = wsub(wadd(m, shr(m, 1)), shr(m, 4));
  if (DI_LIKELY(k >= 0 && k <= 46 && m_f >= ((i64)1 << 15) && m_f < ((i64)1 << 31)))
    return imax((i64)rhad_est((double)((i64)1 << k), make_divest(m_f, 1.0)), 1);
  return di_exp_tpos(m, k);
}

DI_HD uint32_t dexp_est(uint32_t n, const ExpEst& E) {
  const uint32_t q1 = (uint32_t)fma((double)n, E.rt, 1.0 + 0x1p-26);
  const uint32_t m = mad_u24(q1, E.t, E.t - n);
  return m >> (q1 < 31u ? q1 : 31u);
}

// dexp_est of n = mx - st taken from sp = st + t - mx (attention adds t - mx
// to the scores for free in the MFMA accumulator): |sp| < 2^23, and
// fma(sp, -fl(1/t), fl(t fl(1/t) + 1 + 2^-26)) = 2 - sp/t + 2^-26 =
// n/t + 1 + 2^-26 within 2^-29 (roundings of 1/t, of the constant and of the
// fma on values below 2^24), so the same truncation argument holds, and
// q1 t + sp = q1 t + t - n.
DI_HD double dexp_sp_const(const ExpEst& E) { return fma((double)E.t, E.rt, 1.0 + 0x1p-26); }

DI_HD uint32_t dexp_est_sp(int32_t sp, const ExpEst& E, double kx) {
  const uint32_t q1 = (uint32_t)fma((double)sp, -E.rt, kx);
  const uint32_t m = mad_u24(q1, E.t, (uint32_t)sp);
  return m >> (q1 < 31u ? q1 : 31u);
}

// floor(sqrt(n)) for 0 <= n < 2^62 (int_prims.py:31-44 isqrt, negative n
// give 0): fp64 sqrt of fl(n) is within 2^-21 of sqrt(n) (relative 2^-53
// on n, one rounding of the square root), so its truncation is the integer
// root or one off either way; one exact integer step each way settles it
// ((r + 1)^2 <= 2^62 stays in range).
DI_HD i64 isqrt_est(i64 n) {
  if (n <= 0) return 0;
  i64 r = (i64)sqrt((double)n);
  if (r * r > n) r -= 1;
  if ((r + 1) * (r + 1) <= n) r += 1;
  return r;
}

// ---- exact integers carried as fp64 values ----------------------------
//
// An integer of magnitude below 2^53 is an exact double, and fp64 multiply,
// fma and floor are correctly rounded (IEEE), so a product of two such
// integers whose true value is below 2^53 comes out exact. The row kernels
// keep their int32 x mantissa products in this form where the operands are
// bounded (a 64-bit integer multiply costs four quarter-rate instructions on
// gfx950, an fp64 multiply one full-rate instruction); the bounds each use
// needs are checked per row, with the integer routines as the fallback.

// Bit length of an integer-valued double (0 for 0): e with 2^(e-1) <= |x| <
// 2^e, the exponent frexp returns (v_frexp_exp_i32_f64 on the device).
DI_HD uint32_t bitlen_f64(double x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return x == 0.0 ? 0u : (uint32_t)__builtin_amdgcn_frexp_exp(x);
#else
  int e = 0;
  frexp(x, &e);
  return x == 0.0 ? 0u : (uint32_t)e;
#endif
}

// The bit pattern of a non-negative double as an int64 orders like the
// double, so a block maximum of magnitudes reduces these patterns.
DI_HD i64 f64_bits(double x) {
  i64 b;
  __builtin_memcpy(&b, &x, 8);
  return b;
}
DI_HD double f64_from_bits(i64 b) {
  double x;
  __builtin_memcpy(&x, &b, 8);
  return x;
}

// rshift_round(x, sh) (intmath.py:120-147: (x + 2^(sh-1)) >> sh, floor) for an
// integer-valued double with |x| < 2^52 and 0 <= sh < 1000: x 2^-sh is exact
// (a power-of-two scaling), a multiple of 2^-sh below 2^(52-sh) in magnitude,
// so adding 1/2 in the fma stays exact (the sum is below 2^(53-sh) and a
// multiple of 2^-sh), and floor gives the integer. At sh = 0 that is
// floor(x + 1/2) = x, the identity rshift_round keeps for a zero shift.
DI_HD double rshift_round_f64(double x, int sh) {
  return floor(fma(x, ldexp(1.0, -sh), 0.5));
}

// The bit length of max |x| over integer-valued doubles (|x| < 2^53) from the
// high words of their bit patterns: the high word of |x| (sign bit cleared)
// orders like |x| up to ties within one exponent, so the maximum of the high
// words over a row holds the largest biased exponent e, and the bit length
// is e - 1022 (0 for a row of zeros). One AND and one 32-bit maximum per
// element. The high word of +inf (0x7FF00000) reads 1025: a row that enters
// it is marked inexact (any bit length of 64 or more).
DI_HD uint32_t f64_hiword_abs(double x) {
  return (uint32_t)((uint64_t)f64_bits(x) >> 32) & 0x7FFFFFFFu;
}
DI_HD uint32_t bitlen_from_hiword(uint32_t hw) { return hw == 0u ? 0u : (hw >> 20) - 1022u; }


// ops/di_swiglu.py:39-58 on one element for |g|, |u| <= 2^14 (gate and up
// after requant_i32_common(14)) and tpos < 2^23: |g| < 2^22 for dexp_est,
// E <= tpos and den = tpos + E < 2^24 for sigmoid_est24, g * sig (sig <= 128)
// fits int32 and g * sig * u int64. Same integer as swiglu_elem.
DI_HD i64 swiglu_elem_est(int32_t g, int32_t u, const ExpEst& E) {
  const uint32_t e = dexp_est((uint32_t)(g < 0 ? -g : g), E);
  const uint32_t sig = sigmoid_est24(g >= 0 ? E.t : e, E.t + e);
  return (i64)(g * (int32_t)sig) * (i64)u;
}

// g * sig of swiglu_elem_est (|g| <= 2^14, sig <= 128: an int32 product)
DI_HD int32_t swiglu_gsig_est(int32_t g, const ExpEst& E) {
  const uint32_t e = dexp_est((uint32_t)(g < 0 ? -g : g), E);
  const uint32_t sig = sigmoid_est24(g >= 0 ? E.t : e, E.t + e);
  return g * (int32_t)sig;
}

}  // namespace di
