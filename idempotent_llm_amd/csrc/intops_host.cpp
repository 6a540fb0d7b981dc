// Host (CPU) build of intops.h for the CPU test suite: batch wrappers that let
// tests compare the exact same integer routines the kernels use against the
// numpy oracle and brute force, without a GPU.
#include "intops.h"

using namespace di;

extern "C" {

void di_host_rhad_r(const int64_t* a, const int64_t* d, int64_t n, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = rhad_r(a[i], make_recip(d[i]));
}
void di_host_rhad(const int64_t* a, const int64_t* d, int64_t n, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = rhad(a[i], d[i]);
}
void di_host_floor_div_r(const int64_t* a, const int64_t* d, int64_t n, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = floor_div_r(a[i], make_recip(d[i]));
}
void di_host_di_exp(const int64_t* x, const int64_t* tpos, int64_t n, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = di_exp_r(x[i], tpos[i], make_recip(tpos[i]));
}
void di_host_di_exp_tpos(const int64_t* m, const int64_t* k, int64_t n, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = di_exp_tpos(m[i], k[i]);
}
void di_host_sigmoid_div(const int64_t* num, const int64_t* den, int64_t n, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = sigmoid_div(num[i], den[i]);
}
void di_host_swiglu(const int64_t* g, const int64_t* u, const int64_t* tpos, int64_t n,
                    int64_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = swiglu_elem(g[i], u[i], tpos[i], make_recip(tpos[i]));
}
void di_host_scalar(int op, const int64_t* a, const int64_t* b, const int64_t* c, int64_t n,
                    int64_t* o1, int64_t* o2) {
  for (int64_t i = 0; i < n; ++i) {
    int64_t x = 0, y = 0;
    switch (op) {
      case 0: o1[i] = isqrt(a[i]); break;
      case 1: o1[i] = ilog2(a[i]); break;
      case 2: norm_scale(a[i], b[i], &x, &y); o1[i] = x; o2[i] = y; break;
      case 3: fit_dyadic_ratio(a[i], b[i], &x, &y); o1[i] = x; o2[i] = y; break;
      case 5: fit_dyadic_ratio_127(a[i], &x, &y); o1[i] = x; o2[i] = y; break;
      case 6: o1[i] = rhad_pow2(a[i], (int)b[i]); break;
      case 7: o1[i] = di_exp_tpos_fast(a[i], b[i]); break;
      case 8: o1[i] = isqrt_est(a[i]); break;
      case 9: o1[i] = floor_div127((uint32_t)a[i]); break;
      default: o1[i] = scaled_round_div(a[i], b[i], c[i]); break;
    }
  }
}
// bitlen_f64 / rshift_round_f64 on integer inputs: out[i] = bit length of
// a[i] (op 0) or rshift_round_f64(a[i], b[i]) converted back (op 1); op 5:
// in_range(a[i], b[i])
void di_host_f64_int_op(int op, const int64_t* a, const int64_t* b, int64_t n, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) {
    if (op == 0) out[i] = (int64_t)bitlen_f64((double)a[i]);
    else if (op == 1) out[i] = (int64_t)rshift_round_f64((double)a[i], (int)b[i]);
    else if (op == 2) out[i] = rhad_est_i8_f64((double)a[i], make_divest(b[i], 1.0));
    else if (op == 4) out[i] = (int64_t)bitlen_from_hiword(f64_hiword_abs((double)a[i]));
    else if (op == 5) out[i] = in_range(a[i], b[i]) ? 1 : 0;
    else out[i] = rhad_est_signed_f64((double)a[i], make_divest(b[i], 127.0));
  }
}
void di_host_di_exp_neg(const int64_t* neg, const int64_t* tpos, int64_t n, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = di_exp_neg((u64)neg[i], make_exp(tpos[i]));
}
void di_host_swiglu_e(const int64_t* g, const int64_t* u, const int64_t* tpos, int64_t n,
                      int64_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = swiglu_elem_e(g[i], u[i], make_exp(tpos[i]));
}
void di_host_sigmoid_div32(const int64_t* num, const int64_t* den, int64_t n, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = sigmoid_div32((uint32_t)num[i], (uint32_t)den[i]);
}
void di_host_rshift_round(const int64_t* a, const int64_t* k, int64_t n, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = rshift_round(a[i], k[i]);
}

void di_host_rhad_est(const int64_t* m, const int64_t* d, const double* sc, int64_t n,
                      int64_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = rhad_est((double)m[i], make_divest(d[i], sc[i]));
}
void di_host_sigmoid_est(const int64_t* num, const int64_t* den, int64_t n, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = sigmoid_est((uint32_t)num[i], (uint32_t)den[i]);
}
void di_host_sigmoid_est24(const int64_t* num, const int64_t* den, int64_t n, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = sigmoid_est24((uint32_t)num[i], (uint32_t)den[i]);
}
// Mismatches of dexp_est(n) and dexp_est_sp(t - n) against the integer DI-Exp
// for every n in [n_lo, n_hi) at one tpos.
int64_t di_host_dexp_est_mismatches(int64_t tpos, int64_t n_lo, int64_t n_hi) {
  const ExpR R = make_exp(tpos);
  const ExpEst E = make_expest(tpos);
  const double kx = dexp_sp_const(E);
  int64_t bad = 0;
  for (int64_t n = n_lo; n < n_hi; ++n) {
    const int64_t want = di_exp_r(-n, tpos, R.R);
    bad += (int64_t)dexp_est((uint32_t)n, E) != want;
    bad += (int64_t)dexp_est_sp((int32_t)(tpos - n), E, kx) != want;
  }
  return bad;
}

void di_host_swiglu_est(const int64_t* g, const int64_t* u, const int64_t* tpos, int64_t n,
                        int64_t* out) {
  for (int64_t i = 0; i < n; ++i)
    out[i] = swiglu_elem_est((int32_t)g[i], (int32_t)u[i], make_expest(tpos[i]));
}

// op 0: rhad_est_signed(a, divest(d, s)); 1: rhad_est_i8(a, divest(d, 1));
// 2: rhad_est_corr_signed(a, s, d, divest(d, s))
void di_host_rhad_est_op(int op, const int64_t* a, const int64_t* d, const int64_t* sc,
                         int64_t n, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) {
    const DivEst D = make_divest(d[i], op == 1 ? 1.0 : (double)sc[i]);
    out[i] = op == 0 ? rhad_est_signed(a[i], D)
                     : (op == 1 ? rhad_est_i8(a[i], D) : rhad_est_corr_signed(a[i], (int)sc[i], d[i], D));
  }
}

}  // extern "C"
