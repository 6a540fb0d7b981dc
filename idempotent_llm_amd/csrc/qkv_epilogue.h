// Q/K/V epilogue of one (token row, head slot), shared by the standalone
// epilogue kernel (prefill) and the fused decode attention kernel.
//
// One wave per (token row r, head slot): slots [0, n_q) are query heads,
// [n_q, n_q + n_kv) key heads, then value heads. Lane l owns channels l and
// l + 64, which is exactly the rotate_half pairing of RoPE. Reference:
// model.py:200-216 (_qk_head_pipeline), :303-340 (QK smoothing, Q
// quant_i8_pertoken, K/V requant_i8_static, cache write), :351-358 (score
// scale and DI-Exp constant).
#pragma once

#include "common.h"

namespace di {

struct QKVArgs {
  int T;
  int n_q, n_kv;
  const int32_t* P;  // [nsplit][R][(n_q + 2 n_kv) * 128]
  int nsplit;
  i64 split_stride;
  const int64_t* xm;
  const int64_t* xk;
  const int64_t* positions;  // [R]
  const int64_t* q_m;
  const int64_t* k_m;
  const int64_t* v_m;
  i64 q_k, k_k, v_k;
  const int64_t* q_norm_m;
  const int64_t* k_norm_m;
  i64 q_norm_k, k_norm_k;
  const int64_t* qs_m;  // [n_kv * 128]
  i64 qs_k;
  const int64_t* kq_m;  // [n_kv * 128]
  const int64_t* kq_k;
  const int64_t* kq_est;  // optional [n_kv * 128][4] (kq_channel_est), else computed
  const int64_t* ks_m;  // [n_kv]
  const int64_t* ks_k;
  const int64_t* vq_m;
  const int64_t* vq_k;
  const int16_t* cos_t;
  const int16_t* sin_t;
  i64 max_pos;
  int8_t* q8;      // [B][n_q][T][128]
  int64_t* tpos;   // [B][n_q][T]
  int64_t* dbg;    // optional [B][n_q][T][4]: qm, qk, sm, sk
  KVPages kv;      // the layer's paged cache: K and V of slot base + t are written
  const int64_t* slot_base_dev;  // optional device scalar (graph replay)
  i64 slot_base;
  int32_t* err;  // optional device error word (DI_ERR_POSITION)
};

// The static K requantisation's divisor of one channel (model.py:326-329,
// requant_i8_static with row scale (1, rowk)): den = kq_m << max(rowk - kq_k,
// 0) (wrapping as torch's shift does; 1 if it is 0, where the reference's
// division raises), the numerator's up-shift max(kq_k - rowk, 0), and
// DivEst(den, 1) for rhad_est_i8 (used for 0 < den < 2^49 only; a negative
// wrapped divisor takes the generic floor division, as torch computes it). Every input is a layer constant, so the
// estimate can be computed once per channel (kq_est) instead of per element.
struct KqChan {
  i64 den, up;
  DivEst D;
};

__device__ __forceinline__ KqChan kq_channel(i64 km, i64 kk, i64 rowk) {
  const i64 shift = wsub(rowk, kk);
  KqChan q;
  q.up = imax(wneg(shift), 0);
  q.den = shl(km, imax(shift, 0));
  if (q.den == 0) q.den = 1;
  q.D = make_divest(q.den > 0 && q.den < ((i64)1 << 49) ? q.den : 1, 1.0);
  return q;
}

// ilog2(max(max |x|, 1)) over the wave's 128 channels (two per lane)
__device__ __forceinline__ i64 wave_ilog2_absmax(i64 a, i64 b) {
  const uint32_t L = BlockRed::wave_max_u32(::max(bitlen_abs(a), bitlen_abs(b)));
  return ilog2_from_bitlen((uint32_t)__builtin_amdgcn_readlane((int)L, 63));
}

__device__ __forceinline__ void wave_rmsnorm128(i64& a, i64& b) {
  // ops/di_rmsnorm.py:33-52 over 128 channels held two per lane
  const i64 sh = 25 - wave_ilog2_absmax(a, b);
  const i64 up = imax(sh, 0), down = imax(-sh, 0);
  a = shl(rshift_round(a, down), up);
  b = shl(rshift_round(b, down), up);
  const i64 ss = wave_sum(wadd(wmul(a, a), wmul(b, b)));
  const i64 rms = imax(isqrt_wave(rhad_pow2(ss, 7)), 1);
  if (DI_LIKELY(rms > ((i64)1 << 16))) {
    // |a|, |b| <= 2^26 after the shift: rhad_est as in rmsnorm_row
    const DivEst D = make_divest(rms, 1048576.0);
    a = rhad_est_signed(a, D);
    b = rhad_est_signed(b, D);
  } else {
    const Recip R = make_recip(rms);
    a = to_i32(rhad_r(shl(a, 20), R));
    b = to_i32(rhad_r(shl(b, 20), R));
  }
}

// Reductions over each aligned row of 16 lanes (result in all 16)
__device__ __forceinline__ i64 row16_max64(i64 v) {
  v = imax(v, dpp64<0xB1, 0xF>(v, v));
  v = imax(v, dpp64<0x4E, 0xF>(v, v));
  v = imax(v, dpp64<0x141, 0xF>(v, v));
  return imax(v, dpp64<0x140, 0xF>(v, v));
}
__device__ __forceinline__ i64 row16_sum64(i64 v) {
  v = wadd(v, dpp64<0xB1, 0xF>(v, 0));
  v = wadd(v, dpp64<0x4E, 0xF>(v, 0));
  v = wadd(v, dpp64<0x141, 0xF>(v, 0));
  return wadd(v, dpp64<0x140, 0xF>(v, 0));
}
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
  v = ::max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xF, 0xF, false));
  v = ::max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false));
  v = ::max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x141, 0xF, 0xF, false));
  return ::max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x140, 0xF, 0xF, false));
}

// The reductions of one head's channels: the 16 lanes of a token row (the
// prefill layout) or the whole wave (one head per wave). Sums of doubles add
// integers whose every partial sum is an exact double.
template <bool WAVE>
struct HeadRed {
  __device__ __forceinline__ uint32_t max_u32(uint32_t v) const {
    if (WAVE) return (uint32_t)__builtin_amdgcn_readlane((int)BlockRed::wave_max_u32(v), 63);
    return row16_max_u32(v);
  }
  __device__ __forceinline__ i64 max(i64 v) const { return WAVE ? wave_max(v) : row16_max64(v); }
  __device__ __forceinline__ double sum(double v) const {
    v += f64_from_bits(dpp64<0xB1, 0xF>(f64_bits(v), 0));
    v += f64_from_bits(dpp64<0x4E, 0xF>(f64_bits(v), 0));
    v += f64_from_bits(dpp64<0x141, 0xF>(f64_bits(v), 0));
    v += f64_from_bits(dpp64<0x140, 0xF>(f64_bits(v), 0));
    if (!WAVE) return v;
    v += f64_from_bits(dpp64<0x142, 0xA>(f64_bits(v), 0));
    v += f64_from_bits(dpp64<0x143, 0xC>(f64_bits(v), 0));
    return f64_from_bits(readlane64(f64_bits(v), 63));
  }
};

// _qk_head_pipeline (model.py:200-216: requant_i32_common(16), di_rmsnorm,
// gamma, apply_int_rope) then the K requantisation (model.py:326-329) or the
// Q smoothing (model.py:317-320) and the Q quantiser's quotients
// (model.py:322-323), on exact fp64 values. A lane holds N channels: [0, N/2)
// and their RoPE partners (channel + 64) at [N/2, N). Bounds that make every
// step exact, each checked per lane and folded into the first reduction:
//  * |w_m| < 2^21: P w_m is below 2^52; requant_i32_common(16) leaves
//    |y| <= 2^16, so di_rmsnorm's shift 25 - ilog2(max |y|) is an up-shift
//    u >= 9 and the mean of the shifted squares, rhad(ss 2^(2u), 128) with
//    ss = sum y^2 below 2^39, is exactly ss 2^(2u - 7) (below 2^52: every
//    |y 2^u| < 2^26);
//  * rms = isqrt(mean) >= 2^21 unless the head is zero (the largest |y 2^u|
//    is at least 2^25), so the normalised values rhad(y 2^u 2^20, rms) are
//    below 11.32 * 2^20 < 2^24 in magnitude (|y 2^u| <= sqrt(128 mean + 64)),
//    and with |gamma_m| < 2^12 the gamma products a stay below 2^36;
//  * the RoPE sums a cos + a' sin (int16 tables, |entry| <= 2^15) are exact
//    doubles below 2^52, the rotated values r = rshift_round(., 14) below
//    2^38, and with |qs_m| < 2^15 the smoothed q = r qs_m below 2^53.
// The Q quotients rhad(127 |q|, am) come from fp64 estimates for every am
// below 2^53 (exact below 2^43 as in quant_row; above, checked per element).
// Returns false (uniform over the head's lanes) for a head outside them, or
// a zero head: the caller runs the integer routines. On true, o holds the K
// head's int8 values or the Q head's quotients and *am_out the Q head's
// max(max |q|, 1). kq(i): the KqChan of channel i (K heads only).
template <int N, bool WAVE, class KqF>
__device__ __forceinline__ bool qk_head_f64(bool is_q, const int32_t (&p)[N],
                                            const i64 (&wm)[N], const i64 (&gm)[N],
                                            const int32_t (&cs)[N], const int32_t (&sn)[N],
                                            const i64 (&qs)[N], KqF&& kq, int (&o)[N],
                                            i64* am_out) {
  constexpr int H = N / 2;
  constexpr i64 WM_LIM = (i64)1 << 21, G_LIM = (i64)1 << 12, QS_LIM = (i64)1 << 15;
  const HeadRed<WAVE> red;
  double y[N];
  uint32_t pm = 0u;
  bool ok = true;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    ok = ok & in_range(wm[i], WM_LIM) & in_range(gm[i], G_LIM) & (!is_q | in_range(qs[i], QS_LIM));
    y[i] = (double)p[i] * (double)(int32_t)wm[i];
    pm = ::max(pm, f64_hiword_abs(y[i]));
  }
  const uint32_t L = bitlen_from_hiword(red.max_u32(ok ? pm : 0x7FF00000u));
  if (DI_UNLIKELY(L >= 64u)) return false;
  // requant_i32_common(tb = 16) per (token, head)
  const int sh = (int)imax(ilog2_from_bitlen(L) - 15, 0);
  uint32_t ym = 0u;
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    y[i] = rshift_round_f64(y[i], sh);
    ym = ::max(ym, f64_hiword_abs(y[i]));
    ss = fma(y[i], y[i], ss);
  }
  const uint32_t L2 = bitlen_from_hiword(red.max_u32(ym));
  ss = red.sum(ss);
  // di_rmsnorm (ops/di_rmsnorm.py:33-52) with the up-shift u
  const int u = 25 - (int)ilog2_from_bitlen(L2);
  const i64 rms = imax(isqrt_est((i64)ss << (2 * u - 7)), 1);
  if (DI_UNLIKELY(rms <= ((i64)1 << 16))) return false;  // a zero head
  const DivEst D = make_divest(rms, 1048576.0);
  const double su = ldexp(1.0, u);
  double a[N];
#pragma unroll
  for (int i = 0; i < N; ++i)
    a[i] = (double)rhad_est_signed_f64(y[i] * su, D) * (double)(int32_t)gm[i];
  // apply_int_rope (rope.py:38-55)
  double r[N];
#pragma unroll
  for (int i = 0; i < H; ++i) {
    r[i] = rshift_round_f64(fma(a[i], (double)cs[i], -(a[i + H] * (double)sn[i])), 14);
    r[i + H] = rshift_round_f64(fma(a[i + H], (double)cs[i + H], a[i] * (double)sn[i + H]), 14);
  }
  if (!is_q) {
    // requant_i8_static(kk, 1, k_rowk, 1, 0, kq_m, kq_k): n = r << up
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const KqChan q = kq(i);
      const double n = ldexp(r[i], (int)imin(q.up, 64));
      const i64 lim = (i64)1 << 49;  // 2 |n| + den < 2^51 for the estimate
      o[i] = (q.den > 0 && q.den < lim && fabs(n) < 0x1p49)
                 ? rhad_est_i8_f64(n, q.D)
                 : (int)clamp_i8(rhad(shl((i64)r[i], q.up), q.den));
    }
    return true;
  }
  // QK smoothing, then quant_i8_pertoken's quotients (quant_row's two forms)
  double q[N];
  double g = 0.0;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    q[i] = r[i] * (double)(int32_t)qs[i];
    g = fmax(g, fabs(q[i]));
  }
  const double amu = f64_from_bits(red.max(f64_bits(g)));
  const i64 am = imax((i64)amu, 1);
  const DivEst Dq = make_divest(am, 127.0);
  *am_out = am;
  if (DI_LIKELY(amu < 0x1p43)) {
#pragma unroll
    for (int i = 0; i < N; ++i) o[i] = rhad_est_signed_f64(q[i], Dq);
    return true;
  }
  // am in [2^43, 2^53): the estimate e = fma(|q|, fl(127/am), k) of
  // v + 1/(2 am), v = (127 |q| + floor(am/2)) / am, is within 2^-45 (the
  // roundings of 127/am and k, relative 2^-53 on terms up to 128, and of the
  // fma), so a fractional part of e at least 2^-44 away from an integer
  // truncates to floor(v); any other element (rare) takes the integer
  // division
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const double e = fma(fabs(q[i]), Dq.r, Dq.k);
    const double f = e - floor(e);
    if (DI_LIKELY(f > 0x1p-44 && f < 1.0 - 0x1p-44)) {
      const int qc = (int)e;
      o[i] = q[i] < 0 ? -qc : qc;
    } else {
      o[i] = (int)clamp_i8(rhad_r(wmul((i64)q[i], 127), make_recip(am)));
    }
  }
  return true;
}

// The loads of one (token row, head slot) of qkv_head: every global load
// that does not depend on another, issued together (one memory round trip).
struct QKVHeadIn {
  i64 pos_raw, xk, xm, base;
  i64 wm0, wm1, g0, g1, qs0, qs1, kqm0, kqm1, kqk0, kqk1, vqm, vqk, ksm, ksk;
  int32_t p0, p1;          // sign-extended where used (no wait at the load)
  i64 pos;                 // qkv_head_rope_load: the checked position
  bool pos_bad;            // and whether it was out of range (reported by compute)
  int16_t cs0, cs1, sn0, sn1;  // and its RoPE table entries (widened where used)
};

// The slot of the launch's first token: the device scalar when given, else
// the argument. The load goes through a pointer that is always valid and the
// value is selected after it (a select of a kernel-argument address would
// make the load a flat one, which every later scalar-load wait includes).
__device__ __forceinline__ i64 slot_base_of(const QKVArgs& a) {
  const int64_t* bp = a.slot_base_dev ? a.slot_base_dev : a.positions;
  const i64 bv = bp[0];
  // the argument as a value that is not a load (else the optimizer folds the
  // two loads back into one through the selected address)
  const u64 sb = (u64)a.slot_base;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)sb);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(sb >> 32));
  return a.slot_base_dev ? bv : (i64)(((u64)hi << 32) | lo);
}

// The kv head of head slot slotw
__device__ __forceinline__ int qkv_kv_head(const QKVArgs& a, int slotw) {
  const bool is_q = slotw < a.n_q, is_v = slotw >= a.n_q + a.n_kv;
  return is_q ? slotw / (a.n_q / a.n_kv) : (is_v ? slotw - a.n_q - a.n_kv : slotw - a.n_q);
}

// The scalars of one (token row r, head slot): the row's position and input
// scale, the step's slot, the kv head's static V scale and score scale.
struct QKVScalars {
  i64 pos_raw, xk, xm, base, vqm, vqk, ksm, ksk;
};

// QKVScalars by plain loads (base: slot_base_of(a))
__device__ __forceinline__ QKVScalars qkv_scalars(const QKVArgs& a, int r, int slotw, i64 base) {
  const int kvh = qkv_kv_head(a, slotw);
  QKVScalars q;
  q.pos_raw = a.positions[r];
  q.xk = a.xk[r];
  q.xm = a.xm[r];
  q.base = base;
  q.vqm = a.vq_m[kvh];
  q.vqk = a.vq_k[kvh];
  q.ksm = a.ks_m[kvh];
  q.ksk = a.ks_k[kvh];
  return q;
}

// The per-channel loads of one (token row r, head slot), the scalars given.
// ONE: the caller guarantees nsplit == 1 (straight-line loads, no branch
// whose merge would force them to complete early).
template <bool ONE = false>
__device__ __forceinline__ QKVHeadIn qkv_head_load(const QKVArgs& a, int r, int slotw,
                                                   const QKVScalars& sc) {
  const int lane = threadIdx.x & 63;
  const int n_heads = a.n_q + 2 * a.n_kv;
  const int NQKV = n_heads * 128;
  const i64 off = (i64)r * NQKV + (i64)slotw * 128;
  const int group = a.n_q / a.n_kv;
  const bool is_q = slotw < a.n_q, is_v = slotw >= a.n_q + a.n_kv;
  const int h = is_q ? slotw : (is_v ? slotw - a.n_q - a.n_kv : slotw - a.n_q);
  const int kvh = is_q ? h / group : h;
  const int c0 = lane, c1 = lane + 64;
  QKVHeadIn in;
  in.pos_raw = sc.pos_raw;
  in.xk = sc.xk;
  in.xm = sc.xm;
  in.base = sc.base;
  in.vqm = sc.vqm;
  in.vqk = sc.vqk;
  in.ksm = sc.ksm;
  in.ksk = sc.ksk;
  // (each candidate pointer through opaque_ptr: a select between kernel
  // arguments would become a scalar load from the selected argument's
  // address, one more round trip before the loads below)
  const int64_t* wmp =
      (is_q ? opaque_ptr(a.q_m) : (is_v ? opaque_ptr(a.v_m) : opaque_ptr(a.k_m))) + (i64)h * 128;
  in.wm0 = ld_global(wmp + c0);
  in.wm1 = ld_global(wmp + c1);
  const int64_t* gam = is_q ? opaque_ptr(a.q_norm_m) : opaque_ptr(a.k_norm_m);
  in.g0 = ld_global(gam + c0);
  in.g1 = ld_global(gam + c1);
  in.qs0 = a.qs_m[kvh * 128 + c0];
  in.qs1 = a.qs_m[kvh * 128 + c1];
  in.kqm0 = a.kq_m[kvh * 128 + c0];
  in.kqm1 = a.kq_m[kvh * 128 + c1];
  in.kqk0 = a.kq_k[kvh * 128 + c0];
  in.kqk1 = a.kq_k[kvh * 128 + c1];
  if (ONE || a.nsplit == 1) {  // no K split: one load per channel
    in.p0 = a.P[off + c0];
    in.p1 = a.P[off + c1];
  } else {
    uint32_t s0 = 0, s1 = 0;
    for (int k0 = 0; k0 < a.nsplit; k0 += 4) {
      int32_t t0[4], t1[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int k = k0 + kk < a.nsplit ? k0 + kk : a.nsplit - 1;
        t0[kk] = a.P[(i64)k * a.split_stride + off + c0];
        t1[kk] = a.P[(i64)k * a.split_stride + off + c1];
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        if (k0 + kk < a.nsplit) {
          s0 += (uint32_t)t0[kk];
          s1 += (uint32_t)t1[kk];
        }
    }
    in.p0 = (int32_t)s0;
    in.p1 = (int32_t)s1;
  }
  return in;
}

// The RoPE table rows of the head's position (loads that depend on the
// position loaded by qkv_head_load), indexed as torch_index does; an out of
// range position is reported (DI_ERR_POSITION) by qkv_head_report, after
// the head's computation: a pending atomic among the loads would make the
// compiler wait for all of them at the first use of any.
__device__ __forceinline__ void qkv_head_rope_load(const QKVArgs& a, int slotw, QKVHeadIn& in) {
  const int lane = threadIdx.x & 63;
  const int c0 = lane, c1 = lane + 64;
  in.pos = torch_index(in.pos_raw, a.max_pos, nullptr, DI_ERR_POSITION);
  const i64 x = in.pos_raw < 0 ? in.pos_raw + a.max_pos : in.pos_raw;
  in.pos_bad = x < 0 || x >= a.max_pos;
  in.cs0 = a.cos_t[in.pos * 128 + c0];
  in.cs1 = a.cos_t[in.pos * 128 + c1];
  in.sn0 = a.sin_t[in.pos * 128 + c0];
  in.sn1 = a.sin_t[in.pos * 128 + c1];
}

// DI_ERR_POSITION for a position out of range (one lane of a Q or K head)
__device__ __forceinline__ void qkv_head_report(const QKVArgs& a, int slotw, const QKVHeadIn& in) {
  const bool is_v = slotw >= a.n_q + a.n_kv;
  if (in.pos_bad && !is_v && (threadIdx.x & 63) == 0 && a.err) atomicOr(a.err, DI_ERR_POSITION);
}

// A query head's DI-Exp constant from its int8 row's quantisation maximum
// am: the scale fit of am * 2^-20-normalised (m, k) (quant_i8_pertoken's
// (m, k)), the score scale norm_scale(qm * ks_m, qk + ks_k) (model.py:
// 351-353) and di_exp_tpos of it. One lane's serial chain.
__device__ __forceinline__ i64 q_head_tpos(const QKVArgs& a, i64 am, i64 ksm, i64 ksk,
                                           i64* dbg4) {
  const i64 qkk = 20 + a.q_norm_k + a.qs_k;
  i64 m, k;
  norm_scale(1, qkk, &m, &k);
  i64 qm, e;
  fit_dyadic_ratio_127(wmul(am, m), &qm, &e);
  const i64 qk = wadd(k, e);
  // score scale: norm_scale(qm * ks_m[h//g], qk + ks_k[h//g])   (model.py:351-353)
  i64 sm, sk;
  norm_scale(wmul(qm, ksm), wadd(qk, ksk), &sm, &sk);
  if (dbg4) {
    dbg4[0] = qm;
    dbg4[1] = qk;
    dbg4[2] = sm;
    dbg4[3] = sk;
  }
  return di_exp_tpos_fast(sm, sk);
}

// The whole wave must be active. K and V go to the cache; a query head's
// int8 row goes to q8_out[0..128) and its DI-Exp constant to *tpos_out
// (global memory for the standalone kernel, LDS for the fused one), or,
// with am_out, its quantisation maximum am to *am_out for q_head_tpos
// later. `in`: qkv_head_load then qkv_head_rope_load of the same (r, slotw).
__device__ __forceinline__ void qkv_head_compute(const QKVArgs& a, int r, int slotw,
                                                 const QKVHeadIn& in, int8_t* q8_out,
                                                 int64_t* tpos_out, int8_t* k_lds = nullptr,
                                                 int64_t* am_out = nullptr) {
  const int lane = threadIdx.x & 63;
  const int b = r / a.T, t = r - b * a.T;
  const bool is_q = slotw < a.n_q, is_v = slotw >= a.n_q + a.n_kv;
  const int h = is_q ? slotw : (is_v ? slotw - a.n_q - a.n_kv : slotw - a.n_q);
  const int c0 = lane, c1 = lane + 64;
  const i64 xk = in.xk, xm = in.xm, base = in.base;
  const i64 wm0 = in.wm0, wm1 = in.wm1, g0 = in.g0, g1 = in.g1, qs0 = in.qs0, qs1 = in.qs1;
  const i64 kqm0 = in.kqm0, kqm1 = in.kqm1, kqk0 = in.kqk0, kqk1 = in.kqk1;
  const i64 vqm = in.vqm, vqk = in.vqk, ksm = in.ksm, ksk = in.ksk;
  const i64 p0 = in.p0, p1 = in.p1;
  const i64 cs0 = in.cs0, cs1 = in.cs1, sn0 = in.sn0, sn1 = in.sn1;
  const i64 slot = base + t;

  if (is_v) {
    // ---- V head: requant_i8_static(Pv, xm, xk, v_m, v_k, vq_m[h], vq_k[h])
    const i64 shift = wsub(wadd(xk, a.v_k), vqk);
    const i64 up = imax(wneg(shift), 0), down = imax(shift, 0);
    i64 den = shl(vqm, down);
    if (den == 0) den = 1;  // the reference's division raises there
    const int pg = a.kv.page(b, slot);
    int8_t o0, o1;
    // the prefill form's exact fp64 n where the operands allow it
    constexpr i64 WM_LIM = (i64)1 << 21;
    const double xs = (double)xm * ldexp(1.0, (int)imin(up, 64));
    const double nd0 = (double)(int32_t)p0 * (double)(int32_t)wm0 * xs;
    const double nd1 = (double)(int32_t)p1 * (double)(int32_t)wm1 * xs;
    if (DI_LIKELY(den > 0 && den < ((i64)1 << 49) && wm0 > -WM_LIM && wm0 < WM_LIM &&
                  wm1 > -WM_LIM && wm1 < WM_LIM && fabs(nd0) < 0x1p49 && fabs(nd1) < 0x1p49)) {
      const DivEst D = make_divest(den, 1.0);
      o0 = (int8_t)rhad_est_i8_f64(nd0, D);
      o1 = (int8_t)rhad_est_i8_f64(nd1, D);
    } else {
      const i64 n0 = shl(wmul(wmul(p0, wm0), xm), up);
      const i64 n1 = shl(wmul(wmul(p1, wm1), xm), up);
      if (den > 0) {
        const Recip R = make_recip(den);
        o0 = (int8_t)clamp_i8(rhad_r(n0, R));
        o1 = (int8_t)clamp_i8(rhad_r(n1, R));
      } else {  // a wrapped, negative divisor: torch's floor division
        o0 = (int8_t)clamp_i8(rhad(n0, den));
        o1 = (int8_t)clamp_i8(rhad(n1, den));
      }
    }
    if (pg >= 0) {
      a.kv.vchan(pg, h, c0)[slot & (DI_PAGE - 1)] = o0;
      a.kv.vchan(pg, h, c1)[slot & (DI_PAGE - 1)] = o1;
    }
    return;
  }
  const i64 rowk = 20 + a.k_norm_k;
  auto kq = [&](int i) { return kq_channel(i ? kqm1 : kqm0, i ? kqk1 : kqk0, rowk); };
  int o[2];
  i64 am = 1;
  bool done;
  {
    const int32_t pp[2] = {(int32_t)p0, (int32_t)p1}, cc[2] = {(int32_t)cs0, (int32_t)cs1},
                  ss[2] = {(int32_t)sn0, (int32_t)sn1};
    const i64 ww[2] = {wm0, wm1}, gg[2] = {g0, g1}, qq[2] = {qs0, qs1};
    done = qk_head_f64<2, true>(is_q, pp, ww, gg, cc, ss, qq, kq, o, &am);
  }
  if (DI_UNLIKELY(!done)) {
    // the integer routines (same integers, any operands)
    // requant_i32_common(tb = 16) per (token, head)   (model.py:207-211); the
    // (m, k) it returns are dropped by _qk_head_pipeline
    i64 y0 = wmul(p0, wm0), y1 = wmul(p1, wm1);
    {
      const i64 sh = imax(wave_ilog2_absmax(y0, y1) - 15, 0);
      y0 = to_i32(rshift_round(y0, sh));
      y1 = to_i32(rshift_round(y1, sh));
    }
    // di_rmsnorm_gamma  (model.py:212)
    wave_rmsnorm128(y0, y1);
    y0 = wmul(y0, g0);
    y1 = wmul(y1, g1);
    // apply_int_rope at this token's position   (model.py:213-215; rope.py:38-55)
    const i64 r0 = rshift_round(wadd(wmul(y0, cs0), wmul(wneg(y1), sn0)), 14);
    const i64 r1 = rshift_round(wadd(wmul(y1, cs1), wmul(y0, sn1)), 14);
    if (!is_q) {
      // K: requant_i8_static(kk, 1, k_rowk, 1, 0, kq_m, kq_k)   (model.py:326-329)
      const i64 rv[2] = {r0, r1};
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const KqChan c = kq(q);
        const i64 n = shl(rv[q], c.up);
        const i64 lim = (i64)1 << 49;  // 2 |n| + den < 2^51 for rhad_est_i8
        o[q] = (c.den > 0 && c.den < lim && n > -lim && n < lim) ? rhad_est_i8(n, c.D)
                                                               : (int)clamp_i8(rhad(n, c.den));
      }
    } else {
      // Q: QK smoothing (model.py:317-320) then quant_i8_pertoken (model.py:322-323)
      const i64 q0 = wmul(r0, qs0);
      const i64 q1 = wmul(r1, qs1);
      // the head's maximum of |q| as an unsigned value, as in quant_row: a
      // q of INT64_MIN (|q| wraps to itself, skipped by dyadic.py's maximum)
      // reads 2^63 and takes the exact path, which recomputes the maximum
      constexpr u64 top = (u64)1 << 63;
      const u64 amu =
          (u64)wave_max((i64)(::max((u64)wabs(q0), (u64)wabs(q1)) ^ top)) ^ top;
      if (DI_LIKELY(amu < ((u64)1 << 43))) {  // as in quant_row: no 127 q wraps, 255 am < 2^51
        am = imax((i64)amu, 1);
        const DivEst D = make_divest(am, 127.0);
        o[0] = rhad_est_signed(q0, D);
        o[1] = rhad_est_signed(q1, D);
      } else {
        am = DI_UNLIKELY(amu >> 63) ? imax(wave_max(imax(wabs(q0), wabs(q1))), 1) : (i64)amu;
        const Recip R = make_recip(am);
        o[0] = (int)clamp_i8(rhad_r(wmul(q0, 127), R));
        o[1] = (int)clamp_i8(rhad_r(wmul(q1, 127), R));
      }
    }
  }
  if (!is_q) {
    const int pg = a.kv.page(b, slot);
    if (pg >= 0) {
      int8_t* krow = a.kv.krow(pg, h, (int)(slot & (DI_PAGE - 1)));
      krow[c0] = (int8_t)o[0];
      krow[c1] = (int8_t)o[1];
    }
    if (k_lds) {  // the new K row for the fused attention (it may have prefetched the old one)
      k_lds[c0] = (int8_t)o[0];
      k_lds[c1] = (int8_t)o[1];
    }
    return;
  }
  q8_out[c0] = (int8_t)o[0];
  q8_out[c1] = (int8_t)o[1];
  const i64 qrow = (((i64)b * a.n_q + h) * a.T + t);
  if (lane == 0) {
    if (am_out) *am_out = am;
    else *tpos_out = q_head_tpos(a, am, ksm, ksk, a.dbg ? a.dbg + qrow * 4 : nullptr);
  }
}

__device__ __forceinline__ void qkv_head(const QKVArgs& a, int r, int slotw, int8_t* q8_out,
                                         int64_t* tpos_out, int8_t* k_lds = nullptr) {
  QKVHeadIn in = qkv_head_load(a, r, slotw, qkv_scalars(a, r, slotw, slot_base_of(a)));
  qkv_head_rope_load(a, slotw, in);
  qkv_head_compute(a, r, slotw, in, q8_out, tpos_out, k_lds);
  qkv_head_report(a, slotw, in);
}

}  // namespace di

namespace di {

// ---- prefill layout: one wave per (head slot, 4 consecutive token rows) ----
//
// Lane (g, j) = (lane / 16, lane % 16) handles token row r0 + g and the
// channels c_i = 4j + i and c_{i+4} = 64 + 4j + i (i < 4), so RoPE partners
// (c, c + 64) share a lane and every reduction over a row's 128 channels is a
// 16-lane DPP row reduction. Compared with the one-wave-per-(row, head)
// layout above, the per-row scalar chains (scale fits, divisors) run for four
// rows at once and each head's scale vectors are loaded once per four rows.
// Same arithmetic and the same integers as qkv_head.

// The whole wave must be active. Rows r >= R compute on row R - 1 and store
// nothing.
__device__ __forceinline__ void qkv_rows4(const QKVArgs& a, int R, int r0, int slotw) {
  const int lane = threadIdx.x & 63, g = lane >> 4, j = lane & 15;
  const int n_heads = a.n_q + 2 * a.n_kv;
  const bool rok = r0 + g < R;
  const int r = rok ? r0 + g : R - 1;
  const int b = r / a.T, t = r - b * a.T;
  const i64 off = (i64)r * (n_heads * 128) + (i64)slotw * 128;
  const int group = a.n_q / a.n_kv;
  const bool is_q = slotw < a.n_q, is_v = slotw >= a.n_q + a.n_kv;
  const int h = is_q ? slotw : (is_v ? slotw - a.n_q - a.n_kv : slotw - a.n_q);
  const int kvh = is_q ? h / group : h;
  int c[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    c[i] = 4 * j + i;
    c[i + 4] = 64 + 4 * j + i;
  }

  // ---- loads
  const i64 pos_raw = a.positions[r];
  const i64 xk = a.xk[r], xm = a.xm[r];
  const i64 base = slot_base_of(a);
  // (candidates through opaque_ptr, as in qkv_head_load)
  const int64_t* wmp =
      (is_q ? opaque_ptr(a.q_m) : (is_v ? opaque_ptr(a.v_m) : opaque_ptr(a.k_m))) + (i64)h * 128;
  // the head's column mantissas and product sums (loaded again by the
  // integer routines, so the fp64 path does not keep them live)
  auto load_wp = [&](i64 (&wm)[8], i64 (&p)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) wm[i] = ld_global(wmp + c[i]);
    uint32_t s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int k = 0; k < a.nsplit; ++k) {
      const int32_t* pk = a.P + (i64)k * a.split_stride + off;
      const int4 lo = *(const int4*)(pk + 4 * j);
      const int4 hi = *(const int4*)(pk + 64 + 4 * j);
      s[0] += (uint32_t)lo.x; s[1] += (uint32_t)lo.y; s[2] += (uint32_t)lo.z; s[3] += (uint32_t)lo.w;
      s[4] += (uint32_t)hi.x; s[5] += (uint32_t)hi.y; s[6] += (uint32_t)hi.z; s[7] += (uint32_t)hi.w;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = (int32_t)s[i];
  };
  i64 wm[8], p[8];
  load_wp(wm, p);
  const i64 slot = base + t;
  const int pg = rok ? a.kv.page(b, slot) : -1;
  const bool sok = pg >= 0;

  if (is_v) {
    // V head: requant_i8_static(Pv, xm, xk, v_m, v_k, vq_m[h], vq_k[h])
    const i64 vqm = a.vq_m[kvh], vqk = a.vq_k[kvh];
    const i64 shift = wsub(wadd(xk, a.v_k), vqk);
    const i64 up = imax(wneg(shift), 0), down = imax(shift, 0);
    i64 den = shl(vqm, down);
    if (den == 0) den = 1;  // the reference's division raises there
    // n = P w_m x_m << up as an exact double: P w_m is one (|w_m| < 2^21) and
    // the estimate's bound |n| < 2^49 leaves no room for a rounded product
    // (one at or above 2^53 fails it); a lane outside runs the int64 form
    constexpr i64 WM_LIM = (i64)1 << 21;
    bool fast = den > 0 && den < ((i64)1 << 49);
    const double xs = (double)xm * ldexp(1.0, (int)imin(up, 64));
    double nd[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      nd[i] = (double)(int32_t)p[i] * (double)(int32_t)wm[i] * xs;
      fast = fast & in_range(wm[i], WM_LIM) & (fabs(nd[i]) < 0x1p49);
    }
    int8_t o[8];
    if (DI_LIKELY(fast)) {
      const DivEst D = make_divest(den, 1.0);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (int8_t)rhad_est_i8_f64(nd[i], D);
    } else {
      i64 n[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) n[i] = shl(wmul(wmul(p[i], wm[i]), xm), up);
      if (den > 0) {
        const Recip Rr = make_recip(den);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (int8_t)clamp_i8(rhad_r(n[i], Rr));
      } else {  // a wrapped, negative divisor: torch's floor division
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (int8_t)clamp_i8(rhad(n[i], den));
      }
    }
    if (sok) {
#pragma unroll
      for (int i = 0; i < 8; ++i) a.kv.vchan(pg, kvh, c[i])[slot & (DI_PAGE - 1)] = o[i];
    }
    return;
  }
  const int64_t* gam = is_q ? opaque_ptr(a.q_norm_m) : opaque_ptr(a.k_norm_m);
  const i64 pos = torch_index(pos_raw, a.max_pos, (j == 0 && rok) ? a.err : nullptr,
                              DI_ERR_POSITION);
  // the head's gamma, RoPE and smoothing entries (loaded again by the
  // integer routines)
  auto load_ch = [&](i64 (&gm)[8], int32_t (&cs)[8], int32_t (&sn)[8], i64 (&qs)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      gm[i] = ld_global(gam + c[i]);
      cs[i] = a.cos_t[pos * 128 + c[i]];
      sn[i] = a.sin_t[pos * 128 + c[i]];
      qs[i] = a.qs_m[kvh * 128 + c[i]];  // (unconditional: K heads ignore it)
    }
  };
  i64 gm[8], qs[8];
  int32_t cs[8], sn[8], p32[8];
  load_ch(gm, cs, sn, qs);
#pragma unroll
  for (int i = 0; i < 8; ++i) p32[i] = (int32_t)p[i];
  const i64 rowk = 20 + a.k_norm_k;
  auto kq = [&](int i) -> KqChan {
    KqChan q;
    if (a.kq_est) {
      const int64_t* e = a.kq_est + (i64)(kvh * 128 + c[i]) * 4;
      q.den = e[0];
      q.up = e[1];
      q.D.r = __longlong_as_double(e[2]);
      q.D.k = __longlong_as_double(e[3]);
    } else {
      q = kq_channel(a.kq_m[kvh * 128 + c[i]], a.kq_k[kvh * 128 + c[i]], rowk);
    }
    return q;
  };
  int o[8];
  i64 am = 1;
  const bool done = qk_head_f64<8, false>(is_q, p32, wm, gm, cs, sn, qs, kq, o, &am);
  if (DI_UNLIKELY(!done)) {
    // the integer routines (same integers, any operands)
    i64 wm[8], p[8], gm[8], qs[8];
    int32_t cs[8], sn[8];
    load_wp(wm, p);
    load_ch(gm, cs, sn, qs);
    // requant_i32_common(tb = 16) per (token, head)   (model.py:207-211)
    i64 y[8];
    uint32_t L = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      y[i] = wmul(p[i], wm[i]);
      L = ::max(L, bitlen_abs(y[i]));
    }
    {
      const i64 sh = imax(ilog2_from_bitlen(row16_max_u32(L)) - 15, 0);
      L = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        y[i] = to_i32(rshift_round(y[i], sh));
        L = ::max(L, bitlen_abs(y[i]));
      }
    }
    // di_rmsnorm over the 128 channels (model.py:212)
    {
      const i64 sh = 25 - ilog2_from_bitlen(row16_max_u32(L));
      const i64 up = imax(sh, 0), down = imax(-sh, 0);
      i64 ss = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        y[i] = shl(rshift_round(y[i], down), up);
        ss = wadd(ss, wmul(y[i], y[i]));
      }
      const i64 rms = imax(isqrt_est(rhad_pow2(row16_sum64(ss), 7)), 1);
      if (DI_LIKELY(rms > ((i64)1 << 16))) {  // |y| <= 2^26 after the shift: rhad_est
        const DivEst D = make_divest(rms, 1048576.0);
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = rhad_est_signed(y[i], D);
      } else {
        const Recip Rr = make_recip(rms);
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = to_i32(rhad_r(shl(y[i], 20), Rr));
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = wmul(y[i], gm[i]);
    // apply_int_rope at this token's position   (model.py:213-215; rope.py:38-55)
    i64 rv[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      rv[i] = rshift_round(wadd(wmul(y[i], (i64)cs[i]), wmul(wneg(y[i + 4]), (i64)sn[i])), 14);
      rv[i + 4] = rshift_round(wadd(wmul(y[i + 4], (i64)cs[i + 4]), wmul(y[i], (i64)sn[i + 4])), 14);
    }
    if (!is_q) {
      // K: requant_i8_static(kk, 1, k_rowk, 1, 0, kq_m, kq_k)   (model.py:326-329)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const KqChan q = kq(i);
        const i64 n = shl(rv[i], q.up);
        const i64 lim = (i64)1 << 49;  // 2 |n| + den < 2^51 for rhad_est_i8
        o[i] = (q.den > 0 && q.den < lim && n > -lim && n < lim) ? rhad_est_i8(n, q.D)
                                                                 : (int)clamp_i8(rhad(n, q.den));
      }
    } else {
      // Q: QK smoothing (model.py:317-320) then quant_i8_pertoken (model.py:322-323)
      i64 q[8];
      u64 amx = 0;  // unsigned: a q of INT64_MIN reads 2^63 (see the one-token form)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        q[i] = wmul(rv[i], qs[i]);
        amx = ::max(amx, (u64)wabs(q[i]));
      }
      constexpr u64 top = (u64)1 << 63;
      const u64 amu = (u64)row16_max64((i64)(amx ^ top)) ^ top;
      if (DI_LIKELY(amu < ((u64)1 << 43))) {  // as in quant_row: no 127 q wraps, 255 am < 2^51
        am = imax((i64)amu, 1);
        const DivEst D = make_divest(am, 127.0);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = rhad_est_signed(q[i], D);
      } else {
        if (DI_UNLIKELY(amu >> 63)) {  // uniform over the row's 16 lanes
          i64 sx = 0;
#pragma unroll
          for (int i = 0; i < 8; ++i) sx = imax(sx, wabs(q[i]));
          am = imax(row16_max64(sx), 1);
        } else {
          am = (i64)amu;
        }
        const Recip Rr = make_recip(am);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (int)clamp_i8(rhad_r(wmul(q[i], 127), Rr));
      }
    }
  }
  uint32_t w[2] = {0, 0};
#pragma unroll
  for (int i = 0; i < 8; ++i) w[i >> 2] |= (uint32_t)(uint8_t)(int8_t)o[i] << (8 * (i & 3));
  if (!is_q) {
    if (sok) {
      int8_t* krow = a.kv.krow(pg, h, (int)(slot & (DI_PAGE - 1)));
      *(uint32_t*)(krow + 4 * j) = w[0];
      *(uint32_t*)(krow + 64 + 4 * j) = w[1];
    }
    return;
  }
  const i64 qkk = 20 + a.q_norm_k + a.qs_k;
  i64 m, k;
  norm_scale(1, qkk, &m, &k);
  const i64 qrow = ((i64)b * a.n_q + h) * a.T + t;
  if (rok) {
    *(uint32_t*)(a.q8 + qrow * 128 + 4 * j) = w[0];
    *(uint32_t*)(a.q8 + qrow * 128 + 64 + 4 * j) = w[1];
  }
  if (j == 0 && rok) {
    const i64 ksm = a.ks_m[kvh], ksk = a.ks_k[kvh];
    i64 qm, e;
    fit_dyadic_ratio_127(wmul(am, m), &qm, &e);
    const i64 qk = wadd(k, e);
    // score scale: norm_scale(qm * ks_m[h//g], qk + ks_k[h//g])   (model.py:351-353)
    i64 sm, sk;
    norm_scale(wmul(qm, ksm), wadd(qk, ksk), &sm, &sk);
    a.tpos[qrow] = di_exp_tpos_fast(sm, sk);
    if (a.dbg) {
      a.dbg[qrow * 4 + 0] = qm;
      a.dbg[qrow * 4 + 1] = qk;
      a.dbg[qrow * 4 + 2] = sm;
      a.dbg[qrow * 4 + 3] = sk;
    }
  }
}

}  // namespace di
