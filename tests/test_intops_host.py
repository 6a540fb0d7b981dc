"""CPU checks of intops.h — the integer routines every HIP kernel shares —
through its host build (libdetllm_intops_host.so).

Pinned against Python's exact integer arithmetic (division by invariant
divisors near multiples of d, at int64 extremes) and against the oracle,
which is itself pinned to the reference's golden vectors."""

import ctypes
import os
import random

import numpy as np
import pytest

from oracle import dyadic as ody
from oracle import intmath as oim
from oracle import ops as oops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "idempotent_llm_amd", "libdetllm_intops_host.so")
I64 = np.int64


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(HOST):
        from idempotent_llm_amd.build import build_host_shim
        build_host_shim()
    return ctypes.CDLL(HOST)


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _call2(lib, name, a, b):
    a = np.ascontiguousarray(a, I64)
    b = np.ascontiguousarray(b, I64)
    out = np.empty_like(a)
    getattr(lib, name)(_p(a), _p(b), ctypes.c_int64(a.size), _p(out))
    return out


def _py_floor_div(a, d):
    return a // d


def _py_rhad(a, d):
    q = (abs(a) + d // 2) // d
    return -q if a < 0 else q


def _wrap(v):
    v &= (1 << 64) - 1
    return v - (1 << 64) if v >= 1 << 63 else v


def _divisor_cases(seed=0, n=40000):
    rnd = random.Random(seed)
    A, D = [], []
    ds = [1, 2, 3, 7, 127, 128, 1 << 20, (1 << 31) - 1, 1 << 31, (1 << 32) + 1,
          (1 << 47) - 3, (1 << 62) + 11, (1 << 63) - 1]
    ds += [rnd.randrange(1, 1 << rnd.randrange(1, 63)) for _ in range(200)]
    for d in ds:
        for _ in range(n // len(ds)):
            kind = rnd.randrange(4)
            if kind == 0:       # near a multiple of d
                q = rnd.randrange(0, max(1, ((1 << 63) - 1) // d))
                a = q * d + rnd.choice([-1, 0, 1, d // 2, d // 2 + 1, (d - 1) // 2])
            elif kind == 1:
                a = rnd.randrange(-(1 << 63), 1 << 63)
            elif kind == 2:
                a = rnd.randrange(-(1 << 24), 1 << 24)
            else:
                a = rnd.choice([0, 1, -1, (1 << 63) - 1, -(1 << 63) + 1, -(1 << 63)])
            a = max(-(1 << 63), min((1 << 63) - 1, a))
            A.append(a)
            D.append(d)
    return np.array(A, dtype=I64), np.array(D, dtype=I64)


def test_floor_div_by_reciprocal_exact(lib):
    A, D = _divisor_cases(1)
    got = _call2(lib, "di_host_floor_div_r", A, D)
    want = [_py_floor_div(int(a), int(d)) for a, d in zip(A, D)]
    assert got.tolist() == want


def test_rhad_by_reciprocal_matches_generic_and_python(lib):
    A, D = _divisor_cases(2)
    got_r = _call2(lib, "di_host_rhad_r", A, D)
    got = _call2(lib, "di_host_rhad", A, D)
    # the reference's formula on wrapping int64: mag + half may wrap
    want = []
    for a, d in zip(A.tolist(), D.tolist()):
        mag = _wrap(abs(a)) if a != -(1 << 63) else -(1 << 63)
        s = _wrap(mag + d // 2)
        q = s // d
        want.append(_wrap(-q) if a < 0 else q)
    assert got.tolist() == want
    assert got_r.tolist() == want


def test_rshift_round_matches_oracle(lib):
    rnd = np.random.default_rng(3)
    a = np.concatenate([rnd.integers(-(1 << 62), 1 << 62, 20000, dtype=I64),
                        np.array([0, -1, 1, (1 << 63) - 1, -(1 << 63)], I64)])
    k = rnd.integers(0, 70, a.size, dtype=I64)
    got = _call2(lib, "di_host_rshift_round", a, k)
    assert np.array_equal(got, oim.rshift_round_t(a, k))


def test_di_exp_matches_oracle(lib):
    rnd = np.random.default_rng(4)
    rows = 64
    m = rnd.integers(1 << 15, 1 << 16, (rows, 1), dtype=I64)
    k = rnd.integers(5, 62, (rows, 1), dtype=I64)
    x = -rnd.integers(0, 1 << 40, (rows, 300), dtype=I64)
    x[:, 0] = 0
    want, tpos = oops.di_exp(x, m, k)
    t = _call2(lib, "di_host_di_exp_tpos", m.ravel(), k.ravel())
    assert np.array_equal(t, tpos.ravel())
    got = _call2(lib, "di_host_di_exp", x.ravel(), np.broadcast_to(tpos, x.shape).ravel())
    assert np.array_equal(got.reshape(x.shape), want)


def test_sigmoid_div_matches_rhad(lib):
    rnd = np.random.default_rng(5)
    den = rnd.integers(1, 1 << 50, 20000, dtype=I64)
    num = (den * rnd.integers(0, 1001, den.size) // 1000).astype(I64)
    num[:5] = den[:5]
    num[5:10] = 0
    got = _call2(lib, "di_host_sigmoid_div", num, den)
    assert np.array_equal(got, oim.rhad(oim.shl(num, 7), den))


def test_swiglu_elem_matches_oracle(lib):
    rnd = np.random.default_rng(6)
    rows, C = 16, 777
    gate = rnd.integers(-(1 << 14), (1 << 14) + 1, (rows, C), dtype=I64)
    up = rnd.integers(-(1 << 14), (1 << 14) + 1, (rows, C), dtype=I64)
    gm = rnd.integers(1 << 15, 1 << 16, (rows, 1), dtype=I64)
    gk = rnd.integers(10, 40, (rows, 1), dtype=I64)
    y, _, _ = oops.di_swiglu(gate, gm, gk, up, gm, gk)
    tpos = oops.di_exp_tpos(gm, gk)
    g = np.ascontiguousarray(gate.ravel())
    u = np.ascontiguousarray(up.ravel())
    t = np.ascontiguousarray(np.broadcast_to(tpos, gate.shape).ravel())
    out = np.empty_like(g)
    lib.di_host_swiglu(_p(g), _p(u), _p(t), ctypes.c_int64(g.size), _p(out))
    assert np.array_equal(out.reshape(gate.shape), y)


def _scalar(lib, op, a, b=None, c=None):
    a = np.ascontiguousarray(a, I64)
    b = np.ascontiguousarray(b if b is not None else np.zeros_like(a), I64)
    c = np.ascontiguousarray(c if c is not None else np.zeros_like(a), I64)
    o1 = np.empty_like(a)
    o2 = np.empty_like(a)
    lib.di_host_scalar(ctypes.c_int(op), _p(a), _p(b), _p(c), ctypes.c_int64(a.size), _p(o1),
                       _p(o2))
    return o1, o2


def test_scalar_ops_match_oracle(lib, golden_dir):
    D = dict(np.load(os.path.join(golden_dir, "dyadic.npz")))
    rnd = np.random.default_rng(7)
    v = np.concatenate([rnd.integers(-(1 << 62), 1 << 62, 20000, dtype=I64),
                        np.arange(-5, 70000, dtype=I64)])
    assert np.array_equal(_scalar(lib, 0, v)[0], oim.isqrt(v))
    assert np.array_equal(_scalar(lib, 1, v)[0], oim.ilog2(v))
    m2, k2 = _scalar(lib, 2, D["ns_m"], D["ns_k"])
    assert np.array_equal(m2, D["ns_m2"]) and np.array_equal(k2, D["ns_k2"])
    m, e = _scalar(lib, 3, D["fit_num"], D["fit_den"])
    assert np.array_equal(m, D["fit_m"]) and np.array_equal(e, D["fit_e"])
    out, _ = _scalar(lib, 4, D["srd_num"], D["srd_den"], D["srd_e"])
    assert np.array_equal(out, D["srd_out"])
    m, e = _scalar(lib, 3, D["fit_num"], np.full_like(D["fit_num"], 127))
    assert np.array_equal(m, D["fit127_m"]) and np.array_equal(e, D["fit127_e"])
    wm, we = ody.norm_scale(D["ns_m"], D["ns_k"])
    assert np.array_equal(wm, m2) and np.array_equal(we, k2)


def test_fit127_fast_path_matches_generic_and_golden(lib, golden_dir):
    """fit_dyadic_ratio(num, 127) through the constant-127 reciprocal path
    (what every fused kernel runs) equals the generic routine and the
    reference's golden vectors, across the fast-path boundary (2^62) and at
    the adjustment edges (mantissas near 2^15 and 2^16)."""
    D = dict(np.load(os.path.join(golden_dir, "dyadic.npz")))
    m, e = _scalar(lib, 5, D["fit_num"])
    assert np.array_equal(m, D["fit127_m"]) and np.array_equal(e, D["fit127_e"])
    rnd = np.random.default_rng(11)
    num = np.concatenate([
        rnd.integers(1, 1 << 62, 50000, dtype=I64),
        (I64(1) << rnd.integers(0, 62, 20000).astype(I64)) + rnd.integers(-3, 4, 20000),
        np.arange(1, 5000, dtype=I64),
        np.array([(1 << 56) - 1, 1 << 56, (1 << 56) + 1, (1 << 55) + 12345, 127, 254, 127 << 20,
                  (127 << 20) - 1, (1 << 63) - 1, (1 << 62) - 1, 1 << 62, (1 << 62) + 1,
                  (1 << 62) - (127 << 40), (1 << 61) + (127 << 39) - 1], I64),
        rnd.integers(1 << 56, 1 << 62, 20000, dtype=I64)])
    num = num[num > 0]
    fm, fe = _scalar(lib, 5, num)
    gm, ge = _scalar(lib, 3, num, np.full_like(num, 127))
    assert np.array_equal(fm, gm) and np.array_equal(fe, ge)
    om, oe = ody.fit_dyadic_ratio(num, 127)
    assert np.array_equal(fm, om) and np.array_equal(fe, oe)


def test_floor_div127_estimate(lib):
    """floor(y / 127) from one fp64 fma (the divisions inside the constant-127
    fit): every y below 2^20, and around every multiple of 127 up to 2^32 in
    strides, against integer division."""
    ks = np.arange(0, (1 << 32) // 127, 997, dtype=I64)
    y = np.concatenate([np.arange(0, 1 << 20, dtype=I64)] +
                       [ks * 127 + d for d in (-1, 0, 1, 63, 126)] +
                       [np.array([(1 << 32) - 1, (1 << 32) - 2, (1 << 24) - 1, 1 << 24], I64)])
    y = y[(y >= 0) & (y < (1 << 32))]
    got, _ = _scalar(lib, 9, y)
    assert np.array_equal(got, y // 127)


def test_rhad_pow2_matches_rhad(lib):
    rnd = np.random.default_rng(12)
    a = np.concatenate([rnd.integers(-(1 << 63), (1 << 63) - 1, 40000, dtype=I64, endpoint=True),
                        np.array([-(1 << 63), (1 << 63) - 1, 0, 1, -1, 511, 512, -512, 513], I64)])
    for k in (0, 1, 7, 10, 20, 40, 62):
        got, _ = _scalar(lib, 6, a, np.full_like(a, k))
        want = _call2(lib, "di_host_rhad", a, np.full_like(a, 1 << k))
        assert np.array_equal(got, want), k


def _call2_3(lib, name, a, b, c=None):
    a = np.ascontiguousarray(a, I64)
    b = np.ascontiguousarray(b, I64)
    out = np.empty_like(a)
    if c is None:
        getattr(lib, name)(_p(a), _p(b), ctypes.c_int64(a.size), _p(out))
    else:
        c = np.ascontiguousarray(c, I64)
        getattr(lib, name)(_p(a), _p(b), _p(c), ctypes.c_int64(a.size), _p(out))
    return out


def test_di_exp_neg_32bit_path_matches_generic(lib):
    """The 32-bit DI-Exp (tpos < 2^31, neg < 2^32) equals the 64-bit form
    di_exp_r(-neg) for tpos on both sides of 2^31, neg near multiples of tpos
    and across the 2^32 boundary."""
    rnd = np.random.default_rng(31)
    tp = np.concatenate([np.arange(1, 300, dtype=I64),
                         rnd.integers(1, 1 << 31, 3000, dtype=I64),
                         np.array([(1 << 31) - 1, 1 << 31, (1 << 31) + 1, 1 << 40], I64)])
    tpos = np.repeat(tp, 40)
    k = rnd.integers(0, 70, tpos.size)
    jitter = rnd.integers(-2, 3, tpos.size)
    neg = np.clip(tpos * k + jitter, 0, None).astype(I64)
    neg[::7] = rnd.integers(0, 1 << 33, neg[::7].size)
    neg[::11] = (1 << 32) - 1 - rnd.integers(0, 3, neg[::11].size)
    got = _call2_3(lib, "di_host_di_exp_neg", neg, tpos)
    want = _call2_3(lib, "di_host_di_exp", -neg, tpos)
    assert np.array_equal(got, want)   # di_host_di_exp is pinned to the oracle above


def test_sigmoid_div32_matches_64bit(lib):
    rnd = np.random.default_rng(32)
    den = np.concatenate([rnd.integers(1, 1 << 31, 50000, dtype=I64),
                          np.array([1, 2, 3, 127, 128, 255, (1 << 31) - 1], I64)])
    num = (rnd.random(den.size) * (den + 1)).astype(I64)
    num = np.minimum(num, den)
    num[::5] = den[::5]
    num[::9] = 0
    got = _call2_3(lib, "di_host_sigmoid_div32", num, den)
    want = _call2_3(lib, "di_host_sigmoid_div", num, den)
    assert np.array_equal(got, want)
    py = [((int(a) << 7) + int(b) // 2) // int(b) for a, b in zip(num[:2000], den[:2000])]
    assert got[:2000].tolist() == py


def test_swiglu_elem_fast_path_matches_generic(lib):
    rnd = np.random.default_rng(33)
    n = 60000
    g = np.concatenate([rnd.integers(-(1 << 15), 1 << 15, n // 2),
                        rnd.integers(-(1 << 31), 1 << 31, n // 2)]).astype(I64)
    u = rnd.integers(-(1 << 15), 1 << 15, n).astype(I64)
    tpos = np.concatenate([rnd.integers(1, 1 << 20, n // 3), rnd.integers(1, 1 << 30, n // 3),
                           rnd.integers(1 << 29, 1 << 33, n - 2 * (n // 3))]).astype(I64)
    got = _call2_3(lib, "di_host_swiglu_e", g, u, tpos)
    want = _call2_3(lib, "di_host_swiglu", g, u, tpos)
    assert np.array_equal(got, want)


# ------------------------------------------- exact integers from fp64 estimates

def _rhad_est_cases(seed=11):
    rnd = random.Random(seed)
    M, D, S = [], [], []
    scales = [1.0, 127.0, float(1 << 14), float(1 << 20)]
    ds = [1, 2, 3, 5, 127, 128, 255, 4097, (1 << 20) + 1, (1 << 31) - 1, (1 << 34) - 3,
          (1 << 40) + 7, (1 << 47) - 1]
    ds += [rnd.randrange(1, 1 << rnd.randrange(1, 48)) for _ in range(300)]
    for d in ds:
        for s in scales:
            si = int(s)
            # m s + d/2 < 2^32 d (quotient below 2^32) and 2 m s + d < 2^51
            mmax = min(((1 << 51) - d) // (2 * si), ((1 << 32) * d - d // 2) // si - 1)
            if mmax < 0:
                continue
            for _ in range(24):
                kind = rnd.randrange(4)
                if kind == 0:   # numerator at / next to a multiple of d
                    q = rnd.randrange(0, max(1, mmax * si // d + 1))
                    tgt = q * d - d // 2 + rnd.choice([-1, 0, 1])
                    m = max(0, min(mmax, tgt // si + rnd.choice([0, 1])))
                elif kind == 1:
                    m = rnd.randrange(0, mmax + 1)
                elif kind == 2:
                    m = mmax - rnd.randrange(0, min(mmax, 16) + 1)
                else:
                    m = rnd.randrange(0, min(mmax, 4 * d) + 1)
                M.append(m)
                D.append(d)
                S.append(s)
    return np.array(M, I64), np.array(D, I64), np.array(S, np.float64)


def test_rhad_est_exact(lib):
    """rhad_est (fp64 estimate, intops.h) equals floor((m s + floor(d/2)) / d)
    in exact integer arithmetic across divisor magnitudes 1..2^47, the scales
    the kernels use, numerators at multiples of d and at the stated bound."""
    M, D, S = _rhad_est_cases()
    out = np.empty_like(M)
    lib.di_host_rhad_est(_p(M), _p(D), _p(S), ctypes.c_int64(M.size), _p(out))
    want = [(int(m) * int(s) + int(d) // 2) // int(d) for m, d, s in zip(M, D, S)]
    assert out.tolist() == want


def test_sigmoid_est_matches_restoring_division(lib):
    """sigmoid_est == round_half_away_div(num << 7, den) for num <= den < 2^31,
    including every num for small den and ties."""
    rnd = random.Random(5)
    num, den = [], []
    for d in range(1, 300):
        for n in range(0, d + 1):
            num.append(n)
            den.append(d)
    for _ in range(200000):
        d = rnd.randrange(1, 1 << rnd.randrange(1, 32))
        d = min(d, (1 << 31) - 1)
        num.append(rnd.choice([0, d, d - 1, d // 2, rnd.randrange(0, d + 1)]))
        den.append(d)
    num = np.array(num, I64)
    den = np.array(den, I64)
    got = _call2(lib, "di_host_sigmoid_est", num, den)
    want = [(int(n) * 128 + int(d) // 2) // int(d) for n, d in zip(num, den)]
    assert got.tolist() == want


def _sigmoid24_cases(seed):
    """(num, den) pairs for the single-precision sigmoid division: every num
    for den < 300, the top of the range and random pairs over every bit
    length up to 24, with num at 0, den, den - 1, den / 2 and random."""
    rnd = random.Random(seed)
    num, den = [], []
    for d in list(range(1, 300)) + [(1 << 24) - 1, (1 << 24) - 2, (1 << 23) + 1, 1 << 23]:
        for n in (range(0, d + 1) if d < 300 else [0, 1, d // 2, d // 2 + 1, d - 1, d]):
            num.append(n)
            den.append(d)
    for _ in range(300000):
        d = rnd.randrange(1, 1 << rnd.randrange(1, 25))
        num.append(rnd.choice([0, d, d - 1, d // 2, rnd.randrange(0, d + 1)]))
        den.append(d)
    return np.array(num, I64), np.array(den, I64)


def test_sigmoid_est24_matches_restoring_division(lib):
    """sigmoid_est24 (single-precision reciprocal plus one remainder step) ==
    round_half_away_div(num << 7, den) for num <= den < 2^24."""
    num, den = _sigmoid24_cases(7)
    got = _call2(lib, "di_host_sigmoid_est24", num, den)
    want = [(int(n) * 128 + int(d) // 2) // int(d) for n, d in zip(num, den)]
    assert got.tolist() == want


@pytest.mark.parametrize("tpos", [1, 2, 3, 7, 100, 4095, 4096, 46341, 65537, 360626,
                                  (1 << 22) + 1, (1 << 23) - 1])
def test_dexp_est_exhaustive(lib, tpos):
    """dexp_est(n) and dexp_est_sp(t - n) equal the integer DI-Exp (di_exp_r,
    pinned to the oracle above) for every n < 2^22 at tpos up to 2^23 - 1."""
    lib.di_host_dexp_est_mismatches.restype = ctypes.c_int64
    bad = lib.di_host_dexp_est_mismatches(ctypes.c_int64(tpos), ctypes.c_int64(0),
                                          ctypes.c_int64(1 << 22))
    assert bad == 0


def test_di_exp_tpos_fast_matches_oracle(lib):
    """di_exp_tpos_fast (division by m_f from the fp64 estimate where its
    bounds hold) equals the oracle's DI-Exp constant for mantissas across
    and beyond the normalised range and shifts k from -3 to 66."""
    rnd = np.random.default_rng(17)
    m = np.concatenate([rnd.integers(1 << 15, 1 << 16, 40000, dtype=I64),
                        rnd.integers(1, 1 << 40, 10000, dtype=I64),
                        np.array([1, 2, 10, 32767, 32768, 65535, 65536, (1 << 31) - 1], I64)])
    k = rnd.integers(-3, 67, m.size, dtype=I64)
    k[:70] = np.arange(-3, 67)
    got, _ = _scalar(lib, 7, m, k)
    assert np.array_equal(got, oops.di_exp_tpos(m, k))


def test_swiglu_elem_est_matches_oracle(lib):
    """The fused kernel's SwiGLU element (dexp_est + sigmoid_est) equals the
    oracle's di_swiglu (ops/di_swiglu.py:39-58) for |g|, |u| <= 2^14 and
    tpos < 2^23: every g in [-2^14, 2^14] at a few row scales, random pairs
    elsewhere; tpos comes from the oracle's constant for each (gm, gk)."""
    rnd = np.random.default_rng(41)
    full = np.arange(-(1 << 14), (1 << 14) + 1, dtype=I64)
    n = 200000
    g = np.concatenate([full] * 4 + [rnd.integers(-(1 << 14), (1 << 14) + 1, n, dtype=I64)])
    gm = np.concatenate([np.full(full.size, m, I64) for m in (32768, 40000, 50000, 65535)]
                        + [rnd.integers(1 << 15, 1 << 16, n, dtype=I64)])
    gk = np.concatenate([np.full(full.size, k, I64) for k in (15, 28, 31, 38)]
                        + [rnd.integers(0, 39, n, dtype=I64)])
    tpos = oops.di_exp_tpos(gm, gk)
    keep = tpos < (1 << 23)
    g, gm, gk, tpos = g[keep], gm[keep], gk[keep], tpos[keep]
    u = rnd.integers(-(1 << 14), (1 << 14) + 1, g.size, dtype=I64)
    got = _call2_3(lib, "di_host_swiglu_est", g, u, tpos)
    want, _, _ = oops.di_swiglu(g, gm, gk, u, np.ones_like(u), np.zeros_like(u))
    assert g.size > 150000 and np.array_equal(got, want)


def _est_op(lib, op, a, d, s):
    a, d, s = (np.ascontiguousarray(x, I64) for x in (a, d, s))
    out = np.empty_like(a)
    lib.di_host_rhad_est_op(ctypes.c_int(op), _p(a), _p(d), _p(s), ctypes.c_int64(a.size), _p(out))
    return out


def test_rhad_est_signed_i8_and_corrected(lib):
    """The signed, int8-clamped and remainder-corrected fp64-estimate
    divisions of the row kernels against exact rhad (Python integers) at
    their stated bounds: quantisation (s = 127, |a| <= d < 2^43), RMSNorm
    (s = 2^20, |a| <= 2^26), static requant (s = 1, |a|, d < 2^49, clamped),
    merge (s = 127, |a| <= d < 2^46, corrected), large-row quantisation
    (s = 127, |a| <= d < 2^53, corrected)."""
    rnd = random.Random(23)

    def rh(a, d):
        q = (abs(a) + d // 2) // d
        return -q if a < 0 else q

    def near_ties(d, s, amax, n):
        out = []
        for _ in range(n):
            q = rnd.randrange(0, 128)
            t = (q * d - d // 2) // s + rnd.choice([-1, 0, 1])
            a = max(-amax, min(amax, t * rnd.choice([1, -1])))
            out.append(a)
        return out

    # quantisation: |a| <= d < 2^43
    A, D = [], []
    for _ in range(4000):
        d = rnd.randrange(1, 1 << rnd.randrange(1, 43))
        for a in near_ties(d, 127, d, 3) + [rnd.randrange(-d, d + 1), d, -d, 0]:
            A.append(a)
            D.append(d)
    got = _est_op(lib, 0, A, D, [127] * len(A))
    assert got.tolist() == [rh(127 * a, d) for a, d in zip(A, D)]
    # RMSNorm: |a| <= 2^26, d in (2^16, 2^26]
    A, D = [], []
    for _ in range(20000):
        d = rnd.randrange((1 << 16) + 1, (1 << 26) + 1)
        a = rnd.choice([rnd.randrange(-(1 << 26), (1 << 26) + 1), (1 << 26), -(1 << 26),
                        ((rnd.randrange(0, 1 << 15) * d - d // 2) >> 20) + rnd.choice([-1, 0, 1])])
        A.append(a)
        D.append(d)
    got = _est_op(lib, 0, A, D, [1 << 20] * len(A))
    assert got.tolist() == [rh(a << 20, d) for a, d in zip(A, D)]
    # static requant to int8, clamped: |a|, d < 2^49
    A, D = [], []
    for _ in range(20000):
        d = rnd.randrange(1, 1 << rnd.randrange(1, 49))
        q = rnd.choice([rnd.randrange(0, 300), rnd.randrange(0, 1 << 20)])
        a = q * d - d // 2 + rnd.choice([-1, 0, 1, rnd.randrange(0, d)])
        a = max(-(1 << 49) + 1, min((1 << 49) - 1, a * rnd.choice([1, -1])))
        A.append(a)
        D.append(d)
    got = _est_op(lib, 1, A, D, [1] * len(A))
    assert got.tolist() == [max(-128, min(127, rh(a, d))) for a, d in zip(A, D)]
    # merge: |a| <= d < 2^46 with the correction step
    A, D = [], []
    for _ in range(6000):
        d = rnd.randrange(1 << 40, 1 << 46)
        for a in near_ties(d, 127, d, 3) + [rnd.randrange(-d, d + 1), d, -d]:
            A.append(a)
            D.append(d)
    got = _est_op(lib, 2, A, D, [127] * len(A))
    assert got.tolist() == [rh(127 * a, d) for a, d in zip(A, D)]
    # quantisation of rows with a maximum in [2^43, 2^53): |a| <= d < 2^53
    # with the correction step (the fp64 row quantiser's large-row path)
    A, D = [], []
    for _ in range(8000):
        d = rnd.randrange(1 << 43, 1 << rnd.randrange(44, 54))
        for a in near_ties(d, 127, d, 3) + [rnd.randrange(-d, d + 1), d, -d]:
            A.append(a)
            D.append(d)
    for d in ((1 << 53) - 1, (1 << 53) - 2, (1 << 52) + 1, 1 << 43):
        for a in (d, -d, d - 1, (d - 1) // 2, d // 127, -(d // 127) - 1, 0):
            A.append(a)
            D.append(d)
    got = _est_op(lib, 2, A, D, [127] * len(A))
    assert got.tolist() == [rh(127 * a, d) for a, d in zip(A, D)]


def test_isqrt_est_matches_oracle(lib):
    """isqrt_est (fp64 square root + one integer step each way) equals the
    oracle's isqrt (int_prims.py bitwise method) below 2^62: random values at
    every magnitude, perfect squares and their neighbours."""
    rnd = np.random.default_rng(29)
    r = rnd.integers(0, 1 << 31, 30000, dtype=I64)
    sq = r * r
    v = np.concatenate([sq, sq - 1, sq + 1, sq + 2 * r, sq + 2 * r + 1,
                        (rnd.random(30000) * 2.0 ** rnd.integers(0, 62, 30000)).astype(I64),
                        np.arange(-3, 5000, dtype=I64)])
    v = v[(v < (1 << 62))]
    got, _ = _scalar(lib, 8, v)
    assert np.array_equal(got, oim.isqrt(v))


def test_in_range_bounds(lib):
    """in_range(x, lim) (the row kernels' branch-free operand bounds) is
    -lim < x < lim, at both edges and the int64 extremes, for every limit
    the kernels use and random others."""
    rnd = np.random.default_rng(78)
    lims = [1 << 12, 1 << 15, 1 << 18, 1 << 21, 1, 2, 3] + [int(v) for v in rnd.integers(1, 1 << 40, 20)]
    xs, ls = [], []
    for lim in lims:
        for x in (-lim - 1, -lim, -lim + 1, -1, 0, 1, lim - 1, lim, lim + 1,
                  -(1 << 63), (1 << 63) - 1, -(1 << 62), (1 << 62)):
            xs.append(x); ls.append(lim)
        for x in rnd.integers(-(2 * lim), 2 * lim + 1, 50):
            xs.append(int(x)); ls.append(lim)
    x = np.array(xs, dtype=np.int64); b = np.array(ls, dtype=np.int64)
    out = np.empty_like(x)
    lib.di_host_f64_int_op(ctypes.c_int(5), _p(x), _p(b), ctypes.c_int64(x.size), _p(out))
    assert [int(v) for v in out] == [int(-l < v < l) for v, l in zip(xs, ls)]


def test_f64_integer_helpers(lib):
    """bitlen_f64 (the fp64 exponent) and bitlen_from_hiword (the exponent in
    the high word of |x|) equal int.bit_length of |x|, and
    rshift_round_f64 equals rshift_round (intmath.py:120-147, (x + 2^(sh-1))
    >> sh with floor) for |x| < 2^52 and every shift from 0 to 70, on random
    magnitudes of every size, exact powers of two and their neighbours, and
    the halfway cases x = (2j + 1) 2^(sh-1)."""
    rnd = np.random.default_rng(77)
    mags = np.concatenate([rnd.integers(0, 1 << 52, 20000),
                           (1 << rnd.integers(0, 52, 2000)).astype(np.int64)])
    mags = np.concatenate([mags, np.maximum(mags - 1, 0), np.minimum(mags + 1, (1 << 52) - 1)])
    sign = np.where(rnd.integers(0, 2, mags.size) == 1, -1, 1)
    x = (mags * sign).astype(np.int64)
    out = np.empty_like(x)
    lib.di_host_f64_int_op(ctypes.c_int(0), _p(x), _p(x), ctypes.c_int64(x.size), _p(out))
    assert [int(v) for v in out] == [abs(int(v)).bit_length() for v in x]
    # the same bit length from the high word of |x| (bitlen_from_hiword)
    lib.di_host_f64_int_op(ctypes.c_int(4), _p(x), _p(x), ctypes.c_int64(x.size), _p(out))
    assert [int(v) for v in out] == [abs(int(v)).bit_length() for v in x]
    for sh in range(0, 71):
        xs = x.copy()
        if 1 <= sh <= 51:   # halfway cases
            j = rnd.integers(-(1 << (51 - sh)), 1 << (51 - sh), 500)
            xs = np.concatenate([xs[:5000], ((2 * j + 1) << (sh - 1)).astype(np.int64)])
        k = np.full(xs.size, sh, dtype=np.int64)
        lib.di_host_f64_int_op(ctypes.c_int(1), _p(xs), _p(k), ctypes.c_int64(xs.size),
                               _p(out[:xs.size]))
        want = [int(v) if sh == 0 else (int(v) + (1 << (sh - 1))) >> sh for v in xs]
        assert [int(v) for v in out[:xs.size]] == want, sh


def test_f64_division_estimates(lib):
    """rhad_est_i8_f64 equals clamp_i8(rhad(n, d)) and rhad_est_signed_f64
    equals sign(a) rhad(127 |a|, d) (intmath.py:60-80 rhad, :150-153 clamp)
    on integer-valued doubles within the estimates' bounds (2 |n| + d and
    2 127 |a| + d below 2^51): random magnitudes of every size, exact
    multiples of the divisor, the halfway cases, and every divisor size."""
    rnd = np.random.default_rng(78)
    n = 40000
    d = np.concatenate([rnd.integers(1, 64, n // 4), (1 << rnd.integers(0, 48, n // 4)),
                        rnd.integers(1, 1 << 48, n // 2)]).astype(np.int64)
    rnd.shuffle(d)
    # clamp_i8(rhad(n, d)): quotients around the clamp and far beyond it
    q = rnd.integers(-300, 301, n)
    r = np.where(rnd.integers(0, 3, n) == 0, d // 2, rnd.integers(0, np.maximum(d, 1)))
    num = q * d + np.where(q < 0, -r, r)
    num = np.where(np.abs(num) < (1 << 49), num, rnd.integers(-(1 << 40), 1 << 40, n))
    out = np.empty_like(num)
    lib.di_host_f64_int_op(ctypes.c_int(2), _p(num), _p(d), ctypes.c_int64(n), _p(out))
    want = [max(-128, min(127, _py_rhad(int(a), int(b)))) for a, b in zip(num, d)]
    assert [int(v) for v in out] == want
    # sign(a) rhad(127 |a|, d) with |a| <= d (quantiser quotients <= 127)
    a = (rnd.random(n) * d).astype(np.int64) * np.where(rnd.integers(0, 2, n) == 1, -1, 1)
    a = np.where(rnd.integers(0, 4, n) == 0, np.sign(a) * d, a).astype(np.int64)
    lib.di_host_f64_int_op(ctypes.c_int(3), _p(a), _p(d), ctypes.c_int64(n), _p(out))
    want = [(-1 if v < 0 else 1) * _py_rhad(127 * abs(int(v)), int(b)) for v, b in zip(a, d)]
    assert [int(v) for v in out] == want
