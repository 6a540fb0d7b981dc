"""Pin the oracle's dyadic and operator functions against golden vectors
written from the reference CPU path (tests/golden/make_golden.py), and
against the exact special cases the reference's own tests assert."""

import os

import numpy as np
import pytest

from oracle import dyadic as dy
from oracle import ops

HERE = os.path.dirname(os.path.abspath(__file__))
I64 = np.int64


@pytest.fixture(scope="module")
def D():
    return dict(np.load(os.path.join(HERE, "golden", "dyadic.npz")))


@pytest.fixture(scope="module")
def O():
    return dict(np.load(os.path.join(HERE, "golden", "ops.npz")))


def eq(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    assert a.shape == b.shape, (a.shape, b.shape)
    assert np.array_equal(a.astype(I64), b.astype(I64))


def test_scaled_round_div(D):
    eq(dy.scaled_round_div(D["srd_num"], D["srd_den"], D["srd_e"]), D["srd_out"])


def test_fit_dyadic_ratio(D):
    m, e = dy.fit_dyadic_ratio(D["fit_num"], D["fit_den"])
    eq(m, D["fit_m"]); eq(e, D["fit_e"])
    m, e = dy.fit_dyadic_ratio(D["fit_num"], 127)
    eq(m, D["fit127_m"]); eq(e, D["fit127_e"])


def test_fit_exact_powers():
    # tests/test_dyadic.py:29-33: powers of two are represented exactly
    num = np.array([1, 2, 1 << 15, 1 << 30], dtype=I64)
    m, e = dy.fit_dyadic_ratio(num, 1)
    assert [int(mm) * 2.0 ** -int(ee) for mm, ee in zip(m, e)] == [float(v) for v in num]


def test_norm_scale(D):
    m2, k2 = dy.norm_scale(D["ns_m"], D["ns_k"])
    eq(m2, D["ns_m2"]); eq(k2, D["ns_k2"])


def test_quant_i8_pertoken(D):
    for p in ("q", "q64"):
        x8, mo, ko = dy.quant_i8_pertoken(D[p + "_x"], D[p + "_m"], D[p + "_k"])
        assert x8.dtype == np.int8
        eq(x8, D[p + "_x8"]); eq(mo, D[p + "_mo"]); eq(ko, D[p + "_ko"])


def test_quant_max_maps_to_127_and_zero_row():
    # tests/test_dyadic.py:68-78
    x8, _, _ = dy.quant_i8_pertoken(np.array([[3, -1000, 500]]), np.ones((1, 1), I64),
                                    np.zeros((1, 1), I64))
    assert np.abs(x8.astype(I64)).max() == 127
    x8, _, _ = dy.quant_i8_pertoken(np.zeros((2, 8), np.int32), np.ones((2, 1), I64),
                                    np.zeros((2, 1), I64))
    assert (x8 == 0).all()


def test_requant_i32_common(D):
    for tb in (12, 14, 16, 20):
        y, m, k = dy.requant_i32_common(D["rq_P"], D["rq_rm"], D["rq_rk"], D["rq_cm"], 24, tb)
        assert y.dtype == np.int32
        eq(y, D[f"rq{tb}_y"]); eq(m, D[f"rq{tb}_m"]); eq(k, D[f"rq{tb}_k"])


def test_requant_i8_rowcol(D):
    y8, m, k = dy.requant_i8_rowcol(D["rq_P"], D["rq_rm"], D["rq_rk"], D["rq_cm"], 24)
    eq(y8, D["rc_y8"]); eq(m, D["rc_m"]); eq(k, D["rc_k"])
    y8, m, k = dy.requant_i8_rowcol(D["rc64_P"], D["rc64_rm"], D["rc64_rk"], D["rc64_cm"], 30)
    eq(y8, D["rc64_y8"]); eq(m, D["rc64_m"]); eq(k, D["rc64_k"])


def test_requant_i8_static(D):
    y8 = dy.requant_i8_static(D["rs_P"], D["rs_rm"], D["rs_rk"], D["rs_cm"], 24,
                              D["rs_sm"], D["rs_sk"])
    eq(y8, D["rs_y8"])
    y8 = dy.requant_i8_static(D["rsk_x"], 1, 31, 1, 0, D["rsk_m"], D["rsk_k"])
    eq(y8, D["rsk_y8"])
    y8 = dy.requant_i8_static(D["rq_P"], 1, 0, D["rq_cm"], 20, 1, 0)
    eq(y8, D["rs0_y8"])


def test_residual(D):
    h, k = dy.residual_renorm(D["rr_h64"], D["rr_k"])
    assert h.dtype == np.int32
    eq(h, D["rr_h"]); eq(k, D["rr_k2"])
    h, k = dy.residual_from_delta(D["rf_d"], D["rf_dm"], D["rf_dk"])
    eq(h, D["rf_h"]); eq(k, D["rf_k"])
    h3, k3 = dy.residual_add(h, k, D["ra_d"], D["ra_dm"], D["ra_dk"])
    eq(h3, D["ra_h"]); eq(k3, D["ra_k"])


def test_di_exp(O):
    res, tpos = ops.di_exp(O["exp_x"], O["exp_m"], O["exp_k"])
    eq(res, O["exp_res"]); eq(tpos, O["exp_tpos"])
    eq(ops.di_exp_tpos(O["exp_m"], O["exp_k"]), O["exp_tpos"])


def test_di_exp_special_cases():
    # tests/test_ops.py:123-134: e^0 == tpos exactly; deep tail -> 0
    m = np.array([[1 << 15]], I64)
    k = np.array([[15]], I64)
    res, tpos = ops.di_exp(np.zeros((1, 1), I64), m, k)
    assert res.item() == tpos.item()
    res, _ = ops.di_exp(np.array([[-50 << 15, -100 << 15]], I64), m, k)
    assert (res == 0).all()


def test_di_softmax(O):
    args = (O["sm_x"], O["sm_m"], O["sm_k"], O["sm_valid"])
    eq(ops.di_softmax(*args), O["sm_p15"])
    eq(ops.di_softmax(*args, p_out_bits=8), O["sm_p8"])
    eq(ops.di_softmax(*args, clip_c=15), O["sm_pc15"])


def test_di_softmax_masking_invariants(O):
    # tests/test_ops.py:164-181
    x, m, k = O["sm_x"][0, 0], O["sm_m"][0, 0], O["sm_k"][0, 0]
    valid = np.ones(x.shape, bool)
    valid[:, 100:] = False
    p1 = ops.di_softmax(x, m, k, valid)
    assert (p1[:, 100:] == 0).all()
    x2 = x.copy()
    x2[:, 100:] = 999999
    assert np.array_equal(p1, ops.di_softmax(x2, m, k, valid))
    assert (ops.di_softmax(x, m, k, np.zeros(x.shape, bool)) == 0).all()


def test_di_rmsnorm(O):
    for n in (1024, 128, 3072):
        eq(ops.di_rmsnorm(O[f"rms{n}_x"]), O[f"rms{n}_y"])
    eq(ops.di_rmsnorm(O["rms64_x"]), O["rms64_y"])
    y, k = ops.di_rmsnorm_gamma(O["rmsg_x"], O["rmsg_gm"], 13)
    eq(y, O["rmsg_y"]); assert k == int(O["rmsg_k"])


def test_di_rmsnorm_invariants():
    # tests/test_ops.py:202-212
    rng = np.random.default_rng(9)
    x = rng.integers(-(1 << 20), 1 << 20, (4, 128)).astype(np.int32)
    assert np.array_equal(ops.di_rmsnorm(x), ops.di_rmsnorm(x << 4))
    assert (ops.di_rmsnorm(np.zeros((2, 128), np.int32)) == 0).all()


def test_di_swiglu(O):
    y, m, k = ops.di_swiglu(O["sw_g"], O["sw_gm"], O["sw_gk"], O["sw_u"], O["sw_um"], O["sw_uk"])
    eq(y, O["sw_y"]); eq(m, O["sw_ym"]); eq(k, O["sw_yk"])


def test_rope(O):
    import hashlib

    from idempotent_llm_amd.artifact import rope_tables
    cos_t, sin_t = ops.build_rope_tables(128, 4096, 1e6)
    assert hashlib.sha256(cos_t.tobytes()).digest() == O["rope_cos_digest"].tobytes()
    assert hashlib.sha256(sin_t.tobytes()).digest() == O["rope_sin_digest"].tobytes()
    c2, s2 = rope_tables(128, 4096, 1e6)
    assert np.array_equal(c2, cos_t) and np.array_equal(s2, sin_t)
    eq(ops.apply_int_rope(O["rope_x"], cos_t, sin_t, O["rope_pos"]), O["rope_y"])
