"""GPU parity of every op-level HIP kernel (through the C-ABI) against the
golden vectors written from the reference CPU path, the oracle and closed
forms. Zero tolerance: every comparison is exact equality."""

import math
import os

import numpy as np
import pytest
import torch

from oracle import dyadic as ody
from oracle import gemm as ogemm
from oracle import intmath as oim
from oracle import ops as oops

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
I64 = np.int64


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from idempotent_llm_amd import _lib
    _lib.load()   # fails loudly if the HIP library is missing


@pytest.fixture(scope="module")
def D():
    return dict(np.load(os.path.join(HERE, "golden", "dyadic.npz")))


@pytest.fixture(scope="module")
def O():
    return dict(np.load(os.path.join(HERE, "golden", "ops.npz")))


def g(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def eq(got, want):
    got = got.cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.array_equal(got.astype(I64), want.astype(I64))


def test_isqrt_ilog2_vs_closed_forms():
    from idempotent_llm_amd import dyadic as dd
    rnd = np.random.default_rng(0)
    v = np.concatenate([rnd.integers(0, 1 << 62, 200000, dtype=I64),
                        np.arange(0, 70000, dtype=I64),
                        np.array([0, 1, 2, 3, 4, (1 << 31) - 1, 1 << 31, (1 << 52) + 7,
                                  (1 << 62) - 1], I64)])
    got = dd.isqrt(g(v)).cpu().numpy()
    assert got.tolist() == [math.isqrt(int(x)) for x in v]
    w = np.concatenate([rnd.integers(1, 1 << 62, 200000, dtype=I64),
                        np.arange(1, 1 << 16, dtype=I64),
                        np.array([1, 2, 3, (1 << 62) + 123, (1 << 63) - 1], I64)])
    got = dd.ilog2_floor(g(w)).cpu().numpy()
    assert got.tolist() == [int(x).bit_length() - 1 for x in w]
    x = rnd.integers(0, 1 << 50, (17, 33, 5), dtype=I64)
    eq(dd.isqrt(g(x)), oim.isqrt(x))


def test_device_fast_paths_vs_closed_forms(D):
    """The forms the fused kernels run: the wave-parallel isqrt (op 6) is
    floor(sqrt) (math.isqrt) and fit_dyadic_ratio(., 127) by the constant-127
    path (op 5) equals the reference's golden vectors and the generic form."""
    from idempotent_llm_amd._lib import call
    rnd = np.random.default_rng(5)
    v = np.concatenate([rnd.integers(0, 1 << 62, 100000, dtype=I64),
                        (I64(1) << rnd.integers(0, 62, 5000).astype(I64)) - 1,
                        np.arange(-3, 70000, dtype=I64),
                        np.array([(1 << 63) - 1, (1 << 62) - 1, 1 << 62, 3037000499 ** 2,
                                  3037000499 ** 2 - 1, -(1 << 63)], I64)])
    x = g(v)
    out = torch.empty_like(x)
    call("detllm_op_scalar", 6, x, None, None, x.numel(), out, None)
    assert out.cpu().numpy().tolist() == [math.isqrt(int(t)) if t > 0 else 0 for t in v]
    num = np.concatenate([D["fit_num"], rnd.integers(1, 1 << 62, 50000, dtype=I64)])
    xn = g(num)
    m5, e5 = torch.empty_like(xn), torch.empty_like(xn)
    call("detllm_op_scalar", 5, xn, None, None, xn.numel(), m5, e5)
    den = g(np.full_like(num, 127))
    m3, e3 = torch.empty_like(xn), torch.empty_like(xn)
    call("detllm_op_scalar", 3, xn, den, None, xn.numel(), m3, e3)
    eq(m5, m3.cpu().numpy()); eq(e5, e3.cpu().numpy())
    n0 = D["fit_num"].size
    eq(m5[:n0], D["fit127_m"]); eq(e5[:n0], D["fit127_e"])


def test_sigmoid_division_single_precision_on_device():
    """The fused SwiGLU's sigmoid division in its device form (v_rcp_f32
    reciprocal, one remainder step) == round_half_away_div(num << 7, den)
    (ops/di_swiglu.py:52-55) for 0 <= num <= den < 2^24: every num for
    den < 300, the top of the range and random pairs of every bit length."""
    from idempotent_llm_amd._lib import call
    import random
    rnd = random.Random(11)
    num, den = [], []
    for d in list(range(1, 300)) + [(1 << 24) - 1, (1 << 24) - 2, (1 << 23) + 1, 1 << 23]:
        for n in (range(0, d + 1) if d < 300 else [0, 1, d // 2, d // 2 + 1, d - 1, d]):
            num.append(n)
            den.append(d)
    for _ in range(1000000):
        d = rnd.randrange(1, 1 << rnd.randrange(1, 25))
        num.append(rnd.choice([0, d, d - 1, d // 2, rnd.randrange(0, d + 1)]))
        den.append(d)
    a, b = np.array(num, I64), np.array(den, I64)
    out = torch.empty(a.size, dtype=torch.int64, device="cuda")
    call("detllm_op_scalar", 7, g(a), g(b), None, a.size, out, None)
    eq(out, (a * 128 + b // 2) // b)


def test_dyadic_scalars(D):
    from idempotent_llm_amd import dyadic as dd
    eq(dd.scaled_round_div(g(D["srd_num"]), g(D["srd_den"]), g(D["srd_e"])), D["srd_out"])
    m, e = dd.fit_dyadic_ratio(g(D["fit_num"]), g(D["fit_den"]))
    eq(m, D["fit_m"]); eq(e, D["fit_e"])
    m, e = dd.fit_dyadic_ratio(g(D["fit_num"]), 127)
    eq(m, D["fit127_m"]); eq(e, D["fit127_e"])
    m2, k2 = dd.norm_scale(g(D["ns_m"]), g(D["ns_k"]))
    eq(m2, D["ns_m2"]); eq(k2, D["ns_k2"])


def test_quant_i8_pertoken(D):
    from idempotent_llm_amd import dyadic as dd
    for p in ("q", "q64"):
        x8, mo, ko = dd.quant_i8_pertoken(g(D[p + "_x"]), g(D[p + "_m"]), g(D[p + "_k"]))
        assert x8.dtype == torch.int8
        eq(x8, D[p + "_x8"]); eq(mo, D[p + "_mo"]); eq(ko, D[p + "_ko"])


def test_requant_i32_common(D):
    from idempotent_llm_amd import dyadic as dd
    for tb in (12, 14, 16, 20):
        y, m, k = dd.requant_i32_common(g(D["rq_P"]), g(D["rq_rm"]), g(D["rq_rk"]),
                                        g(D["rq_cm"]), 24, target_bits=tb)
        assert y.dtype == torch.int32
        eq(y, D[f"rq{tb}_y"]); eq(m, D[f"rq{tb}_m"]); eq(k, D[f"rq{tb}_k"])


def test_requant_i32_common_grouped_cols():
    # per-(head, channel) column scales as in _qk_head_pipeline (model.py:207-211)
    from idempotent_llm_amd import dyadic as dd
    rnd = np.random.default_rng(3)
    P = rnd.integers(-(1 << 24), 1 << 24, (2, 5, 4, 128)).astype(np.int32)
    rm = rnd.integers(1 << 15, 1 << 16, (2, 5, 1, 1), dtype=I64)
    rk = rnd.integers(10, 40, (2, 5, 1, 1), dtype=I64)
    cm = rnd.integers(1 << 14, 1 << 16, (4, 128), dtype=I64)
    y, m, k = dd.requant_i32_common(g(P), g(rm), g(rk), g(cm), 24, target_bits=16)
    wy, wm, wk = ody.requant_i32_common(P, rm, rk, cm, 24, 16)
    eq(y, wy); eq(k, wk)


def test_requant_i8_rowcol(D):
    from idempotent_llm_amd import dyadic as dd
    y8, m, k = dd.requant_i8_rowcol(g(D["rq_P"]), g(D["rq_rm"]), g(D["rq_rk"]), g(D["rq_cm"]), 24)
    eq(y8, D["rc_y8"]); eq(m, D["rc_m"]); eq(k, D["rc_k"])
    y8, m, k = dd.requant_i8_rowcol(g(D["rc64_P"]), g(D["rc64_rm"]), g(D["rc64_rk"]),
                                    g(D["rc64_cm"]), 30)
    eq(y8, D["rc64_y8"]); eq(m, D["rc64_m"]); eq(k, D["rc64_k"])


def test_requant_i8_static(D):
    from idempotent_llm_amd import dyadic as dd
    eq(dd.requant_i8_static(g(D["rs_P"]), g(D["rs_rm"]), g(D["rs_rk"]), g(D["rs_cm"]), 24,
                            g(D["rs_sm"]), g(D["rs_sk"])), D["rs_y8"])
    eq(dd.requant_i8_static(g(D["rsk_x"]), 1, 31, 1, 0, g(D["rsk_m"]), g(D["rsk_k"])),
       D["rsk_y8"])
    eq(dd.requant_i8_static(g(D["rq_P"]), 1, 0, g(D["rq_cm"]), 20, 1, 0), D["rs0_y8"])


def test_residual(D):
    from idempotent_llm_amd import dyadic as dd
    h, k = dd.residual_renorm(g(D["rr_h64"]), g(D["rr_k"]))
    eq(h, D["rr_h"]); eq(k, D["rr_k2"])
    h, k = dd.residual_from_delta(g(D["rf_d"]), g(D["rf_dm"]), g(D["rf_dk"]))
    eq(h, D["rf_h"]); eq(k, D["rf_k"])
    h3, k3 = dd.residual_add(h, k, g(D["ra_d"]), g(D["ra_dm"]), g(D["ra_dk"]))
    eq(h3, D["ra_h"]); eq(k3, D["ra_k"])


def test_di_exp(O):
    from idempotent_llm_amd import ops
    res, tpos = ops.di_exp(g(O["exp_x"]), g(O["exp_m"]), g(O["exp_k"]))
    eq(res, O["exp_res"]); eq(tpos, O["exp_tpos"])


def test_di_softmax(O):
    from idempotent_llm_amd import ops
    args = (g(O["sm_x"]), g(O["sm_m"]), g(O["sm_k"]), g(O["sm_valid"]))
    eq(ops.di_softmax(*args), O["sm_p15"])
    eq(ops.di_softmax(*args, p_out_bits=8), O["sm_p8"])
    eq(ops.di_softmax(*args, clip_c=15), O["sm_pc15"])
    z = ops.di_softmax(args[0], args[1], args[2], torch.zeros_like(args[3]))
    assert int(z.abs().max()) == 0


def test_di_rmsnorm(O):
    from idempotent_llm_amd import ops
    for n in (1024, 128, 3072):
        eq(ops.di_rmsnorm(g(O[f"rms{n}_x"])), O[f"rms{n}_y"])
    eq(ops.di_rmsnorm(g(O["rms64_x"])), O["rms64_y"])
    y, k = ops.di_rmsnorm_gamma(g(O["rmsg_x"]), g(O["rmsg_gm"]), 13)
    eq(y, O["rmsg_y"]); assert k == int(O["rmsg_k"])


def test_di_swiglu(O):
    from idempotent_llm_amd import ops
    y, m, k = ops.di_swiglu(g(O["sw_g"]), g(O["sw_gm"]), g(O["sw_gk"]), g(O["sw_u"]),
                            g(O["sw_um"]), g(O["sw_uk"]))
    eq(y, O["sw_y"]); eq(m, O["sw_ym"]); eq(k, O["sw_yk"])


def test_rope(O):
    from idempotent_llm_amd import ops
    cos_t, sin_t = oops.build_rope_tables(128, 4096, 1e6)
    eq(ops.apply_int_rope(g(O["rope_x"]), g(cos_t), g(sin_t), g(O["rope_pos"])), O["rope_y"])


@pytest.mark.parametrize("M,K,N", [(7, 33, 5), (1, 1024, 4096), (8, 3072, 1024), (64, 1024, 3072),
                                   (65, 1024, 3072), (200, 128, 300), (512, 2048, 1024),
                                   (2048, 1024, 4096), (2048, 3072, 1024), (2048, 1024, 6144),
                                   (1000, 2048, 1000), (129, 64, 130), (300, 192, 64),
                                   (3000, 512, 9000), (2100, 1024, 4096), (1900, 256, 6144),
                                   (9000, 256, 1100),
                                   # LM-head streaming path (M <= 16, N >= 32768) and its edges
                                   (1, 1024, 151936), (8, 1024, 40000), (16, 1040, 32768),
                                   (13, 4096, 33000), (5, 2048, 50001), (17, 1024, 40000),
                                   (16, 1024, 32767)])
def test_int_gemm_exact(M, K, N):
    from idempotent_llm_amd.backends import int_gemm
    rnd = np.random.default_rng(M * 7 + K + N)
    a = rnd.integers(-128, 128, (M, K)).astype(np.int8)
    b = rnd.integers(-128, 128, (K, N)).astype(np.int8)
    got = int_gemm(g(a), g(b), "rocm")
    assert got.dtype == torch.int32
    eq(got, ogemm.int_gemm(a, b))   # exact: float64 BLAS on int8 operands, |sum| < 2^53


def test_int_gemm_extremes_and_batched():
    from idempotent_llm_amd.backends import int_gemm, int_gemm_u8i8, int_gemm_u16i8
    a = np.full((70, 3072), -128, np.int8)
    b = np.full((3072, 40), -128, np.int8)
    eq(int_gemm(g(a), g(b), "rocm"), np.full((70, 40), 3072 * 128 * 128))
    rnd = np.random.default_rng(9)
    a = rnd.integers(-128, 128, (3, 4, 37, 128)).astype(np.int8)
    b = rnd.integers(-128, 128, (3, 4, 128, 45)).astype(np.int8)
    eq(int_gemm(g(a), g(b), "rocm"), a.astype(I64) @ b.astype(I64))
    # batched through the pipelined prefill kernel (M > 64, K % 64 == 0)
    a = rnd.integers(-128, 128, (2, 3, 200, 256)).astype(np.int8)
    b = rnd.integers(-128, 128, (2, 3, 256, 96)).astype(np.int8)
    eq(int_gemm(g(a), g(b), "rocm"), a.astype(I64) @ b.astype(I64))
    a = np.full((300, 1024), -128, np.int8)
    b = np.full((1024, 200), -128, np.int8)
    eq(int_gemm(g(a), g(b), "rocm"), np.full((300, 200), 1024 * 128 * 128))
    p = rnd.integers(0, 129, (9, 21)).astype(np.int32)
    v = rnd.integers(-128, 128, (21, 6)).astype(np.int8)
    got = int_gemm_u8i8(g(p), g(v), "rocm")
    assert got.dtype == torch.int64   # the reference's int32 colsum promotes
    eq(got, p.astype(I64) @ v.astype(I64))
    p = rnd.integers(0, (1 << 14) + 1, (9, 300)).astype(np.int32)
    v = rnd.integers(-128, 128, (300, 6)).astype(np.int8)
    got = int_gemm_u16i8(g(p), g(v), "rocm")
    assert got.dtype == torch.int64
    eq(got, ogemm.int_gemm_u16i8(p, v))


def test_config0_gemm_requant():
    """Config c0: [64,1024] x [1024,3072] then requant_i8_static(P,1,0,m,20,1,0)
    and the rowcol variant, bit-identical to the CPU path."""
    from idempotent_llm_amd import artifact as art
    from idempotent_llm_amd import dyadic as dd
    from idempotent_llm_amd.backends import int_gemm
    A = art.rand_i8(0, "c0.A", (64, 1024))
    W = art.rand_i8(0, "c0.W", (1024, 3072))
    m = art.uniform_int(0, "c0.m", (3072,), 1 << 14, 1 << 15)
    P = int_gemm(g(A), g(W), "rocm")
    Pw = ogemm.int_gemm(A, W)
    eq(P, Pw)
    eq(dd.requant_i8_static(P, 1, 0, g(m), 20, 1, 0), ody.requant_i8_static(Pw, 1, 0, m, 20, 1, 0))
    y8, mo, ko = dd.requant_i8_rowcol(P, 1, 0, g(m), 20)
    wy, wm, wk = ody.requant_i8_rowcol(Pw, np.ones((64, 1), I64), np.zeros((64, 1), I64), m, 20)
    eq(y8, wy); eq(mo, wm); eq(ko, wk)
    # the bench's c0 path: skinny GEMM partials, then the fused static epilogue
    from idempotent_llm_amd._lib import call, gemv_plan
    from idempotent_llm_amd.backends import gemm_nt
    ks = gemv_plan(64, 3072, 1024)
    Pp = gemm_nt(g(A), g(W.T.copy()), ksplit=ks)
    y8s = torch.empty(64, 3072, dtype=torch.int8, device="cuda")
    call("detllm_requant_static_cols", Pp, ks, 64 * 3072, 64, 3072, None, None, g(m), 20, 1, 0,
         y8s)
    eq(y8s, ody.requant_i8_static(Pw, 1, 0, m, 20, 1, 0))


def test_igemv_requant_static_c0_and_general():
    """detllm_igemv_requant_static (int_gemm + requant_i8_static in one
    launch, the product kept in registers): config c0 against the oracle
    (backends.py:88-135, dyadic.py:142-163), then ragged shapes (M = 1, 17,
    64; N not a multiple of 16; K not a multiple of 256) with per-row scales,
    up- and down-shifts, numerators past the fp64 estimate's bound (the
    exact integer path) and divisors that wrap negative (rows with row_k
    22: torch's floor division by the wrapped value), each equal to the
    oracle."""
    from idempotent_llm_amd import artifact as art
    from idempotent_llm_amd._lib import call
    A = art.rand_i8(0, "c0.A", (64, 1024))
    W = art.rand_i8(0, "c0.W", (1024, 3072))
    m = art.uniform_int(0, "c0.m", (3072,), 1 << 14, 1 << 15)
    y8 = torch.empty(64, 3072, dtype=torch.int8, device="cuda")
    call("detllm_igemv_requant_static", g(A), g(W.T.copy()), 64, 3072, 1024, None, None, g(m),
         20, 1, 0, y8)
    eq(y8, ody.requant_i8_static(ogemm.int_gemm(A, W), 1, 0, m, 20, 1, 0))
    rnd = np.random.default_rng(44)
    for M, N, K in ((1, 301, 272), (17, 4100, 1024), (64, 48, 1040)):
        A = rnd.integers(-128, 128, (M, K)).astype(np.int8)
        W = rnd.integers(-128, 128, (K, N)).astype(np.int8)
        Pw = ogemm.int_gemm(A, W)
        row_m = rnd.integers(1, 1 << 16, (M, 1)).astype(I64)
        row_k = rnd.integers(0, 30, (M, 1)).astype(I64)
        col_m = rnd.integers(1 << 14, 1 << 16, (N,)).astype(I64)
        col_m[::7] = rnd.integers(1 << 30, 1 << 40, col_m[::7].shape)   # |n| past 2^49
        for col_k, s_m, s_k in ((20, 1, 0), (5, 40000, 60), (24, (1 << 20) + 7, 3)):
            want = ody.requant_i8_static(Pw, row_m, row_k, col_m, col_k, s_m, s_k)
            y8 = torch.empty(M, N, dtype=torch.int8, device="cuda")
            call("detllm_igemv_requant_static", g(A), g(W.T.copy()), M, N, K, g(row_m[:, 0]),
                 g(row_k[:, 0]), g(col_m), col_k, s_m, s_k, y8)
            eq(y8, want)


@pytest.mark.parametrize("seed", [0, 1])
def test_requant_static_cols_general(seed):
    """detllm_requant_static_cols with per-row scales, up- and down-shifts
    and numerators past the estimate's bound (the exact integer path),
    against dyadic.py:142-163 restated in the oracle."""
    from idempotent_llm_amd._lib import call
    rnd = np.random.default_rng(40 + seed)
    R, C, ks = 7, 301, 3
    parts = rnd.integers(-(1 << 29), 1 << 29, (ks, R, C)).astype(np.int32)
    Pw = parts.astype(I64).sum(axis=0)
    Pw = ((Pw + (1 << 31)) % (1 << 32) - (1 << 31)).astype(np.int32)   # int32 wrap of the sum
    row_m = rnd.integers(1, 1 << 16, (R, 1)).astype(I64)
    row_k = rnd.integers(0, 30, (R, 1)).astype(I64)
    # rows whose divisor s_m << shift wraps negative at the third target
    # ((2^20 + 7) << 43 and << 61 pass 2^63): torch's floor division by the
    # wrapped value, as the reference's tensor rhad computes it
    row_k[0, 0], row_k[1, 0] = 22, 40
    col_m = rnd.integers(1 << 14, 1 << 16, (C,)).astype(I64)
    for col_k, s_m, s_k in ((20, 1, 0), (5, 40000, 60), (24, (1 << 20) + 7, 3)):
        want = ody.requant_i8_static(Pw, row_m, row_k, col_m, col_k, s_m, s_k)
        y8 = torch.empty(R, C, dtype=torch.int8, device="cuda")
        call("detllm_requant_static_cols", g(parts), ks, R * C, R, C, g(row_m[:, 0]),
             g(row_k[:, 0]), g(col_m), col_k, s_m, s_k, y8)
        eq(y8, want)


def test_di_matmul_composition():
    """ops/di_matmul.py:34-40 (quant_i8_pertoken -> int_gemm ->
    requant_i8_rowcol) on the device equals the oracle's composition."""
    from idempotent_llm_amd import ops as dops
    rnd = np.random.default_rng(21)
    x = rnd.integers(-(1 << 30), 1 << 30, (37, 256)).astype(I64)
    xm = rnd.integers(1 << 15, 1 << 16, (37, 1)).astype(I64)
    xk = rnd.integers(20, 40, (37, 1)).astype(I64)
    w = rnd.integers(-127, 128, (256, 96)).astype(np.int8)
    wm = rnd.integers(1 << 14, 1 << 16, (96,)).astype(I64)
    y8, m, k = dops.di_matmul(g(x), g(xm), g(xk), g(w), g(wm), 24)
    oy, om, ok = oops.di_matmul(x, xm, xk, w, wm, 24)
    eq(y8, oy); eq(m, om); eq(k, ok)


def _normq_oracle(P, row_m, row_k, col_m, col_k, h, k_res, sm_m, sm_k):
    """model.py:410-415 (+ :187-198) on the oracle: requant_i32_common(20),
    residual_add, then _norm_quant with optional smoothing."""
    d, dm, dk = ody.requant_i32_common(P, row_m[:, None], row_k[:, None], col_m, col_k,
                                       target_bits=20)
    h2, k2 = ody.residual_add(h, k_res[:, None], d, dm, dk)
    y = oops.di_rmsnorm(h2)
    kq = np.full((P.shape[0], 1), 20, I64)
    if sm_m is not None:
        y = y.astype(I64) * sm_m.astype(I64)
        kq = kq + sm_k
    x8, xm, xk = ody.quant_i8_pertoken(y, np.ones_like(kq), kq)
    return h2, k2[:, 0], x8, xm[:, 0], xk[:, 0]


@pytest.mark.parametrize("C", [1024, 256, 3072])
@pytest.mark.parametrize("smooth", [False, True])
def test_residual_normq_renorm_branches(C, smooth):
    """The fused residual + RMSNorm + quant kernel against the oracle on rows
    chosen to take every renormalisation branch: the sum crosses 2^30 (down
    shift, the RMSNorm maximum is reduced again), small rows (up shift, the
    RMSNorm maximum follows from the renorm), rows left in [2^26, 2^30), a
    zero row, and a row of one non-zero element."""
    from idempotent_llm_amd._lib import call
    print(f"[residual_normq branches C={C} smooth={smooth}]", flush=True)
    rng = np.random.default_rng(C + smooth)
    R = 8
    scale = [2 ** 29 - 3, 2 ** 20, 2 ** 28, 0, 0, 2 ** 27, 2 ** 12, 2 ** 29]
    h = np.stack([rng.integers(-s, s + 1, C) if s else np.zeros(C, I64) for s in scale])
    h[4, C // 3] = 5
    P = rng.integers(-(1 << 20), 1 << 20, (1, R, C)).astype(np.int32)
    P[0, 3] = 0
    P[0, 4] = 0
    row_m = rng.integers(1 << 15, 1 << 16, R).astype(I64)
    row_k = np.array([20, 24, 26, 20, 20, 30, 40, 19], I64)
    k_res = np.array([24, 24, 24, 24, 24, 24, 24, 24], I64)
    col_m = rng.integers(1 << 15, 1 << 16, C).astype(I64)
    sm_m = rng.integers(1 << 15, 1 << 16, C).astype(I64) if smooth else None
    want = _normq_oracle(P[0], row_m, row_k, col_m, 20, h.astype(np.int32), k_res, sm_m, 15)
    hg = g(h.astype(np.int32))
    kg = g(k_res.copy())
    x8 = torch.empty(R, C, dtype=torch.int8, device="cuda")
    xm = torch.empty(R, dtype=torch.int64, device="cuda")
    xk = torch.empty(R, dtype=torch.int64, device="cuda")
    call("detllm_residual_normq", g(P), 1, 0, R, C, g(row_m), g(row_k), g(col_m), 20, 20, hg,
         kg, g(sm_m) if smooth else None, 15, x8, xm, xk, None, 0, 0, 0, 0)
    for got, w in zip((hg, kg, x8, xm, xk), want):
        eq(got, w)
    # the rows do take the branches named above
    d, dm, dk = ody.requant_i32_common(P[0], row_m[:, None], row_k[:, None], col_m, 20, 20)
    rel = dk[:, 0] - k_res
    dd = d.astype(I64) * dm
    al = oim.shl(oim.rshift_round_t(dd, np.broadcast_to(np.maximum(rel, 0)[:, None], dd.shape)),
                 np.broadcast_to(np.maximum(-rel, 0)[:, None], dd.shape))
    top = np.abs(h.astype(I64) + al).max(axis=1)
    assert (top >= 2 ** 30).any() and ((top > 0) & (top < 2 ** 26)).any()
    assert ((top >= 2 ** 26) & (top < 2 ** 30)).any() and (top == 0).any()


@pytest.mark.parametrize("big_col", [False, True])
def test_residual_normq_every_path(big_col):
    """The GEMM residual add (requant_i32_common(20) + residual_add + renorm)
    runs on exact doubles for rows whose operands keep every product below
    2^52 and on int64 routines otherwise. Rows here take each side: an
    alignment down-shift of 58 (the delta rounds to 0 both ways) and of 70
    (past 63 torch's shift clamps differ from a rounding: int64 side), an
    up-shift of 25 (doubles), of 40 (delta above 2^51: int64) and of 60 (the
    int64 shift wraps), a row mantissa of 2^33 and of -2^31 (int64 side).
    With big_col one column mantissa is 2^21 (every row on the int64 side);
    without, one is -(2^21 - 1) (the doubles' limit). Both the row kernel and
    the decode GEMV with the row kernel fused in are checked against the
    oracle."""
    from idempotent_llm_amd._lib import call
    print(f"[residual_normq every path big_col={big_col}]", flush=True)
    rng = np.random.default_rng(11 + big_col)
    R, C, N = 8, 1024, 1024
    col_m = rng.integers(1 << 15, 1 << 16, C).astype(I64)
    col_m[C // 2] = (1 << 21) if big_col else -((1 << 21) - 1)
    k_res = np.full(R, 24, I64)
    # (row_m, P magnitude, target rel = dk - k_res; None: row_k 20)
    rows = [(40000, 1 << 20, None), (40000, 1 << 20, 58), (40000, 1 << 20, 70),
            (3, 4, -25), (3, 4, -40), (3, 4, -60), (1 << 33, 1 << 20, None),
            (-(1 << 31), 1 << 20, None)]
    P = np.stack([rng.integers(-p, p + 1, C) for _, p, _ in rows]).astype(np.int32)
    row_m = np.array([m for m, _, _ in rows], I64)
    _, _, dk0 = ody.requant_i32_common(P, row_m[:, None], np.zeros((R, 1), I64), col_m, 20,
                                       target_bits=20)
    row_k = np.array([20 if rel is None else k_res[i] + rel - dk0[i, 0]
                      for i, (_, _, rel) in enumerate(rows)], I64)
    h = rng.integers(-(1 << 26), 1 << 26, (R, C)).astype(np.int32)
    sm_m = rng.integers(1 << 15, 1 << 16, C).astype(I64)
    want = _normq_oracle(P, row_m, row_k, col_m, 20, h, k_res, sm_m, 15)
    # the rows take the shifts named above
    _, _, dk = ody.requant_i32_common(P, row_m[:, None], row_k[:, None], col_m, 20, 20)
    rel = dk[:, 0] - k_res
    assert list(rel[1:6]) == [58, 70, -25, -40, -60]
    hg, kg = g(h), g(k_res.copy())
    x8 = torch.empty(R, C, dtype=torch.int8, device="cuda")
    xm = torch.empty(R, dtype=torch.int64, device="cuda")
    xk = torch.empty(R, dtype=torch.int64, device="cuda")
    call("detllm_residual_normq", g(P), 1, 0, R, C, g(row_m), g(row_k), g(col_m), 20, 20, hg,
         kg, g(sm_m), 15, x8, xm, xk, None, 0, 0, 0, 0)
    for got, w in zip((hg, kg, x8, xm, xk), want):
        eq(got, w)
    # the decode GEMV with this row kernel fused in (partials split in two)
    w8 = rng.integers(-128, 128, (N, C)).astype(np.int8)
    P2 = np.stack([P, np.zeros_like(P)]).astype(np.int32)
    P2[1] = rng.integers(-50, 51, (R, C))
    P2[0] -= P2[1]
    ks = 1
    h_out = torch.full((R, C), -1, dtype=torch.int32, device="cuda")
    k_out = torch.full((R,), -1, dtype=torch.int64, device="cuda")
    fm = torch.full((R,), -1, dtype=torch.int64, device="cuda")
    fk = torch.full((R,), -1, dtype=torch.int64, device="cuda")
    Cg = torch.full((ks, R, N), -7, dtype=torch.int32, device="cuda")
    call("detllm_igemv_resnormq", g(w8), Cg, R, N, C, ks, R * N, g(P2), 2, R * C, g(row_m),
         g(row_k), g(col_m), 20, 20, g(h), g(k_res), h_out, k_out, g(sm_m), 15, fm, fk,
         None, 0, None, 0)
    eq(h_out, want[0]); eq(k_out, want[1]); eq(fm, want[3]); eq(fk, want[4])
    eq(Cg.sum(0), ogemm.int_gemm(want[2], w8.T))


def test_igemv_prefetch_variant_same_product():
    """detllm_igemv_nt_pf (skinny GEMM + prefetch hint) gives the product of
    detllm_igemv_nt, with 0-4 ranges of any multiple-of-4 size; bad ranges are
    argument errors."""
    from idempotent_llm_amd._lib import call, gemv_plan
    print("[igemv prefetch]", flush=True)
    rng = np.random.default_rng(3)
    M, N, K = 8, 1024, 3072
    a = g(rng.integers(-128, 128, (M, K)).astype(np.int8))
    w = g(rng.integers(-128, 128, (N, K)).astype(np.int8))
    ks = gemv_plan(M, N, K)
    ref = torch.empty(ks, M, N, dtype=torch.int32, device="cuda")
    call("detllm_igemv_nt", a, w, ref, M, N, K, ks, M * N)
    pfs = [g(rng.integers(0, 9, n).astype(np.int64)) for n in (1, 17, 3072, 40000)]
    for nr in range(5):
        out = torch.full((ks, M, N), -1, dtype=torch.int32, device="cuda")
        args = []
        for t in pfs[:nr]:
            args += [t, t.numel() * 8]
        args += [None, 0] * (4 - nr)
        call("detllm_igemv_nt_pf", a, w, out, M, N, K, ks, M * N, *args)
        assert torch.equal(out, ref)
    want = ogemm.int_gemm(a.cpu().numpy(), w.cpu().numpy().T)
    eq(ref.sum(0), want)
    with pytest.raises(RuntimeError):   # size not a multiple of 4
        call("detllm_igemv_nt_pf", a, w, ref, M, N, K, ks, M * N, pfs[0], 6, None, 0, None, 0,
             None, 0)
    with pytest.raises(RuntimeError):   # size without a pointer
        call("detllm_igemv_nt_pf", a, w, ref, M, N, K, ks, M * N, None, 8, None, 0, None, 0,
             None, 0)



def test_merge_rowcol_extreme_rows():
    """The attention-output merge (detllm_merge_rowcol) on rows whose scaled
    values reach every branch of its row maximum: ordinary magnitudes, values
    in [2^62, 2^63), an exact INT64_MIN in a row that is shifted and in one
    that is not, products that wrap modulo 2^64, a zero row and a row of
    INT64_MIN only, against the oracle's requant_i8_rowcol of the same int64
    products (dyadic.py:123-139)."""
    from idempotent_llm_amd._lib import call
    print("[merge_rowcol extreme rows]", flush=True)
    rng = np.random.default_rng(77)
    R, C = 6, 2048
    os_m = rng.integers(1 << 10, 1 << 12, C).astype(I64)
    col_m = rng.integers(1 << 10, 1 << 12, C).astype(I64)
    fac = os_m * col_m                        # the per-column factor, below 2^24
    attn = np.zeros((R, C), I64)
    attn[0] = rng.integers(-(1 << 30), 1 << 30, C)
    attn[1] = rng.integers(-(1 << 40), 1 << 40, C)            # |v| up to ~2^63
    attn[2] = rng.integers(-(1 << 30), 1 << 30, C)
    j = int(rng.integers(0, C))
    f2 = int(fac[j]) & -int(fac[j])                           # largest power of two in fac[j]
    fac[j] = f2 if f2 > 1 else 2
    attn[2, j] = -(1 << 63) // int(fac[j])                    # attn * fac = INT64_MIN exactly
    attn[3] = rng.integers(-(1 << 50), 1 << 50, C)            # products wrap modulo 2^64
    # row 5: small values and one INT64_MIN, which the unshifted row keeps
    attn[5] = rng.integers(-1000, 1001, C)
    j5 = (j + 1 + int(rng.integers(0, C - 1))) % C
    fac[j5] = 1 << 12
    attn[5, j5] = -(1 << 51)
    # row 5: INT64_MIN in every column (factor a power of two per column)
    p2 = np.ones(C, I64) << rng.integers(1, 23, C)
    attn5 = -(np.ones(C, I64) << (63 - np.log2(p2).astype(I64)))
    with np.errstate(over="ignore"):
        v = attn * fac
    v5 = attn5 * p2
    assert (v5 == np.iinfo(np.int64).min).all()
    for attn_r, fac_r, v_r in ((attn, fac, v), (np.stack([attn5] * R), p2, np.stack([v5] * R))):
        a8 = torch.empty(R, C, dtype=torch.int8, device="cuda")
        am = torch.empty(R, dtype=torch.int64, device="cuda")
        ak = torch.empty(R, dtype=torch.int64, device="cuda")
        call("detllm_merge_rowcol", g(np.ascontiguousarray(attn_r[None])), 1, R * C, R, C,
             g(fac_r), 7, g(np.ones(C, I64)), 9, a8, am, ak, None, 0, 0, 0, 0)
        wy, wm, wk = ody.requant_i8_rowcol(v_r, np.ones((R, 1), I64), np.full((R, 1), 7, I64),
                                           np.ones(C, I64), 9)
        np.testing.assert_array_equal(a8.cpu().numpy(), wy)
        np.testing.assert_array_equal(am.cpu().numpy(), wm.reshape(-1))
        np.testing.assert_array_equal(ak.cpu().numpy(), wk.reshape(-1))
    assert v[5].min() == np.iinfo(np.int64).min and np.abs(v[5][v[5] > -(1 << 62)]).max() < 1 << 46


def test_quant_i8_pertoken_extreme_rows():
    """detllm_op_quant_i8_pertoken (dyadic.py:93-105) on rows holding
    INT64_MIN, whose |x| wraps to itself and is skipped by the row maximum:
    alone among small values, a whole row of it, next to INT64_MAX, and
    ordinary rows on both quotient paths, against the oracle."""
    from idempotent_llm_amd import dyadic as dd
    print("[quant_i8_pertoken extreme rows]", flush=True)
    rng = np.random.default_rng(78)
    lo, hi = np.iinfo(np.int64).min, np.iinfo(np.int64).max
    for C in (1024, 3000):
        x = np.zeros((6, C), I64)
        x[0] = rng.integers(-1000, 1001, C)
        x[0, C // 3] = lo
        x[1] = lo
        x[2] = rng.integers(-(1 << 60), 1 << 60, C)
        x[2, 5], x[2, 7] = lo, hi
        x[3] = rng.integers(-(1 << 40), 1 << 40, C)               # below 2^43: estimate path
        x[4] = rng.integers(-(1 << 50), 1 << 50, C)               # above: exact path
        m = rng.integers(1 << 14, 1 << 16, (6, 1)).astype(I64)
        k = np.full((6, 1), 20, I64)
        want = ody.quant_i8_pertoken(x, m, k)
        got = dd.quant_i8_pertoken(g(x), g(m), g(k))
        for a, b in zip(got, want):
            np.testing.assert_array_equal(a.cpu().numpy(), b)


def test_deferred_scale_fit():
    """detllm_merge_rowcol / detllm_swiglu_quant with defer_fit = 1 store
    (num, k without e) in place of (m, k), where (m, e) = fit_dyadic_ratio(num,
    127) (dyadic.py:52-72); detllm_residual_normq with row_fit = 1 finishes
    that fit. Each producer's int8 rows equal the undeferred launch's, its
    stored pair fits (by the oracle) to the undeferred (m, k), and the
    consumer's residual, int8 operand and scales equal the undeferred
    chain's bit for bit. Flags other than 0 and 1 are refused."""
    from idempotent_llm_amd._lib import call
    print("[deferred scale fit]", flush=True)
    rng = np.random.default_rng(91)
    R, C, H, I = 8, 2048, 1024, 3072

    def residual(P, rm, rk, fit):
        h = g(rng_h.copy())
        kr = g(np.full(R, 24, I64))
        x8 = torch.empty(R, H, dtype=torch.int8, device="cuda")
        xm = torch.empty(R, dtype=torch.int64, device="cuda")
        xk = torch.empty(R, dtype=torch.int64, device="cuda")
        call("detllm_residual_normq", P, 1, 0, R, H, rm, rk, col_m, 20, 20, h, kr, sm_m, 15,
             x8, xm, xk, None, 0, 0, 0, fit)
        return [t.cpu().numpy() for t in (h, kr, x8, xm, xk)]

    def fits_to(num, k_def, m_ref, k_ref):
        m, e = ody.fit_dyadic_ratio(num.cpu().numpy(), 127)
        np.testing.assert_array_equal(np.asarray(m).reshape(-1), m_ref.cpu().numpy())
        np.testing.assert_array_equal(k_def.cpu().numpy() + np.asarray(e).reshape(-1),
                                      k_ref.cpu().numpy())

    rng_h = rng.integers(-(1 << 29), 1 << 29, (R, H)).astype(np.int32)
    col_m = g(rng.integers(1 << 15, 1 << 16, H).astype(I64))
    sm_m = g(rng.integers(1 << 15, 1 << 16, H).astype(I64))
    P_o = g(rng.integers(-(1 << 19), 1 << 19, (1, R, H)).astype(np.int32))
    # merge -> (o GEMM partials) -> residual
    mags = [1 << 20, 1 << 26, 1 << 5, 0, 1 << 23, 1 << 29, 1 << 12, 1 << 27]
    attn = np.stack([rng.integers(-m, m + 1, C) if m else np.zeros(C, I64) for m in mags])
    os_m = g(rng.integers(1 << 10, 1 << 12, C).astype(I64))
    cm = g(rng.integers(1 << 10, 1 << 12, C).astype(I64))
    outs = []
    for d in (0, 1):
        a8 = torch.empty(R, C, dtype=torch.int8, device="cuda")
        am = torch.empty(R, dtype=torch.int64, device="cuda")
        ak = torch.empty(R, dtype=torch.int64, device="cuda")
        call("detllm_merge_rowcol", g(attn[None]), 1, R * C, R, C, os_m, 7, cm, 9, a8, am, ak,
             None, 0, 0, 0, d)
        outs.append((a8, am, ak))
    assert torch.equal(outs[0][0], outs[1][0])
    fits_to(outs[1][1], outs[1][2], outs[0][1], outs[0][2])
    for u, v in zip(residual(P_o, outs[0][1], outs[0][2], 0),
                    residual(P_o, outs[1][1], outs[1][2], 1)):
        np.testing.assert_array_equal(u, v)
    # swiglu -> (down GEMM partials) -> residual
    P_gu = g(rng.integers(-(1 << 20), 1 << 20, (1, R, 2 * I)).astype(np.int32))
    xm = g(rng.integers(1 << 15, 1 << 16, R).astype(I64))
    xk = g(np.full(R, 20, I64))
    gm = g(rng.integers(1 << 14, 1 << 16, I).astype(I64))
    um = g(rng.integers(1 << 14, 1 << 16, I).astype(I64))
    dsm = g(rng.integers(1 << 14, 1 << 16, I).astype(I64))
    outs = []
    for d in (0, 1):
        y8 = torch.empty(R, I, dtype=torch.int8, device="cuda")
        ym = torch.empty(R, dtype=torch.int64, device="cuda")
        yk = torch.empty(R, dtype=torch.int64, device="cuda")
        call("detllm_swiglu_quant", P_gu, 1, R * 2 * I, R, I, xm, xk, gm, 20, um, 20, dsm, 15,
             y8, ym, yk, None, 0, 0, 0, d)
        outs.append((y8, ym, yk))
    assert torch.equal(outs[0][0], outs[1][0])
    fits_to(outs[1][1], outs[1][2], outs[0][1], outs[0][2])
    for u, v in zip(residual(P_o, outs[0][1], outs[0][2], 0),
                    residual(P_o, outs[1][1], outs[1][2], 1)):
        np.testing.assert_array_equal(u, v)
    # flags other than 0 / 1
    with pytest.raises(RuntimeError, match="code -22"):
        call("detllm_merge_rowcol", g(attn[None]), 1, R * C, R, C, os_m, 7, cm, 9,
             outs[0][0][:, :1].contiguous(), outs[0][1], outs[0][2], None, 0, 0, 0, 2)
    with pytest.raises(RuntimeError, match="code -22"):
        residual(P_o, outs[0][1], outs[0][2], 2)
    torch.cuda.synchronize()


@pytest.mark.parametrize("R", [3, 100])
def test_swiglu_quant_every_path(R):
    """detllm_swiglu_quant (model.py:416-423: requant_i32_common(14) of gate
    and up, di_swiglu, the ds_m smoothing multiply, quant_i8_pertoken)
    against the oracle's composition, at decode (3 rows) and prefill (100
    rows) sizes, on inputs that take each path of the kernel: ordinary
    mantissas (fp64 chain); a gate mantissa of 2^21 or more (integer
    requantisation); a ds_m of 2^18 or more (integer quantisation); ds_m
    near 2^17 with large products (a row maximum of 2^43 or more); a row
    scale giving tpos >= 2^23 (64-bit DI-Exp); and a zero row."""
    from idempotent_llm_amd._lib import call
    rng = np.random.default_rng(93)
    I = 3072
    base = dict(gm=rng.integers(1 << 14, 1 << 16, I), um=rng.integers(1 << 14, 1 << 16, I),
                dsm=rng.integers(1 << 12, 1 << 14, I))
    cases = {"fp64": {}, "big_gate_m": {"gm_big": True}, "big_ds_m": {"ds_big": True},
             "row_max_2^43": {"ds_near": True}, "big_tpos": {"xk": 50}}
    for name, c in cases.items():
        gm, um, dsm = base["gm"].copy(), base["um"].copy(), base["dsm"].copy()
        if c.get("gm_big"):
            gm[17] = 1 << 22
        if c.get("ds_big"):
            dsm[5] = (1 << 18) + 3
        if c.get("ds_near"):
            dsm[:] = rng.integers((1 << 17) - 1000, 1 << 17, I)
        P = rng.integers(-(1 << 24), 1 << 24, (R, 2 * I)).astype(np.int32)
        P[0] = 0
        xm = rng.integers(1 << 15, 1 << 16, (R, 1)).astype(I64)
        xk = np.full((R, 1), c.get("xk", 20), I64)
        gate, ogm, ogk = ody.requant_i32_common(P[:, :I], xm, xk, gm.astype(I64), 20, 14)
        up, oum, ouk = ody.requant_i32_common(P[:, I:], xm, xk, um.astype(I64), 20, 14)
        ys, ym, yk = oops.di_swiglu(gate, ogm, ogk, up, oum, ouk)
        wy, wm, wk = ody.quant_i8_pertoken(ys * dsm.astype(I64), ym, yk + 15)
        y8 = torch.empty(R, I, dtype=torch.int8, device="cuda")
        gym = torch.empty(R, dtype=torch.int64, device="cuda")
        gyk = torch.empty(R, dtype=torch.int64, device="cuda")
        print(f"[swiglu_quant R={R} {name}]", flush=True)
        call("detllm_swiglu_quant", g(P[None]), 1, R * 2 * I, R, I, g(xm[:, 0]), g(xk[:, 0]),
             g(gm.astype(I64)), 20, g(um.astype(I64)), 20, g(dsm.astype(I64)), 15, y8, gym, gyk,
             None, 0, 0, 0, 0)
        eq(y8, wy); eq(gym, wm[:, 0]); eq(gyk, wk[:, 0])


@pytest.mark.parametrize("C", [1024, 3072])
@pytest.mark.parametrize("big_sm", [False, True])
def test_norm_quant_every_path(C, big_sm):
    """_norm_quant (model.py:187-198: di_rmsnorm, the smoothing product,
    quant_i8_pertoken) through detllm_norm_quant against the oracle, on rows
    that take each side of the row kernel's fp64 path: random rows of every
    magnitude (up- and down-shifts of the normalisation), a zero row (rms 1:
    the integer routines), a one-hot row, and at 3072 columns a row of
    near-maximal values whose sum of squares passes 2^63 and wraps as
    torch's does. With big_sm one smoothing mantissa is 2^21 (the quantiser
    on int64 products); without, one is -(2^21 - 1)."""
    from idempotent_llm_amd._lib import call
    print(f"[norm_quant every path C={C} big_sm={big_sm}]", flush=True)
    rng = np.random.default_rng(C + 5 * big_sm)
    scale = [2 ** 12, 2 ** 20, 2 ** 29 - 3, 2 ** 30, 0, 0, 2 ** 25, 7]
    R = len(scale)
    h = np.stack([rng.integers(-s, s + 1, C) if s else np.zeros(C, I64) for s in scale])
    h[5, C // 2] = -3                                  # one-hot
    if C == 3072:
        h[3] = np.where(rng.integers(0, 2, C) == 1, 1, -1) * ((1 << 30) - 1)
    h = h.astype(np.int32)
    sm_m = rng.integers(1 << 15, 1 << 16, C).astype(I64)
    sm_m[C // 3] = (1 << 21) if big_sm else -((1 << 21) - 1)
    y = oops.di_rmsnorm(h).astype(I64) * sm_m
    if C == 3072:
        xp = oim.rshift_round(h[3].astype(I64), 4)       # the shift to [2^25, 2^26]
        assert sum(int(v) * int(v) for v in xp) >= 1 << 63  # the sum of squares wraps
    kq = np.full((R, 1), 20 + 15, I64)
    want = ody.quant_i8_pertoken(y, np.ones_like(kq), kq)
    x8 = torch.empty(R, C, dtype=torch.int8, device="cuda")
    xm = torch.empty(R, dtype=torch.int64, device="cuda")
    xk = torch.empty(R, dtype=torch.int64, device="cuda")
    call("detllm_norm_quant", g(h), R, C, g(sm_m), 15, x8, xm, xk)
    eq(x8, want[0]); eq(xm, want[1][:, 0]); eq(xk, want[2][:, 0])
