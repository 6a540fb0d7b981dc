"""GPU parity of the decode GEMVs with their operand's row kernel fused in
(detllm_igemv_resnormq, detllm_igemv_merge) against the two launches they
replace: the row kernel (detllm_residual_normq / detllm_merge_rowcol, whose
own parity with the oracle is pinned in test_gpu_ops and the model tests)
followed by detllm_igemv_nt. Every output — partials, residual, row scales —
must be equal bit for bit; the product is also checked against the oracle's
int_gemm of the row kernel's int8 operand."""

import numpy as np
import pytest
import torch

from oracle import gemm as ogemm

pytestmark = pytest.mark.gpu
I64 = np.int64


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from idempotent_llm_amd import _lib
    _lib.load()   # fails loudly if the HIP library is missing


def g(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _fused_split(R, N, K):
    """The product's planned K split when the fused kernel covers it, else
    the widest split it covers (the model only fuses covered plans)."""
    from idempotent_llm_amd._lib import gemv_plan, pro_fits
    ks = gemv_plan(R, N, K)
    if pro_fits(K, ks):
        return ks
    return next(k for k in (4, 2, 1) if pro_fits(K, k))


def _split_product(x8, w, ks):
    from idempotent_llm_amd._lib import call
    R, K = x8.shape
    N = w.shape[0]
    P = torch.full((ks, R, N), -7, dtype=torch.int32, device="cuda")
    call("detllm_igemv_nt", x8, w, P, R, N, K, ks, R * N)
    return P


# residual rows that take the renormalisation branches of residual_normq
# (sum above 2^30, small rows, rows left in range, zero and one-hot rows)
SCALES = [2 ** 29 - 3, 2 ** 20, 2 ** 28, 0, 0, 2 ** 27, 2 ** 12, 2 ** 29]


@pytest.mark.parametrize("R", [1, 3, 8])
@pytest.mark.parametrize("N,K,nsplit,smooth", [
    (4096, 1024, 1, True),     # qkv after the down residual: one column group per block
    (6144, 1024, 1, True),     # gate|up after the o residual: two column groups per block
    (1000, 1024, 2, False),    # ragged N, summed residual partials, no smoothing
    (3072, 512, 3, True),      # shorter rows (masked lanes of the row helpers)
])
def test_igemv_resnormq_equals_two_launches(R, N, K, nsplit, smooth):
    from idempotent_llm_amd._lib import call
    print(f"[igemv_resnormq R={R} N={N} K={K} nsplit={nsplit} smooth={smooth}]", flush=True)
    rng = np.random.default_rng(R * 7919 + N + K + nsplit)
    sc = SCALES[:R] if R > 1 else [2 ** 29 - 3]
    h = np.stack([rng.integers(-s, s + 1, K) if s else np.zeros(K, I64) for s in sc])
    if R > 4:
        h[4, K // 3] = 5
    h = h.astype(np.int32)
    P = rng.integers(-(1 << 19), 1 << 19, (nsplit, R, K)).astype(np.int32)
    if R > 4:
        P[:, 3] = 0
        P[:, 4] = 0
    row_m = g(rng.integers(1 << 15, 1 << 16, R).astype(I64))
    row_k = g(np.array([20, 24, 26, 20, 20, 30, 40, 19][:R], I64))
    k_res = g(np.full(R, 24, I64))
    col_m = g(rng.integers(1 << 15, 1 << 16, K).astype(I64))
    sm_m = g(rng.integers(1 << 15, 1 << 16, K).astype(I64)) if smooth else None
    w = g(rng.integers(-128, 128, (N, K)).astype(np.int8))
    Pg = g(P)
    ks = _fused_split(R, N, K)
    # the two launches
    h_ref, k_ref = g(h), k_res.clone()
    x8 = torch.empty(R, K, dtype=torch.int8, device="cuda")
    xm = torch.empty(R, dtype=torch.int64, device="cuda")
    xk = torch.empty(R, dtype=torch.int64, device="cuda")
    call("detllm_residual_normq", Pg, nsplit, R * K, R, K, row_m, row_k, col_m, 20, 20, h_ref,
         k_ref, sm_m, 15, x8, xm, xk, None, 0, 0, 0, 0)
    want = _split_product(x8, w, ks)
    # fused, twice in a row (the second call must not see the first's outputs)
    h_in = g(h)
    k_in = k_res.clone()
    pf = g(rng.integers(0, 9, 4096).astype(I64))
    for rep in range(2):
        h_out = torch.full((R, K), -1, dtype=torch.int32, device="cuda")
        k_out = torch.full((R,), -1, dtype=torch.int64, device="cuda")
        fm = torch.full((R,), -1, dtype=torch.int64, device="cuda")
        fk = torch.full((R,), -1, dtype=torch.int64, device="cuda")
        C = torch.full((ks, R, N), -7, dtype=torch.int32, device="cuda")
        call("detllm_igemv_resnormq", w, C, R, N, K, ks, R * N, Pg, nsplit, R * K, row_m, row_k,
             col_m, 20, 20, h_in, k_in, h_out, k_out, sm_m, 15, fm, fk,
             pf if rep else None, pf.numel() * 8 if rep else 0, None, 0)
        assert torch.equal(C, want)
        assert torch.equal(h_out, h_ref) and torch.equal(k_out, k_ref)
        assert torch.equal(fm, xm) and torch.equal(fk, xk)
        assert torch.equal(h_in, g(h)) and torch.equal(k_in, k_res)   # inputs untouched
    prod = ogemm.int_gemm(x8.cpu().numpy(), w.cpu().numpy().T)
    assert np.array_equal(want.sum(0).cpu().numpy().astype(I64), prod.astype(I64))


@pytest.mark.parametrize("R", [1, 3, 8])
@pytest.mark.parametrize("N,K,nsplit,combined", [
    (1024, 2048, 1, False),    # o projection (K split 4)
    (1024, 2048, 1, True),     # o projection with the per-column factor pre-multiplied
    (2000, 1024, 3, False),    # ragged N, summed attention partials
])
def test_igemv_merge_equals_two_launches(R, N, K, nsplit, combined):
    from idempotent_llm_amd._lib import call
    print(f"[igemv_merge R={R} N={N} K={K} nsplit={nsplit} combined={combined}]", flush=True)
    rng = np.random.default_rng(R * 104729 + N + K + nsplit + combined)
    # row magnitudes across the quantiser's branches: |attn * os_m * col_m|
    # below 2^43, in [2^43, 2^46) and above (pre-shift), one zero row
    mags = [1 << 20, 1 << 26, 1 << 5, 0, 1 << 23, 1 << 29, 1 << 12, 1 << 27][:R]
    attn = np.stack([rng.integers(-m, m + 1, (nsplit, K)) if m else np.zeros((nsplit, K), I64)
                     for m in mags], axis=1).astype(I64)
    os_m = rng.integers(1 << 10, 1 << 12, K).astype(I64)
    col_m = rng.integers(1 << 10, 1 << 12, K).astype(I64)
    ag = g(attn)
    w = g(rng.integers(-128, 128, (N, K)).astype(np.int8))
    ks = _fused_split(R, N, K)
    a8 = torch.empty(R, K, dtype=torch.int8, device="cuda")
    am = torch.empty(R, dtype=torch.int64, device="cuda")
    ak = torch.empty(R, dtype=torch.int64, device="cuda")
    call("detllm_merge_rowcol", ag, nsplit, R * K, R, K, g(os_m), 7, g(col_m), 9, a8, am, ak, None, 0, 0, 0, 0)
    want = _split_product(a8, w, ks)
    if combined:
        f_os, f_col = g(os_m * col_m), None
    else:
        f_os, f_col = g(os_m), g(col_m)
    for rep in range(2):
        fm = torch.full((R,), -1, dtype=torch.int64, device="cuda")
        fk = torch.full((R,), -1, dtype=torch.int64, device="cuda")
        C = torch.full((ks, R, N), -7, dtype=torch.int32, device="cuda")
        call("detllm_igemv_merge", w, C, R, N, K, ks, R * N, ag, nsplit, R * K, f_os, 7, f_col, 9,
             fm, fk, None, 0, None, 0)
        assert torch.equal(C, want)
        assert torch.equal(fm, am) and torch.equal(fk, ak)
    prod = ogemm.int_gemm(a8.cpu().numpy(), w.cpu().numpy().T)
    assert np.array_equal(want.sum(0).cpu().numpy().astype(I64), prod.astype(I64))
    # the shifted rows do reach every branch of the int8 quantiser
    v = attn.sum(0) * os_m * col_m
    top = np.abs(v).max(axis=1)
    if R == 8:
        assert (top < 2 ** 43).any() and (top >= 2 ** 46).any()
        assert ((top >= 2 ** 43) & (top < 2 ** 46)).any()


def _merge_stats(v, n_ext):
    """detllm_qkv_attn_decode_ext's statistics of rows v [R][K] (int64): per
    part of K / n_ext columns the largest v and the largest ~v, each taken
    together with 0 (for v) and ~0 (for ~v)."""
    R, K = v.shape
    parts = v.reshape(R, n_ext, K // n_ext)
    hi = np.maximum(parts.max(axis=2), 0)
    nm = np.maximum((~parts).max(axis=2), -1)
    return np.stack([hi, nm], axis=2).astype(I64)


@pytest.mark.parametrize("R", [1, 3, 8])
@pytest.mark.parametrize("N,ks_pick,defer", [(1024, "plan", 1), (1024, 4, 0), (2000, 2, 1)])
def test_igemv_merge_ext_equals_two_launches(R, N, ks_pick, defer):
    """The o-GEMV that quantises only its own K range of the merged rows
    from their statistics (detllm_igemv_merge_ext) against detllm_merge_rowcol
    then detllm_igemv_nt: equal partials and row scales (fitted and deferred),
    rows in every tier of the int8 quantiser, a zero row, and rows with values
    at or beyond 2^62 (wrapping products included) that take the full-row
    fallback."""
    from idempotent_llm_amd._lib import call, pro_fits
    K, n_ext = 2048, 8
    ks = _fused_split(R, N, K) if ks_pick == "plan" else ks_pick
    assert pro_fits(K, ks)
    print(f"[igemv_merge_ext R={R} N={N} ks={ks} defer={defer}]", flush=True)
    rng = np.random.default_rng(R * 31337 + N + ks + defer)
    mags = [1 << 20, 1 << 39, 1 << 5, 0, 1 << 23, 1 << 29, 1 << 12, 1 << 38][:R]
    if R == 1:
        mags = [1 << 39] if defer else [1 << 26]
    attn = np.stack([rng.integers(-m, m + 1, K) if m else np.zeros(K, I64) for m in mags]).astype(I64)
    os_m = rng.integers(1 << 10, 1 << 12, K).astype(I64)
    col_m = rng.integers(1 << 10, 1 << 12, K).astype(I64)
    om = os_m * col_m
    with np.errstate(over="ignore"):
        v = attn * om
    ext = _merge_stats(v, n_ext)
    ag = g(attn)
    w = g(rng.integers(-128, 128, (N, K)).astype(np.int8))
    a8 = torch.empty(R, K, dtype=torch.int8, device="cuda")
    am = torch.empty(R, dtype=torch.int64, device="cuda")
    ak = torch.empty(R, dtype=torch.int64, device="cuda")
    call("detllm_merge_rowcol", ag, 1, R * K, R, K, g(os_m), 7, g(col_m), 9, a8, am, ak, None, 0,
         0, 0, defer)
    want = _split_product(a8, w, ks)
    for rep in range(2):
        fm = torch.full((R,), -1, dtype=torch.int64, device="cuda")
        fk = torch.full((R,), -1, dtype=torch.int64, device="cuda")
        C = torch.full((ks, R, N), -7, dtype=torch.int32, device="cuda")
        call("detllm_igemv_merge_ext", w, C, R, N, K, ks, R * N, ag, g(om), 7, 9, g(ext), n_ext,
             fm, fk, defer, None, 0, None, 0)
        assert torch.equal(C, want)
        assert torch.equal(fm, am) and torch.equal(fk, ak)
    prod = ogemm.int_gemm(a8.cpu().numpy(), w.cpu().numpy().T)
    assert np.array_equal(want.sum(0).cpu().numpy().astype(I64), prod.astype(I64))
    if R == 8:
        # the rows reach every tier and the fallback
        top = np.abs(v).max(axis=1)
        assert (top >= 2 ** 62).any() and (top < 2 ** 43).any()
    with pytest.raises(RuntimeError, match="code -22"):
        call("detllm_igemv_merge_ext", w, C, R, N, K, ks, R * N, ag, g(om), 7, 9, g(ext), 9,
             fm, fk, defer, None, 0, None, 0)


@pytest.mark.parametrize("R,C,n_ext", [(1, 2048, 8), (3, 1000, 5), (8, 2048, 8), (17, 2048, 8)])
@pytest.mark.parametrize("defer", [0, 1])
def test_merge_ext_equals_merge_rowcol(R, C, n_ext, defer):
    """detllm_merge_ext (the merge from the attention's row statistics, in
    256-column pieces) against detllm_merge_rowcol: equal int8 rows and row
    scales, fitted and deferred, with rows in every quantiser tier, a zero
    row, ragged columns, and rows at or beyond 2^62 (wrapping products) that
    each piece block merges in full."""
    from idempotent_llm_amd._lib import call
    print(f"[merge_ext R={R} C={C} n_ext={n_ext} defer={defer}]", flush=True)
    rng = np.random.default_rng(R * 131 + C + n_ext + defer)
    base = [1 << 20, 1 << 39, 1 << 5, 0, 1 << 23, 1 << 29, 1 << 12, 1 << 38]
    mags = [base[i % 8] for i in range(R)] if R > 1 else [1 << 26]
    attn = np.stack([rng.integers(-m, m + 1, C) if m else np.zeros(C, I64) for m in mags]).astype(I64)
    os_m = rng.integers(1 << 10, 1 << 12, C).astype(I64)
    col_m = rng.integers(1 << 10, 1 << 12, C).astype(I64)
    om = os_m * col_m
    with np.errstate(over="ignore"):
        v = attn * om
    ext = _merge_stats(v, n_ext)
    ag = g(attn)
    want8 = torch.full((R, C), 99, dtype=torch.int8, device="cuda")
    wm = torch.empty(R, dtype=torch.int64, device="cuda")
    wk = torch.empty(R, dtype=torch.int64, device="cuda")
    call("detllm_merge_rowcol", ag, 1, R * C, R, C, g(os_m), 7, g(col_m), 9, want8, wm, wk, None,
         0, 0, 0, defer)
    w = torch.zeros(4096, C, dtype=torch.int8, device="cuda")   # warming blocks' target
    for rep in range(2):
        a8 = torch.full((R, C), 99, dtype=torch.int8, device="cuda")
        am = torch.full((R,), -1, dtype=torch.int64, device="cuda")
        ak = torch.full((R,), -1, dtype=torch.int64, device="cuda")
        call("detllm_merge_ext", ag, R, C, g(om), 7, 9, g(ext), n_ext, a8, am, ak,
             w if rep else None, 4096 if rep else 0, C if rep else 0, 1, defer)
        torch.cuda.synchronize()
        assert torch.equal(a8, want8)
        assert torch.equal(am, wm) and torch.equal(ak, wk)
    if R == 8:
        top = np.abs(v).max(axis=1)
        assert (top >= 2 ** 62).any() and (top < 2 ** 43).any()


def test_fused_gemv_argument_errors():
    """Rows beyond 8, aliased residual buffers and shapes the fused kernel
    does not cover are refused before any launch (the last with -38, the
    caller's cue to run the two launches)."""
    from idempotent_llm_amd._lib import call, pro_fits
    print("[fused gemv argument errors]", flush=True)
    K, N = 1024, 256
    w = torch.zeros(N, K, dtype=torch.int8, device="cuda")
    P = torch.zeros(1, 9, K, dtype=torch.int32, device="cuda")
    m = torch.ones(9, dtype=torch.int64, device="cuda")
    col = torch.ones(K, dtype=torch.int64, device="cuda")
    h = torch.zeros(9, K, dtype=torch.int32, device="cuda")
    h2 = torch.zeros(9, K, dtype=torch.int32, device="cuda")
    kr = torch.zeros(9, dtype=torch.int64, device="cuda")
    kr2 = torch.zeros(9, dtype=torch.int64, device="cuda")
    C = torch.zeros(8, 9, N, dtype=torch.int32, device="cuda")

    def rn(R, ks, h_out, k_out):
        call("detllm_igemv_resnormq", w, C, R, N, K, ks, 9 * N, P, 1, 9 * K, m, m, col, 20, 20,
             h, kr, h_out, k_out, None, 0, m, m, None, 0, None, 0)

    with pytest.raises(RuntimeError, match="code -22"):
        rn(9, 1, h2, kr2)
    with pytest.raises(RuntimeError, match="code -22"):
        rn(8, 1, h, kr2)
    with pytest.raises(RuntimeError, match="code -38"):
        rn(8, 8, h2, kr2)          # K chunks of 128 bytes
    assert not pro_fits(K, 8) and pro_fits(K, 1) and pro_fits(K, 2)
    assert pro_fits(2048, 4) and pro_fits(2048, 2) and not pro_fits(2048, 1)
    rn(8, 2, h2, kr2)              # covered: runs
    torch.cuda.synchronize()


@pytest.mark.parametrize("I,ks", [(3072, 3), (3072, 6), (1024, 1), (1024, 2)])
@pytest.mark.parametrize("case", ["fp64", "big_gate_m", "big_ds_m", "big_tpos"])
def test_igemv_swiglu_equals_two_launches(I, ks, case):
    """The one-row down GEMV with its SwiGLU operand fused in
    (detllm_igemv_swiglu) against the two launches it replaces
    (detllm_swiglu_quant, then detllm_igemv_nt with the same K split): equal
    partials and row scale, with the scale fit done and deferred, summed
    gate|up partials, and inputs that take each path of the SwiGLU row (fp64
    chain, a gate mantissa of 2^22: integer requantisation, a ds_m of
    2^18 + 3: integer quantisation, tpos >= 2^23: 64-bit DI-Exp). The
    product is checked against the oracle's int_gemm of the row kernel's
    int8 operand, whose parity with the oracle test_gpu_ops pins."""
    from idempotent_llm_amd._lib import call
    print(f"[igemv_swiglu I={I} ks={ks} {case}]", flush=True)
    rng = np.random.default_rng(I + 31 * ks + len(case))
    N, nsplit = 1024, 2
    gm = rng.integers(1 << 14, 1 << 16, I).astype(I64)
    um = rng.integers(1 << 14, 1 << 16, I).astype(I64)
    dsm = rng.integers(1 << 12, 1 << 14, I).astype(I64)
    if case == "big_gate_m":
        gm[17] = 1 << 22
    if case == "big_ds_m":
        dsm[5] = (1 << 18) + 3
    P = rng.integers(-(1 << 23), 1 << 23, (nsplit, 1, 2 * I)).astype(np.int32)
    xm = g(rng.integers(1 << 15, 1 << 16, 1).astype(I64))
    xk = g(np.full(1, 50 if case == "big_tpos" else 20, I64))
    w = g(rng.integers(-128, 128, (N, I)).astype(np.int8))
    Pg = g(P)
    for defer in (0, 1):
        y8 = torch.empty(1, I, dtype=torch.int8, device="cuda")
        ym = torch.full((1,), -1, dtype=torch.int64, device="cuda")
        yk = torch.full((1,), -1, dtype=torch.int64, device="cuda")
        call("detllm_swiglu_quant", Pg, nsplit, 2 * I, 1, I, xm, xk, g(gm), 20, g(um), 20, g(dsm),
             15, y8, ym, yk, None, 0, 0, 0, defer)
        want = _split_product(y8, w, ks)
        for rep in range(2):
            C = torch.full((ks, 1, N), -7, dtype=torch.int32, device="cuda")
            fm = torch.full((1,), -1, dtype=torch.int64, device="cuda")
            fk = torch.full((1,), -1, dtype=torch.int64, device="cuda")
            pf = g(rng.integers(0, 9, 4096).astype(I64))
            call("detllm_igemv_swiglu", w, C, N, I, ks, N, Pg, nsplit, 2 * I, xm, xk, g(gm), 20,
                 g(um), 20, g(dsm), 15, fm, fk, defer, pf if rep else None,
                 pf.numel() * 8 if rep else 0, None, 0)
            assert torch.equal(C, want)
            assert torch.equal(fm, ym) and torch.equal(fk, yk)
        prod = ogemm.int_gemm(y8.cpu().numpy(), w.cpu().numpy().T)
        assert np.array_equal(want.sum(0).cpu().numpy().astype(I64), prod.astype(I64))
