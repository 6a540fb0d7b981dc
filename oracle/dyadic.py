"""Dyadic-scale bookkeeping, restated from ``src/detllm/dyadic.py``.

A quantised tensor is (data, m, k) with value ~= data * m / 2^k; m and k are
int64 arrays broadcastable to the data's leading shape (per-row ``[..., 1]``).

Pinned: tests/golden/dyadic.npz (vectors written from the reference's CPU
path by tests/golden/make_golden.py) plus exact special cases restated from
the reference's tests/test_dyadic.py:29-33, :68-78.
"""

from __future__ import annotations

import numpy as np

from .intmath import (I64, as64, clamp_i8, ilog2, rhad, rshift_round,
                      rshift_round_t, shl, to_i32)


def scaled_round_div(num, den, e):
    """dyadic.py:45-49 — rhad(num << max(e,0), den << max(-e,0))."""
    e = as64(e)
    epos = np.maximum(e, 0)
    eneg = np.maximum(-e, 0)
    return rhad(shl(num, epos), shl(den, eneg))


def fit_dyadic_ratio(num, den, bits: int = 16):
    """dyadic.py:52-72 — m/2^e ~= num/den, m in [2^(bits-1), 2^bits)."""
    num = as64(num)
    den = np.broadcast_to(as64(den), num.shape)
    L = ilog2(num) - ilog2(den)
    e = (bits - 1) - L
    m = scaled_round_div(num, den, e)
    adj = np.where(m >= (1 << bits), -1, 0) + np.where(m < (1 << (bits - 1)), 1, 0)
    adj = adj.astype(I64)
    e = e + adj
    m = np.where(adj != 0, scaled_round_div(num, den, e), m)
    over = m >= (1 << bits)
    m = np.where(over, rshift_round(m, 1), m)
    e = e - over.astype(I64)
    return m.astype(I64), e.astype(I64)


def norm_scale(m, k, bits: int = 16):
    """dyadic.py:75-90 — renormalise m into [2^(bits-1), 2^bits)."""
    m = as64(m)
    k = as64(k)
    sh = (bits - 1) - ilog2(np.maximum(m, 1))
    up = np.maximum(sh, 0)
    down = np.maximum(-sh, 0)
    m2 = rshift_round_t(shl(m, up), down)
    over = m2 >= (1 << bits)
    m2 = np.where(over, rshift_round(m2, 1), m2)
    sh = sh - over.astype(I64)
    return m2.astype(I64), (k + sh).astype(I64)


def quant_i8_pertoken(x, m, k):
    """dyadic.py:93-105 — symmetric per-row int8 quantisation."""
    m, k = norm_scale(m, k)
    x64 = as64(x)
    a = np.abs(x64).max(axis=-1, keepdims=True)
    a = np.maximum(a, 1)
    x8 = clamp_i8(rhad(x64 * I64(127), a))
    m_out, e = fit_dyadic_ratio(a * m, 127)
    return x8, m_out, k + e


def requant_i32_common(P, row_m, row_k, col_m, col_k, target_bits: int = 12):
    """dyadic.py:108-120 — shift-only requant to ~target_bits per row."""
    scaled = as64(P) * as64(col_m)
    a = np.abs(scaled).max(axis=-1, keepdims=True)
    a = np.maximum(a, 1)
    sh = np.maximum(ilog2(a) - (target_bits - 1), 0)
    y = to_i32(rshift_round_t(scaled, np.broadcast_to(sh, scaled.shape)))
    return y, as64(row_m), as64(row_k) + as64(col_k) - sh


def requant_i8_rowcol(P, row_m, row_k, col_m, col_k):
    """dyadic.py:123-139 — GEMM output straight to per-row int8."""
    scaled = as64(P) * as64(col_m)
    a = np.abs(scaled).max(axis=-1, keepdims=True)
    a = np.maximum(a, 1)
    sh = np.maximum(ilog2(a) - 45, 0)
    scaled = rshift_round_t(scaled, np.broadcast_to(sh, scaled.shape))
    a = np.maximum(np.abs(scaled).max(axis=-1, keepdims=True), 1)
    y8 = clamp_i8(rhad(scaled * I64(127), a))
    m_out, e = fit_dyadic_ratio(a * as64(row_m), 127)
    return y8, m_out, as64(row_k) + as64(col_k) + e - sh


def requant_i8_static(P, row_m, row_k, col_m, col_k, s_m, s_k):
    """dyadic.py:142-163 — int8 at a static dyadic target scale s_m/2^s_k."""
    num = as64(P) * as64(col_m) * as64(row_m)
    shift = np.broadcast_to(as64(row_k) + as64(col_k) - as64(s_k), num.shape)
    up = np.maximum(-shift, 0)
    down = np.maximum(shift, 0)
    num = shl(num, up)
    den = shl(np.broadcast_to(as64(s_m), num.shape), down)
    return clamp_i8(rhad(num, den))


RES_MAX_BITS = 30
RES_MIN_BITS = 24


def residual_renorm(h64, k_res):
    """dyadic.py:174-184 — per-row max|h| into [2^26, 2^30)."""
    h64 = as64(h64)
    g = np.abs(h64).max(axis=-1, keepdims=True)
    lg = ilog2(np.maximum(g, 1))
    sh_down = np.maximum(lg - (RES_MAX_BITS - 1), 0)
    sh_up = np.where(g > 0, np.maximum((RES_MIN_BITS + 2) - lg, 0), 0).astype(I64)
    sh_up = np.where(sh_down > 0, 0, sh_up).astype(I64)
    h64 = rshift_round_t(h64, np.broadcast_to(sh_down, h64.shape))
    h64 = shl(h64, np.broadcast_to(sh_up, h64.shape))
    return to_i32(h64), as64(k_res) - sh_down + sh_up


def residual_from_delta(d, dm, dk):
    """dyadic.py:187-190."""
    return residual_renorm(as64(d) * as64(dm), as64(dk))


def residual_add(h, k_res, d, dm, dk):
    """dyadic.py:193-206 — align the delta to k_res, add, renormalise."""
    d64 = as64(d) * as64(dm)
    rel = as64(dk) - as64(k_res)
    down = np.maximum(rel, 0)
    up = np.maximum(-rel, 0)
    d_aligned = shl(rshift_round_t(d64, np.broadcast_to(down, d64.shape)),
                    np.broadcast_to(up, d64.shape))
    return residual_renorm(as64(h) + d_aligned, k_res)
