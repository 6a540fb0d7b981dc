"""Integer operators, restated from ``src/detllm/ops/``.

Pinned: tests/golden/ops.npz (vectors written from the reference CPU path by
tests/golden/make_golden.py) plus the exact special cases the reference's
tests/test_ops.py holds (exp(0) = tpos and tail -> 0 :123-134; masked
invariance and all-masked rows :164-181; RMSNorm scale invariance and zero
rows :202-212), restated in tests/test_oracle_golden.py.
"""

from __future__ import annotations

import numpy as np

from . import dyadic as dy
from .gemm import int_gemm
from .intmath import (I32, I64, as64, floor_div, ilog2, isqrt, rhad,
                      rshift_round, rshift_round_t, shl, shr, to_i32)

P_OUT_BITS = 15          # ops/di_softmax.py:29
OUT_FRAC_BITS = 20       # ops/di_rmsnorm.py:29
TARGET_HI = 25           # ops/di_rmsnorm.py:30
SIG_BITS = 8             # ops/di_swiglu.py:35
ROPE_FRAC_BITS = 14      # ops/rope.py:22
NEG_SENTINEL = np.iinfo(np.int64).min + 1   # ops/di_softmax.py:47


def di_exp(x, m, k):
    """ops/di_exp.py:21-37.

    m_f = m + (m>>1) - (m>>4); tpos = max(rhad(1<<k, m_f), 1); t = -tpos;
    q = floor(x/t); r = x - q*t; result = ((r>>1) - t) >> min(q, 62)."""
    x = as64(x)
    m = as64(m)
    k = as64(k)
    m_f = m + shr(m, 1) - shr(m, 4)
    one = np.ones_like(k)
    tpos = np.maximum(rhad(shl(one, k), m_f), 1)
    t = -tpos
    q = floor_div(x, np.broadcast_to(t, x.shape))
    r = x - q * t
    unshifted = shr(r, 1) - t
    result = shr(unshifted, np.minimum(q, 62))
    return result, tpos


def di_exp_tpos(m, k):
    """The per-row DI-Exp constant tpos alone (model.py:351-358)."""
    m = as64(m)
    k = as64(k)
    m_f = m + shr(m, 1) - shr(m, 4)
    return np.maximum(rhad(shl(np.ones_like(k), k), m_f), 1)


def di_softmax(scores, m, k, valid, clip_c=None, p_out_bits: int = P_OUT_BITS):
    """ops/di_softmax.py:33-61 (probabilities in [0, 2^(p_out_bits-1)])."""
    x = as64(scores)
    m = as64(m)
    k = as64(k)
    valid = np.broadcast_to(np.asarray(valid, dtype=bool), x.shape)
    xm = np.where(valid, x, I64(NEG_SENTINEL))
    row_max = xm.max(axis=-1, keepdims=True)
    any_valid = valid.any(axis=-1, keepdims=True)
    row_max = np.where(any_valid, row_max, 0).astype(I64)
    xd = x - row_max
    xd = np.where(valid, xd, 0).astype(I64)
    if clip_c is not None:
        one = np.ones_like(k)
        c_int = rhad(I64(clip_c) * shl(one, k), m)
        xd = np.maximum(xd, -np.broadcast_to(c_int, xd.shape))
    exps, _tpos = di_exp(xd, m, k)
    exps = np.where(valid, exps, 0).astype(I64)
    denom = np.maximum(exps.sum(axis=-1, keepdims=True), 1)
    probs = rhad(shl(exps, p_out_bits - 1), denom)
    return to_i32(probs)


def di_rmsnorm(x):
    """ops/di_rmsnorm.py:33-52 — y ~= x/rms(x) at scale (1, 20), int32."""
    x64 = as64(x)
    n = x64.shape[-1]
    g = np.abs(x64).max(axis=-1, keepdims=True)
    lg = ilog2(np.maximum(g, 1))
    sh = TARGET_HI - lg
    up = np.maximum(sh, 0)
    down = np.maximum(-sh, 0)
    xp = shl(rshift_round_t(x64, np.broadcast_to(down, x64.shape)),
             np.broadcast_to(up, x64.shape))
    ssum = (xp * xp).sum(axis=-1, keepdims=True)
    mean = rhad(ssum, np.full_like(ssum, n))
    rms = np.maximum(isqrt(mean), 1)
    y = rhad(shl(xp, OUT_FRAC_BITS), np.broadcast_to(rms, xp.shape))
    return to_i32(y)


def di_rmsnorm_gamma(x, gamma_m, gamma_k: int):
    """ops/di_rmsnorm.py:55-64 — (x/rms)*gamma_m, k_out = 20 + gamma_k."""
    y = as64(di_rmsnorm(x)) * as64(gamma_m)
    return y, OUT_FRAC_BITS + gamma_k


def di_swiglu(gate, gm, gk, up, um, uk):
    """ops/di_swiglu.py:39-58 — stable two-branch integer sigmoid."""
    g64 = as64(gate)
    gm = as64(gm)
    gk = as64(gk)
    E, tpos = di_exp(-np.abs(g64), gm, gk)
    tpos_b = np.broadcast_to(tpos, E.shape)
    denom = np.maximum(tpos_b + E, 1)
    num = np.where(g64 >= 0, tpos_b, E)
    sig = rhad(shl(num, SIG_BITS - 1), denom)
    y = g64 * sig * as64(up)
    m_out = gm * as64(um)
    k_out = gk + as64(uk) + (SIG_BITS - 1)
    return y, m_out, k_out


def build_rope_tables(head_dim: int, max_pos: int, base: float):
    """ops/rope.py:25-35 — OFFLINE (float) int16 cos/sin tables, HF tiling."""
    j = np.arange(0, head_dim // 2, dtype=np.float64)
    inv_freq = base ** (-2.0 * j / head_dim)
    pos = np.arange(max_pos, dtype=np.float64)
    ang = np.outer(pos, inv_freq)
    ang = np.concatenate([ang, ang], axis=-1)
    scale = float(1 << ROPE_FRAC_BITS)
    cos_t = np.round(np.cos(ang) * scale).astype(np.int16)
    sin_t = np.round(np.sin(ang) * scale).astype(np.int16)
    return cos_t, sin_t


def apply_int_rope(x, cos_t, sin_t, positions):
    """ops/rope.py:38-55 — rshift_round(x*cos + rotate_half(x)*sin, 14)."""
    d = x.shape[-1]
    half = d // 2
    c = as64(cos_t[positions])
    s = as64(sin_t[positions])
    x64 = as64(x)
    x1 = x64[..., :half]
    x2 = x64[..., half:]
    rot = np.concatenate([-x2, x1], axis=-1)
    return rshift_round(x64 * c + rot * s, ROPE_FRAC_BITS)


def di_linear(x8, xm, xk, w8_t, wm, wk):
    """ops/di_matmul.py:22-31."""
    return int_gemm(x8, w8_t), xm, xk, wm, wk


def di_matmul(x, xm, xk, w8_t, wm, wk):
    """ops/di_matmul.py:34-40 — quantise, GEMM, requantise to int8."""
    x8, qm, qk = dy.quant_i8_pertoken(x, xm, xk)
    P, rm, rk, cm, ck = di_linear(x8, qm, qk, w8_t, wm, wk)
    return dy.requant_i8_rowcol(P, rm, rk, cm, ck)


__all__ = ["di_exp", "di_exp_tpos", "di_softmax", "di_rmsnorm", "di_rmsnorm_gamma",
           "di_swiglu", "build_rope_tables", "apply_int_rope", "di_linear",
           "di_matmul", "I32"]
