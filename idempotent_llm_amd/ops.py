"""Device (rocm) versions of the reference's integer operators
(``src/detllm/ops/``), one HIP kernel each; bit-identical to the CPU path.
"""

from __future__ import annotations

import torch

from ._lib import call, raise_for_error_word
from .dyadic import _dev, _rows

I64 = torch.int64
P_OUT_BITS = 15       # ops/di_softmax.py:29
OUT_FRAC_BITS = 20    # ops/di_rmsnorm.py:29
ROPE_FRAC_BITS = 14   # ops/rope.py:22
SIG_BITS = 8          # ops/di_swiglu.py:35


def di_exp(x: torch.Tensor, m, k):
    """ops/di_exp.py:21-37: returns (result int64, tpos [..., 1])."""
    lead, C = tuple(x.shape[:-1]), x.shape[-1]
    x2 = x.to(I64).contiguous().view(-1, C)
    R = x2.shape[0]
    res = torch.empty(x.shape, dtype=I64, device=x.device)
    tpos = torch.empty(lead + (1,), dtype=I64, device=x.device)
    call("detllm_op_di_exp", x2, _rows(m, lead, x), _rows(k, lead, x), R, C, res, tpos)
    return res, tpos


def di_softmax(scores: torch.Tensor, m, k, valid: torch.Tensor, clip_c: int | None = None,
               p_out_bits: int = P_OUT_BITS):
    """ops/di_softmax.py:33-61: probabilities int32 in [0, 2^(p_out_bits-1)]."""
    lead, C = tuple(scores.shape[:-1]), scores.shape[-1]
    x2 = scores.to(I64).contiguous().view(-1, C)
    R = x2.shape[0]
    v = valid.to(device=scores.device, dtype=torch.bool).broadcast_to(scores.shape)
    v = v.contiguous().view(torch.uint8).view(-1, C)
    probs = torch.empty(scores.shape, dtype=torch.int32, device=scores.device)
    call("detllm_op_softmax", x2, _rows(m, lead, scores), _rows(k, lead, scores), v,
         0 if clip_c is None else 1, 0 if clip_c is None else int(clip_c), p_out_bits, R, C,
         probs)
    return probs


def _rmsnorm(x: torch.Tensor, gamma_m=None):
    C = x.shape[-1]
    x2 = x.to(I64).contiguous().view(-1, C)
    R = x2.shape[0]
    if gamma_m is None:
        y = torch.empty(x.shape, dtype=torch.int32, device=x.device)
        call("detllm_op_rmsnorm", x2, None, R, C, y, None)
    else:
        y = torch.empty(x.shape, dtype=I64, device=x.device)
        g = _dev(gamma_m, x).broadcast_to((C,)).contiguous()
        call("detllm_op_rmsnorm", x2, g, R, C, None, y)
    return y


def di_rmsnorm(x: torch.Tensor) -> torch.Tensor:
    """ops/di_rmsnorm.py:33-52: int32 at fixed scale (1, 20)."""
    return _rmsnorm(x)


def di_rmsnorm_gamma(x: torch.Tensor, gamma_m: torch.Tensor, gamma_k: int):
    """ops/di_rmsnorm.py:55-64: ((x/rms) * gamma_m int64, 20 + gamma_k)."""
    return _rmsnorm(x, gamma_m), OUT_FRAC_BITS + gamma_k


def di_swiglu(gate: torch.Tensor, gm, gk, up: torch.Tensor, um, uk):
    """ops/di_swiglu.py:39-58: (y int64, gm*um, gk + uk + 7)."""
    lead, C = tuple(gate.shape[:-1]), gate.shape[-1]
    g2 = gate.to(I64).contiguous().view(-1, C)
    u2 = up.to(I64).contiguous().view(-1, C)
    R = g2.shape[0]
    y = torch.empty(gate.shape, dtype=I64, device=gate.device)
    ym = torch.empty(lead + (1,), dtype=I64, device=gate.device)
    yk = torch.empty(lead + (1,), dtype=I64, device=gate.device)
    call("detllm_op_swiglu", g2, _rows(gm, lead, gate), _rows(gk, lead, gate), u2,
         _rows(um, lead, gate), _rows(uk, lead, gate), R, C, y, ym, yk)
    return y, ym, yk


def apply_int_rope(x: torch.Tensor, cos_t: torch.Tensor, sin_t: torch.Tensor,
                   positions: torch.Tensor) -> torch.Tensor:
    """ops/rope.py:38-55 for head_dim 128: int64, same shape as x."""
    d = x.shape[-1]
    if d != 128:
        raise NotImplementedError("the rocm RoPE kernel is specialised to head_dim 128")
    x2 = x.to(I64).contiguous().view(-1, d)
    rows = x2.shape[0]
    pos = positions.to(device=x.device, dtype=I64).broadcast_to(x.shape[:-1]).contiguous()
    y = torch.empty(x.shape, dtype=I64, device=x.device)
    err = torch.zeros(1, dtype=torch.int32, device=x.device)
    call("detllm_op_rope", x2, pos, cos_t.contiguous(), sin_t.contiguous(), cos_t.shape[0],
         rows, y, err)
    if not torch.cuda.is_current_stream_capturing():
        raise_for_error_word(err.item(), max_pos=cos_t.shape[0])   # as cos_t[positions] raises
    return y


def di_linear(x8: torch.Tensor, xm, xk, w8_t: torch.Tensor, wm, wk, backend: str = "rocm"):
    """ops/di_matmul.py:22-31: exact int8 GEMM (x8 [..., T, K] against
    w8_t [K, N], shared over the leading dims: the reference expands it, a
    2-D operand folds into the rows here, same integers), scales passed
    through."""
    from .backends import _require_rocm, canonical_backend, int_gemm
    _require_rocm(canonical_backend(backend))
    return int_gemm(x8, w8_t, "rocm"), xm, xk, wm, wk


def di_matmul(x: torch.Tensor, xm, xk, w8_t: torch.Tensor, wm, wk, backend: str = "rocm"):
    """ops/di_matmul.py:34-40: quantise per token, GEMM, requantise to int8."""
    from .backends import _require_rocm, canonical_backend
    from .dyadic import quant_i8_pertoken, requant_i8_rowcol
    _require_rocm(canonical_backend(backend))
    x8, qm, qk = quant_i8_pertoken(x, xm, xk)
    P, rm, rk, cm, ck = di_linear(x8, qm, qk, w8_t, wm, wk)
    return requant_i8_rowcol(P, rm, rk, cm, ck)


__all__ = ["di_exp", "di_softmax", "di_rmsnorm", "di_rmsnorm_gamma", "di_swiglu",
           "apply_int_rope", "di_linear", "di_matmul"]
