"""Device (rocm) versions of the reference's integer primitives and dyadic
requantisations, one HIP kernel each.

Signatures and broadcasting follow ``src/detllm/intmath.py`` and
``src/detllm/dyadic.py``; arguments are integer tensors on the GPU (python
ints where the reference accepts them). Per-row operands are broadcast to the
data's leading shape and per-column operands to its last dimension; the HIP
kernels then work on contiguous 2-D views. Results are bit-identical to the
reference CPU path (tests/test_gpu_ops.py).
"""

from __future__ import annotations

import torch

from ._lib import call

I64 = torch.int64


def _dev(x, like: torch.Tensor) -> torch.Tensor:
    if isinstance(x, torch.Tensor):
        return x.to(device=like.device, dtype=I64)
    return torch.tensor(int(x), dtype=I64, device=like.device)


def _rows(v, lead: tuple, like) -> torch.Tensor:
    """Broadcast a per-row operand ([..., 1] or scalar) to a contiguous [R]."""
    t = _dev(v, like)
    if t.dim() > 0 and t.shape[-1] == 1 and t.dim() == len(lead) + 1:
        t = t[..., 0]
    return t.broadcast_to(lead).contiguous().view(-1)


def _scalar(v) -> int:
    if isinstance(v, torch.Tensor):
        assert v.numel() == 1, "expected a scalar"
        return int(v.item())
    return int(v)


# ---------------------------------------------------------------- intmath

_SCALAR_OPS = {"isqrt": 0, "ilog2": 1, "norm_scale": 2, "fit": 3, "srd": 4}


def _scalar_op(op, a, b=None, c=None, two_out=False):
    shape = torch.broadcast_shapes(*[t.shape for t in (a, b, c) if t is not None])
    a = a.to(I64).broadcast_to(shape).contiguous()
    b = b.to(I64).broadcast_to(shape).contiguous() if b is not None else None
    c = c.to(I64).broadcast_to(shape).contiguous() if c is not None else None
    o1 = torch.empty(shape, dtype=I64, device=a.device)
    o2 = torch.empty(shape, dtype=I64, device=a.device) if two_out else None
    call("detllm_op_scalar", _SCALAR_OPS[op], a, b, c, a.numel(), o1, o2)
    return (o1, o2) if two_out else o1


def isqrt(a: torch.Tensor) -> torch.Tensor:
    """intmath.py:180-202 (int_prims.py:31-44 loop semantics)."""
    return _scalar_op("isqrt", a)


def ilog2_floor(a: torch.Tensor) -> torch.Tensor:
    """intmath.py:164-177 (int_prims.py:47-55 loop semantics)."""
    return _scalar_op("ilog2", a)


# ---------------------------------------------------------------- dyadic

def scaled_round_div(num, den, e):
    """dyadic.py:45-49."""
    num = _dev(num, num if isinstance(num, torch.Tensor) else den)
    return _scalar_op("srd", num, _dev(den, num), _dev(e, num))


def fit_dyadic_ratio(num: torch.Tensor, den, bits: int = 16):
    """dyadic.py:52-72 (bits = 16 only)."""
    if bits != 16:
        raise NotImplementedError("the rocm kernels implement bits=16 (the model's width)")
    return _scalar_op("fit", num.to(I64), _dev(den, num), two_out=True)


def norm_scale(m: torch.Tensor, k: torch.Tensor, bits: int = 16):
    """dyadic.py:75-90 (bits = 16 only)."""
    if bits != 16:
        raise NotImplementedError("the rocm kernels implement bits=16 (the model's width)")
    return _scalar_op("norm_scale", m.to(I64), _dev(k, m), two_out=True)


def quant_i8_pertoken(x: torch.Tensor, m, k):
    """dyadic.py:93-105: returns (x8 int8, m_out [..., 1], k_out [..., 1])."""
    lead, C = tuple(x.shape[:-1]), x.shape[-1]
    x2 = x.to(I64).contiguous().view(-1, C)
    R = x2.shape[0]
    x8 = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    mo = torch.empty(lead + (1,), dtype=I64, device=x.device)
    ko = torch.empty(lead + (1,), dtype=I64, device=x.device)
    call("detllm_op_quant_i8_pertoken", x2, _rows(m, lead, x), _rows(k, lead, x), R, C, x8, mo, ko)
    return x8, mo, ko


def requant_i32_common(P: torch.Tensor, row_m, row_k, col_m, col_k, target_bits: int = 12):
    """dyadic.py:108-120. col_m broadcasts against P's trailing dims."""
    lead, C = tuple(P.shape[:-1]), P.shape[-1]
    P2 = P.to(I64).contiguous().view(-1, C)
    R = P2.shape[0]
    cm = _dev(col_m, P)
    G = 1
    if cm.dim() >= 2:
        # per-(trailing group, column) scales, e.g. [n_heads, hd] against [B, T, n_heads, hd]
        G = int(torch.tensor(cm.shape[:-1]).prod().item())
        cm = cm.broadcast_to(cm.shape).contiguous().view(G, C)
        assert R % G == 0
    cm = cm.broadcast_to((G, C)).contiguous()
    y = torch.empty(P.shape, dtype=torch.int32, device=P.device)
    ko = torch.empty(lead + (1,), dtype=I64, device=P.device)
    call("detllm_op_requant_i32_common", P2, _rows(row_k, lead, P), cm, G, _scalar(col_k),
         target_bits, R, C, y, ko)
    return y, _rows(row_m, lead, P).view(lead + (1,)), ko


def requant_i8_rowcol(P: torch.Tensor, row_m, row_k, col_m, col_k):
    """dyadic.py:123-139."""
    lead, C = tuple(P.shape[:-1]), P.shape[-1]
    P2 = P.to(I64).contiguous().view(-1, C)
    R = P2.shape[0]
    y8 = torch.empty(P.shape, dtype=torch.int8, device=P.device)
    mo = torch.empty(lead + (1,), dtype=I64, device=P.device)
    ko = torch.empty(lead + (1,), dtype=I64, device=P.device)
    cm = _dev(col_m, P).broadcast_to((C,)).contiguous()
    call("detllm_op_requant_i8_rowcol", P2, _rows(row_m, lead, P), _rows(row_k, lead, P), cm,
         _scalar(col_k), R, C, y8, mo, ko)
    return y8, mo, ko


def requant_i8_static(P: torch.Tensor, row_m, row_k, col_m, col_k, s_m, s_k):
    """dyadic.py:142-163 (every operand broadcast to P's shape)."""
    shape = P.shape
    ops = [P, row_m, row_k, col_m, col_k, s_m, s_k]
    full = [_dev(v, P).broadcast_to(shape).contiguous() for v in ops]
    y8 = torch.empty(shape, dtype=torch.int8, device=P.device)
    call("detllm_op_requant_i8_static", *full, P.numel(), y8)
    return y8


def _residual(mode, h, k_res, d=None, dm=None, dk=None):
    lead, C = tuple(h.shape[:-1]), h.shape[-1]
    h2 = h.to(I64).contiguous().view(-1, C)
    R = h2.shape[0]
    out = torch.empty(h.shape, dtype=torch.int32, device=h.device)
    ko = torch.empty(lead + (1,), dtype=I64, device=h.device)
    d2 = d.to(I64).contiguous().view(-1, C) if d is not None else None
    call("detllm_op_residual", mode, h2, _rows(k_res, lead, h), d2,
         _rows(dm, lead, h) if dm is not None else None,
         _rows(dk, lead, h) if dk is not None else None, R, C, out, ko)
    return out, ko


def residual_renorm(h64: torch.Tensor, k_res):
    """dyadic.py:174-184."""
    return _residual(0, h64, k_res)


def residual_from_delta(d: torch.Tensor, dm, dk):
    """dyadic.py:187-190 == residual_add onto a zero row at k_res = dk."""
    zero = torch.zeros(d.shape, dtype=I64, device=d.device)
    return _residual(1, zero, dk, d, dm, dk)


def residual_add(h: torch.Tensor, k_res, d: torch.Tensor, dm, dk):
    """dyadic.py:193-206."""
    return _residual(1, h, k_res, d, dm, dk)
