"""The GEMM dispatch boundary with the third backend, "rocm".

Mirrors ``src/detllm/backends.py``: the same names (``BACKENDS``,
``BACKEND_ALIASES``, ``canonical_backend``, ``int_gemm``, ``int_gemm_u8i8``,
``int_gemm_u16i8``), argument meaning and error behaviour (ValueError for an
unknown backend, AssertionError for non-int8 operands or a K mismatch). This
package implements only "rocm"; "reference" and "cuda" are recognised names
whose implementations live in the reference, so asking this package to run
them raises instead of silently substituting another path.

"rocm": exact int8 x int8 -> int32 on gfx950 i8 MFMA through
``detllm_igemm_nt`` / ``detllm_igemv_nt`` (K zero-padded to a multiple of 16 —
zeros are exact in an integer product; b transposed on the device to the
kernels' [N, K] layout).
"""

from __future__ import annotations

import torch

from . import torch_ops  # noqa: F401  (registers the detllm_rocm:: operators)
from ._lib import call

BACKENDS = ("reference", "cuda", "rocm")
BACKEND_ALIASES = {"cpu": "reference", "hip": "rocm"}


def canonical_backend(name: str) -> str:
    """backends.py:28-34 plus the "rocm" backend (alias "hip")."""
    canon = BACKEND_ALIASES.get(name, name)
    if canon not in BACKENDS:
        raise ValueError(f"unknown backend {name!r}; expected one of "
                         f"{BACKENDS + tuple(BACKEND_ALIASES)}")
    return canon


def _require_rocm(backend: str):
    if backend != "rocm":
        if backend in BACKENDS:
            raise ValueError(f"backend {backend!r} is served by detllm itself; this package "
                             "implements the 'rocm' backend")
        raise ValueError(f"unknown backend {backend!r}")


def _pad_k(x: torch.Tensor, Kp: int) -> torch.Tensor:
    K = x.shape[-1]
    if K == Kp:
        return x.contiguous()
    out = torch.zeros(*x.shape[:-1], Kp, dtype=x.dtype, device=x.device)
    out[..., :K] = x
    return out


def transpose_i8(b: torch.Tensor) -> torch.Tensor:
    """[*, R, C] int8 -> [*, C, R] on the device (HIP transpose kernel)."""
    R, C = b.shape[-2], b.shape[-1]
    src = b.contiguous().view(-1, R, C)
    batch = src.shape[0]
    dst = torch.empty(batch, C, R, dtype=torch.int8, device=b.device)
    call("detllm_transpose_i8", src, dst, R, C, batch, R * C, R * C)
    return dst.view(*b.shape[:-2], C, R)


def gemm_nt(a: torch.Tensor, bt: torch.Tensor, out: torch.Tensor | None = None,
            ksplit: int = 1) -> torch.Tensor:
    """C = a . bt^T for a [M, K], bt [N, K] (K % 16 == 0) -> int32 [ksplit, M, N]
    partial products (ksplit > 1 only on the skinny path; their integer sum
    is the product)."""
    M, K = a.shape
    N = bt.shape[0]
    if M <= 64:
        if out is None:
            out = torch.empty(ksplit, M, N, dtype=torch.int32, device=a.device)
        call("detllm_igemv_nt", a, bt, out, M, N, K, ksplit, M * N)
    else:
        assert ksplit == 1
        if out is None:
            out = torch.empty(1, M, N, dtype=torch.int32, device=a.device)
        call("detllm_igemm_nt", a, bt, out, M, N, K, 1, 0, 0, 0)
    return out


def int_gemm(a: torch.Tensor, b: torch.Tensor, backend: str = "rocm") -> torch.Tensor:
    """Exact integer GEMM: a [*, M, K] int8 x b [*, K, N] int8 -> int32
    (backends.py:88-135). Batched dims must match; a 2-D b is shared. Runs
    as the custom operator detllm_rocm::int_gemm, so torch.compile and
    graph capture see one opaque node (as int_prims.py:96-136 does for the
    reference's kernels)."""
    assert a.dtype == torch.int8 and b.dtype == torch.int8, (a.dtype, b.dtype)
    assert a.shape[-1] == b.shape[-2]
    _require_rocm(backend)
    if b.dim() != 2 or a.dim() == 2:
        assert a.shape[:-2] == b.shape[:-2], (a.shape, b.shape)
    return torch.ops.detllm_rocm.int_gemm(a, b)


def _int_gemm_impl(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """The kernel behind detllm_rocm::int_gemm (operands checked by int_gemm)."""
    if b.dim() == 2 and a.dim() > 2:
        lead = a.shape[:-1]
        out = _int_gemm_impl(a.reshape(-1, a.shape[-1]), b)
        return out.reshape(*lead, b.shape[-1])
    M, K, N = a.shape[-2], a.shape[-1], b.shape[-1]
    if M == 0 or N == 0:
        return torch.zeros(*a.shape[:-1], N, dtype=torch.int32, device=a.device)
    Kp = max(16, (K + 15) // 16 * 16)
    bt = _pad_k(transpose_i8(b), Kp)
    ap = _pad_k(a, Kp)
    if a.dim() == 2:
        return gemm_nt(ap, bt)[0]
    A = ap.reshape(-1, M, Kp)
    Bt = bt.reshape(-1, N, Kp)
    batch = A.shape[0]
    out = torch.empty(batch, M, N, dtype=torch.int32, device=a.device)
    call("detllm_igemm_nt", A, Bt, out, M, N, Kp, batch, M * Kp, N * Kp, M * N)
    return out.reshape(*a.shape[:-2], M, N)


def int_gemm_u8i8(p_u8: torch.Tensor, b: torch.Tensor, backend: str = "rocm") -> torch.Tensor:
    """backends.py:138-149: (p-64)@b + 64*colsum(b) for p in [0, 128].
    int64, as in the reference, where the int32 column sum promotes."""
    shifted = (p_u8 - 64).to(torch.int8)
    core = int_gemm(shifted, b, backend)
    corr = b.to(torch.int64).sum(dim=-2, keepdim=True) * 64
    return core + corr


def int_gemm_u16i8(p_u16: torch.Tensor, b: torch.Tensor, backend: str = "rocm") -> torch.Tensor:
    """backends.py:152-164: 15-bit probabilities as an exact hi/lo split -> int64."""
    hi = p_u16 >> 7
    lo = p_u16 - (hi << 7)
    hi_part = int_gemm_u8i8(hi, b, backend).to(torch.int64)
    lo_part = int_gemm(lo.to(torch.int8), b, backend).to(torch.int64)
    return (hi_part << 7) + lo_part
