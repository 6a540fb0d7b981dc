"""The C-ABI entry points as torch custom operators ("detllm_rocm::...").

The reference registers its device kernels as ``torch.library.custom_op`` with
a ``register_fake`` shape function (src/detllm/ops/int_prims.py:96-136), so
dynamo and inductor see each one as a single opaque node: its compiled layer
(model.py:434-467) and its graph capture through ``torch._dynamo.run``
(graphed.py:108) trace straight through them. The rocm backend's operators
follow the same pattern: each op below runs one extern "C" entry point of
libdetllm_hip.so on torch's current stream, and its fake implementation
returns integer tensors of the right shape, so ``NoFloatMode`` holds during
tracing too. The ops are registered for CUDA (HIP) tensors only: there is no
CPU kernel behind them.

Cache tensors use this backend's paged layout (kvcache.py: per-layer K pool
[n_pages, n_kv, 128, 128], V pool [n_pages, n_kv, 128, 128] holding V
transposed per page, a [B, width] int32 page table, a [B, width * 128] bool
validity mask).
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from ._lib import call

I64 = torch.int64
NS = "detllm_rocm"
GREEDY_CHUNK = 2048


def _op(name, mutates=()):
    return torch.library.custom_op(f"{NS}::{name}", mutates_args=mutates, device_types="cuda")


# ------------------------------------------------------------------ GEMM

@_op("int_gemm")
def int_gemm(a: Tensor, b: Tensor) -> Tensor:
    """backends.int_gemm(a, b, "rocm"): a [*, M, K] int8 x b [*, K, N] int8 ->
    int32 [*, M, N] (a 2-D b is shared by every leading index)."""
    from .backends import _int_gemm_impl
    return _int_gemm_impl(a, b)


@int_gemm.register_fake
def _(a, b):
    return a.new_empty(tuple(a.shape[:-1]) + (b.shape[-1],), dtype=torch.int32)


@_op("isqrt_i64")
def isqrt_i64(a: Tensor) -> Tensor:
    """int_prims.py:96-103 (detllm::isqrt_i64): floor sqrt of int64."""
    from .dyadic import isqrt
    return isqrt(a)


@isqrt_i64.register_fake
def _(a):
    return torch.empty_like(a, dtype=I64)


@_op("ilog2_i64")
def ilog2_i64(a: Tensor) -> Tensor:
    """int_prims.py:106-113 (detllm::ilog2_i64): floor log2 of int64."""
    from .dyadic import ilog2_floor
    return ilog2_floor(a)


@ilog2_i64.register_fake
def _(a):
    return torch.empty_like(a, dtype=I64)


@_op("greedy_pick")
def greedy_pick(logits: Tensor, head_m: Tensor) -> Tensor:
    """IntQwen3.greedy_pick (model.py:482-490): [R, V] int32 -> [R] int64."""
    R, V = logits.shape
    nch = -(-V // GREEDY_CHUNK)
    pv = torch.empty(R, nch, dtype=I64, device=logits.device)
    pi = torch.empty(R, nch, dtype=I64, device=logits.device)
    out = torch.empty(R, dtype=I64, device=logits.device)
    call("detllm_greedy_pick", logits.contiguous(), head_m.contiguous(), R, V, GREEDY_CHUNK, pv,
         pi, out)
    return out


@greedy_pick.register_fake
def _(logits, head_m):
    return logits.new_empty(logits.shape[0], dtype=I64)


# ------------------------------------------------------- fused row kernels

def _rows_out(R, C, dev):
    return (torch.empty(R, C, dtype=torch.int8, device=dev),
            torch.empty(R, dtype=I64, device=dev), torch.empty(R, dtype=I64, device=dev))


def _rows_fake(R, C, like):
    return (like.new_empty(R, C, dtype=torch.int8), like.new_empty(R, dtype=I64),
            like.new_empty(R, dtype=I64))


@_op("embed_normq", mutates=("err",))
def embed_normq(ids: Tensor, e8: Tensor, em: Tensor, ek: Tensor, sm_m: Optional[Tensor],
                sm_k: int, err: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Embedding + residual_from_delta + _norm_quant (model.py:246-249,
    :187-198): ids [R] -> (h int32 [R, H], k_res, x8 int8 [R, H], xm, xk)."""
    R, H = ids.numel(), e8.shape[1]
    dev = ids.device
    h = torch.empty(R, H, dtype=torch.int32, device=dev)
    k_res = torch.empty(R, dtype=I64, device=dev)
    x8, xm, xk = _rows_out(R, H, dev)
    call("detllm_embed_normq", ids.contiguous().view(-1), R, H, e8.shape[0], e8, em, ek, h, k_res,
         sm_m, sm_k, x8, xm, xk, err)
    return h, k_res, x8, xm, xk


@embed_normq.register_fake
def _(ids, e8, em, ek, sm_m, sm_k, err):
    R, H = ids.numel(), e8.shape[1]
    return (ids.new_empty(R, H, dtype=torch.int32), ids.new_empty(R, dtype=I64),
            *_rows_fake(R, H, ids))


@_op("norm_quant")
def norm_quant(h: Tensor, sm_m: Optional[Tensor], sm_k: int) -> tuple[Tensor, Tensor, Tensor]:
    """IntQwen3._norm_quant (model.py:187-198): h [R, C] int32 -> (x8, xm, xk)."""
    R, C = h.shape
    x8, xm, xk = _rows_out(R, C, h.device)
    call("detllm_norm_quant", h.contiguous(), R, C, sm_m, sm_k, x8, xm, xk)
    return x8, xm, xk


@norm_quant.register_fake
def _(h, sm_m, sm_k):
    return _rows_fake(h.shape[0], h.shape[1], h)


@_op("residual_normq", mutates=("h", "k_res"))
def residual_normq(P: Tensor, row_m: Tensor, row_k: Tensor, col_m: Tensor, col_k: int, tb: int,
                   h: Tensor, k_res: Tensor, sm_m: Optional[Tensor],
                   sm_k: int) -> tuple[Tensor, Tensor, Tensor]:
    """requant_i32_common(tb) + residual_add + _norm_quant (model.py:410-415,
    :424-427): P int32 [nsplit, R, C] partials; h [R, C], k_res [R] updated
    in place; returns the next GEMM's (x8, xm, xk)."""
    ns, R, C = P.shape
    x8, xm, xk = _rows_out(R, C, P.device)
    call("detllm_residual_normq", P.contiguous(), ns, R * C, R, C, row_m, row_k, col_m, col_k, tb,
         h, k_res, sm_m, sm_k, x8, xm, xk, None, 0, 0, 0, 0)
    return x8, xm, xk


@residual_normq.register_fake
def _(P, row_m, row_k, col_m, col_k, tb, h, k_res, sm_m, sm_k):
    return _rows_fake(P.shape[1], P.shape[2], P)


@_op("swiglu_quant")
def swiglu_quant(P: Tensor, xm: Tensor, xk: Tensor, gate_m: Tensor, gate_k: int, up_m: Tensor,
                 up_k: int, ds_m: Tensor, ds_k: int) -> tuple[Tensor, Tensor, Tensor]:
    """gate/up requant_i32_common(14) + di_swiglu + quant_i8_pertoken
    (model.py:416-423): P int32 [nsplit, R, 2I] -> (y8 [R, I], ym, yk)."""
    ns, R, C2 = P.shape
    y8, ym, yk = _rows_out(R, C2 // 2, P.device)
    call("detllm_swiglu_quant", P.contiguous(), ns, R * C2, R, C2 // 2, xm, xk, gate_m, gate_k,
         up_m, up_k, ds_m, ds_k, y8, ym, yk, None, 0, 0, 0, 0)
    return y8, ym, yk


@swiglu_quant.register_fake
def _(P, xm, xk, gate_m, gate_k, up_m, up_k, ds_m, ds_k):
    return _rows_fake(P.shape[1], P.shape[2] // 2, P)


@_op("merge_rowcol")
def merge_rowcol(attn: Tensor, os_m: Tensor, os_k: int, col_m: Tensor,
                 col_k: int) -> tuple[Tensor, Tensor, Tensor]:
    """requant_i8_rowcol(attn * os_m, 1, os_k, col_m, col_k) (model.py:404-409):
    attn int64 [R, C] -> (a8, am, ak)."""
    R, C = attn.shape
    a8, am, ak = _rows_out(R, C, attn.device)
    call("detllm_merge_rowcol", attn.contiguous(), 1, 0, R, C, os_m, os_k, col_m, col_k, a8, am,
         ak, None, 0, 0, 0, 0)
    return a8, am, ak


@merge_rowcol.register_fake
def _(attn, os_m, os_k, col_m, col_k):
    return _rows_fake(attn.shape[0], attn.shape[1], attn)


# ------------------------------------------------------------- attention

@_op("qkv_epilogue", mutates=("kpool", "vpool", "err"))
def qkv_epilogue(P: Tensor, B: int, T: int, n_q: int, n_kv: int, xm: Tensor, xk: Tensor,
                 positions: Tensor, q_m: Tensor, q_k: int, k_m: Tensor, k_k: int, v_m: Tensor,
                 v_k: int, q_norm_m: Tensor, q_norm_k: int, k_norm_m: Tensor, k_norm_k: int,
                 qs_m: Tensor, qs_k: int, kq_m: Tensor, kq_k: Tensor, ks_m: Tensor, ks_k: Tensor,
                 vq_m: Tensor, vq_k: Tensor, cos_t: Tensor, sin_t: Tensor, kpool: Tensor,
                 vpool: Tensor, table: Tensor, slot_base: int,
                 err: Tensor) -> tuple[Tensor, Tensor]:
    """_qk_head_pipeline + QK smoothing + Q quant + K/V static requant into
    the cache + score scale / DI-Exp constant (model.py:200-216, :303-358).
    P int32 [nsplit, B*T, (n_q + 2 n_kv) * 128]; returns (q8 [B, n_q, T, 128],
    tpos [B, n_q, T])."""
    ns, R, _ = P.shape
    q8 = torch.empty(B, n_q, T, 128, dtype=torch.int8, device=P.device)
    tpos = torch.empty(B, n_q, T, dtype=I64, device=P.device)
    call("detllm_qkv_epilogue", P.contiguous(), ns, R * P.shape[2], B, T, n_q, n_kv, xm, xk,
         positions.contiguous().view(-1), q_m, q_k, k_m, k_k, v_m, v_k, q_norm_m, q_norm_k,
         k_norm_m, k_norm_k, qs_m, qs_k, kq_m, kq_k, ks_m, ks_k, vq_m, vq_k, cos_t, sin_t,
         cos_t.shape[0], q8, tpos, None, kpool, vpool, table, table.shape[1], None, slot_base,
         None, err)
    return q8, tpos


@qkv_epilogue.register_fake
def _(P, B, T, n_q, n_kv, *rest):
    return P.new_empty(B, n_q, T, 128, dtype=torch.int8), P.new_empty(B, n_q, T, dtype=I64)


@_op("attn_prefill")
def attn_prefill(q8: Tensor, tpos: Tensor, kpool: Tensor, vpool: Tensor, table: Tensor,
                 valid: Tensor, S_past: int) -> Tensor:
    """Prefill attention (model.py:382-402): q8 [B, n_q, T, 128] over the
    cache's first S_past + T slots (causal by slot, valid-masked) -> exact
    int64 context [B, T, n_q * 128]."""
    B, n_q, T, _ = q8.shape
    n_kv = kpool.shape[1]
    out = torch.empty(B, T, n_q * 128, dtype=I64, device=q8.device)
    call("detllm_attn_prefill", q8.contiguous(), tpos.contiguous(), kpool, vpool, table,
         table.shape[1], valid.view(torch.uint8), valid.shape[1], B, T, S_past, n_q, n_kv, out)
    return out


@attn_prefill.register_fake
def _(q8, tpos, kpool, vpool, table, valid, S_past):
    B, n_q, T, _ = q8.shape
    return q8.new_empty(B, T, n_q * 128, dtype=I64)


@_op("attn_decode", mutates=("err",))
def attn_decode(q8: Tensor, tpos: Tensor, kpool: Tensor, vpool: Tensor, table: Tensor,
                valid: Tensor, S: int, err: Tensor) -> Tensor:
    """Decode attention (model.py:347-381, ops/fused_attn.py:47-142): one
    query per row, q8 [B, n_q, 128], over S slots -> int64 [B, n_q * 128]."""
    B, n_q = q8.shape[0], q8.shape[1]
    n_kv = kpool.shape[1]
    G = n_q // n_kv
    Spad = (S + 15) // 16 * 16
    scratch = (torch.empty(B, n_q, Spad, dtype=torch.int32, device=q8.device)
               if G * Spad * 4 > 48 * 1024 else None)
    out = torch.empty(B, n_q * 128, dtype=I64, device=q8.device)
    call("detllm_attn_decode", q8.contiguous(), tpos.contiguous(), kpool, vpool, table,
         table.shape[1], valid.view(torch.uint8), valid.shape[1], B, S, n_q, n_kv, None, scratch,
         out, err)
    return out


@attn_decode.register_fake
def _(q8, tpos, kpool, vpool, table, valid, S, err):
    return q8.new_empty(q8.shape[0], q8.shape[1] * 128, dtype=I64)


OPS = ("int_gemm", "isqrt_i64", "ilog2_i64", "greedy_pick", "embed_normq", "norm_quant",
       "residual_normq", "swiglu_quant", "merge_rowcol", "qkv_epilogue", "attn_prefill",
       "attn_decode")
