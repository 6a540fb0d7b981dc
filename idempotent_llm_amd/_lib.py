"""ctypes binding of libdetllm_hip.so (the extern "C" boundary).

Every entry point takes device pointers, sizes and a hipStream_t and returns
0 on success, a positive hipError_t for a failed launch or a negative errno
for bad arguments; ``call`` raises ``RuntimeError`` on any nonzero return.
There is no fallback: when the library is missing, every compute call fails
loudly.
"""

from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdetllm_hip.so")

P, I, L, S = "p", "i", "l", "s"

# name -> argument kinds (p: device pointer / None, i: int32, l: int64, s: stream)
SIGNATURES = {
    "detllm_igemm_nt": [P, P, P, I, I, I, I, L, L, L, S],
    "detllm_igemv_nt": [P, P, P, I, I, I, I, L, S],
    "detllm_igemv_nt_pf": [P, P, P, I, I, I, I, L, P, L, P, L, P, L, P, L, S],
    "detllm_igemv_plan": [I, I, I, P],
    "detllm_attn_split_plan": [I, I, I, I, P, P],
    "detllm_transpose_i8": [P, P, I, I, I, L, L, S],
    "detllm_greedy_pick": [P, P, I, I, I, P, P, P, S],
    "detllm_greedy_pick_noalloc": [P, P, I, I, P, S],
    "detllm_logits_digest": [P, I, I, P, S],
    "detllm_embed_normq": [P, I, I, L, P, P, P, P, P, P, L, P, P, P, P, S],
    "detllm_residual_normq": [P, I, L, I, I, P, P, P, L, I, P, P, P, L, P, P, P, P, I, I, I, I, S],
    "detllm_norm_quant": [P, I, I, P, L, P, P, P, S],
    "detllm_attn_decode_split": [P, P, P, P, P, I, P, L, I, I, I, I, P, I, P, P, P, P, S],
    "detllm_igemv_resnormq": [P, P, I, I, I, I, L, P, I, L, P, P, P, L, I, P, P, P, P, P, L, P,
                              P, P, L, P, L, S],
    "detllm_igemv_merge": [P, P, I, I, I, I, L, P, I, L, P, L, P, L, P, P, P, L, P, L, S],
    "detllm_igemv_merge_ext": [P, P, I, I, I, I, L, P, P, L, L, P, I, P, P, I, P, L, P, L, S],
    "detllm_swiglu_quant": [P, I, L, I, I, P, P, P, L, P, L, P, L, P, P, P, P, I, I, I, I, S],
    "detllm_igemv_swiglu": [P, P, I, I, I, L, P, I, L, P, P, P, L, P, L, P, L, P, P, I, P, L, P,
                            L, S],
    "detllm_merge_rowcol": [P, I, L, I, I, P, L, P, L, P, P, P, P, I, I, I, I, S],
    "detllm_merge_ext": [P, I, I, P, L, L, P, I, P, P, P, P, I, I, I, I, S],
    "detllm_qkv_epilogue": [P, I, L, I, I, I, I, P, P, P, P, L, P, L, P, L, P, L, P, L, P, L,
                            P, P, P, P, P, P, P, P, L, P, P, P, P, P, P, I, P, L, P, P, S],
    "detllm_kq_est": [P, P, L, L, P, S],
    "detllm_requant_static_cols": [P, I, L, I, I, P, P, P, L, L, L, P, S],
    "detllm_igemv_requant_static": [P, P, I, I, I, P, P, P, L, L, L, P, S],
    "detllm_attn_prefill": [P, P, P, P, P, I, P, L, I, I, I, I, I, P, S],
    "detllm_attn_decode": [P, P, P, P, P, I, P, L, I, I, I, I, P, P, P, P, S],
    "detllm_qkv_attn_decode": [P, I, L, I, I, I, P, P, P, P, L, P, L, P, L, P, L, P, L, P, L,
                               P, P, P, P, P, P, P, P, L, P, P, P, I, P, L, P, L, I, P, P, P, P, S],
    "detllm_qkv_attn_decode_ext": [P, I, L, I, I, I, P, P, P, P, L, P, L, P, L, P, L, P, L, P,
                                   L, P, P, P, P, P, P, P, P, L, P, P, P, I, P, L, P, L, I, P,
                                   P, P, P, P, P, S],
    "detllm_decode_prologue": [P, L, I, L, P, P, P, P, L, S],
    "detllm_op_quant_i8_pertoken": [P, P, P, I, I, P, P, P, S],
    "detllm_op_requant_i32_common": [P, P, P, I, L, I, I, I, P, P, S],
    "detllm_op_requant_i8_rowcol": [P, P, P, P, L, I, I, P, P, P, S],
    "detllm_op_requant_i8_static": [P, P, P, P, P, P, P, L, P, S],
    "detllm_op_residual": [I, P, P, P, P, P, I, I, P, P, S],
    "detllm_op_rmsnorm": [P, P, I, I, P, P, S],
    "detllm_op_softmax": [P, P, P, P, I, L, I, I, I, P, S],
    "detllm_op_di_exp": [P, P, P, I, I, P, P, S],
    "detllm_op_swiglu": [P, P, P, P, P, P, I, I, P, P, P, S],
    "detllm_op_rope": [P, P, P, P, L, L, P, P, S],
    "detllm_op_scalar": [I, P, P, P, L, P, P, S],
}

# host-only entry points (no device work, so no stream argument)
HOST_ONLY = frozenset({"detllm_igemv_plan", "detllm_attn_split_plan"})

_CT = {P: ctypes.c_void_p, I: ctypes.c_int, L: ctypes.c_int64, S: ctypes.c_void_p}

_lib = None


class LibraryMissing(RuntimeError):
    pass


def load():
    """Load the HIP library (raises LibraryMissing when it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryMissing(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(the rocm backend has no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, kinds in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = [_CT[k] for k in kinds]
        fn.restype = ctypes.c_int
    _lib = lib
    return lib


def _arg(kind, v):
    if kind == P:
        if v is None:
            return None
        if isinstance(v, torch.Tensor):
            return v.data_ptr()
        return int(v)
    if kind == S:
        return v
    return int(v)


def stream_handle(stream=None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def gemv_plan(M: int, N: int, K: int) -> int:
    """K split the skinny-GEMM kernel is tuned for at [M, K] x [N, K]^T."""
    lib = load()
    out = ctypes.c_int(0)
    rc = lib.detllm_igemv_plan(int(M), int(N), int(K), ctypes.byref(out))
    if rc != 0:
        raise RuntimeError(f"detllm_igemv_plan failed (code {rc})")
    return out.value


def attn_split_plan(B: int, S: int, n_q: int, n_kv: int):
    """(chunk, nsplit) of the split-S decode attention at this shape."""
    lib = load()
    ch, ns = ctypes.c_int(0), ctypes.c_int(0)
    rc = lib.detllm_attn_split_plan(int(B), int(S), int(n_q), int(n_kv), ctypes.byref(ch),
                                    ctypes.byref(ns))
    if rc != 0:
        raise RuntimeError(f"detllm_attn_split_plan failed (code {rc})")
    return ch.value, ns.value


def pro_fits(K: int, ksplit: int) -> bool:
    """True when the fused decode GEMVs (detllm_igemv_resnormq /
    detllm_igemv_merge / detllm_igemv_swiglu) cover a K split of ``ksplit``: each split a whole
    number of 512-byte chunks, at most two (the check those entry points make
    before returning -38)."""
    if K <= 0 or K % 16 or ksplit < 1:
        return False
    kchunk = -(-K // ksplit)
    kchunk = -(-kchunk // 64) * 64
    if -(-K // kchunk) != ksplit or kchunk % 512:
        return False
    return kchunk // 512 <= 2


# bits of the device error word (include/detllm_hip.h)
ERR_TOKEN, ERR_POSITION, ERR_SLOTS = 1, 2, 4


def raise_for_error_word(word: int, vocab=None, max_pos=None) -> None:
    """Raise what the reference raises for the indices a kernel flagged:
    IndexError for a token id or position outside the table (embed_e8[ids],
    cos_t[positions] in src/detllm/model.py, ops/rope.py:48-49)."""
    word = int(word)
    if not word:
        return
    msgs = []
    if word & ERR_TOKEN:
        msgs.append(f"token id out of range for the embedding table (size {vocab})")
    if word & ERR_POSITION:
        msgs.append(f"position out of range for the RoPE tables (size {max_pos})")
    if word & ERR_SLOTS:
        msgs.append("device slot count exceeded the slots the attention launch was sized for")
    raise IndexError("; ".join(msgs))


def call(name: str, *args, stream=None) -> None:
    """Invoke an entry point; tensors are passed by device pointer and the
    current torch stream is appended as the hipStream_t argument."""
    lib = load()
    kinds = SIGNATURES[name]
    if len(args) != len(kinds) - 1:
        raise TypeError(f"{name}: expected {len(kinds) - 1} arguments, got {len(args)}")
    cargs = [_arg(k, v) for k, v in zip(kinds[:-1], args)]
    cargs.append(stream_handle(stream))
    rc = getattr(lib, name)(*cargs)
    if rc != 0:
        raise RuntimeError(f"{name} failed (code {rc})")
