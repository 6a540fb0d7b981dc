"""Exact integer GEMMs, restated from ``src/detllm/backends.py``.

``int_gemm`` follows the "reference" branch (backends.py:88-96): the exact
int8 x int8 -> int32 product-sum. The oracle evaluates it with a float64
BLAS matmul, which is exact here: every partial sum is an integer of
magnitude <= K * 128 * 128 < 2^53 (asserted), so any summation order gives
the same integer. Pinned: naive-loop brute force (the reference's
tests/test_ops.py:52-61 restated) in tests/test_oracle_model.py.

``int_gemm_u8i8`` / ``int_gemm_u16i8`` follow backends.py:138-164; both are
exact identities, pinned against the plain int64 product (test_ops.py:63-78).
"""

from __future__ import annotations

import numpy as np

from .intmath import I32, I64

_EXACT = float(2 ** 53)
_EXACT32 = 1 << 24
# float32 represents every integer of magnitude <= 2^24 exactly; with int8
# operands (|a|,|b| <= 128) a K-chunk of 1024 keeps every partial sum within it.
F32_CHUNK = _EXACT32 // (128 * 128)


def _exact_matmul(a: np.ndarray, b: np.ndarray, bound_a: int, bound_b: int) -> np.ndarray:
    K = a.shape[-1]
    assert K * bound_a * bound_b < _EXACT, "float64 evaluation would not be exact"
    return np.rint(np.matmul(a.astype(np.float64), b.astype(np.float64))).astype(I64)


def exact_matmul_f32(a: np.ndarray, b32: np.ndarray) -> np.ndarray:
    """Exact int8 GEMM a [*, M, K] x b [K, N] with b pre-converted to float32.

    K is cut into chunks of F32_CHUNK; within a chunk every partial sum is an
    integer of magnitude <= 2^24, exact in float32 whatever the summation
    order; chunk results are summed in int64."""
    K = a.shape[-1]
    out = None
    for k0 in range(0, K, F32_CHUNK):
        part = np.matmul(a[..., k0:k0 + F32_CHUNK].astype(np.float32),
                         b32[k0:k0 + F32_CHUNK])
        part = np.rint(part).astype(I64)
        out = part if out is None else out + part
    return out


def int_gemm(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """a [*, M, K] int8 x b [*, K, N] int8 -> int32 (backends.py:88-96)."""
    assert a.dtype == np.int8 and b.dtype == np.int8, (a.dtype, b.dtype)
    assert a.shape[-1] == b.shape[-2]
    return _exact_matmul(a, b, 128, 128).astype(I32)


def int_gemm_u8i8(p_u8: np.ndarray, b: np.ndarray) -> np.ndarray:
    """backends.py:138-149 — (p-64)@b + 64*colsum(b) for p in [0, 128];
    int64, as the reference's int32 column sum promotes (torch sum of int32
    gives int64)."""
    shifted = (p_u8.astype(I64) - 64).astype(np.int8)
    core = int_gemm(shifted, b)
    corr = b.astype(I64).sum(axis=-2, keepdims=True) * 64
    return core.astype(I64) + corr


def int_gemm_u16i8(p_u16: np.ndarray, b: np.ndarray) -> np.ndarray:
    """backends.py:152-164 — 15-bit probabilities as an exact hi/lo split."""
    p = p_u16.astype(I64)
    hi = p >> 7
    lo = p - (hi << 7)
    hi_part = int_gemm_u8i8(hi, b).astype(I64)
    lo_part = int_gemm(lo.astype(np.int8), b).astype(I64)
    return (hi_part << 7) + lo_part


def matmul_i64(p: np.ndarray, v: np.ndarray) -> np.ndarray:
    """Exact int64 p @ v for |p| <= 2^14 (probabilities) and int8 v: the
    value every exact formulation of the attention context produces
    (model.py:363-381 broadcast path, backends.py:152-164 hi/lo path)."""
    return _exact_matmul(p, v, (1 << 14) + 1, 128)
