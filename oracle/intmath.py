"""Integer primitives with the reference's exact semantics (numpy int64).

Follows ``src/detllm/intmath.py`` and the CPU loops of
``src/detllm/ops/int_prims.py``. Semantics reproduced from torch's CPU
integer kernels (which the reference runs on):
  * add / sub / mul wrap modulo 2^64 (numpy arrays wrap the same way);
  * ``a << k`` is computed on the unsigned value; k >= 64 (or k < 0) gives 0;
  * ``a >> k`` is arithmetic; k >= 63 (or k < 0) gives the sign fill;
  * floor division rounds toward -inf;
  * int64 -> int32 casts truncate modulo 2^32.
numpy's own ``left_shift``/``right_shift``/``floor_divide`` already behave this
way (probed against torch); the helpers below clamp shift amounts explicitly
so the rule is visible in the code rather than inherited.

Pinned: closed forms and brute force in tests/test_oracle_intmath.py
(Python ``//``, ``math.isqrt``, ``int.bit_length``, and the KATs of the
reference's tests/test_intmath.py:21-197 restated as values).
"""

from __future__ import annotations

import numpy as np

I64 = np.int64
I32 = np.int32
I8 = np.int8


def as64(a) -> np.ndarray:
    return np.asarray(a).astype(I64, copy=False)


def shl(a, k) -> np.ndarray:
    """torch.bitwise_left_shift on int64 (intmath.py:103-117)."""
    a, k = np.broadcast_arrays(as64(a), as64(k))
    bad = (k < 0) | (k >= 64)
    kk = np.where(bad, 0, k).astype(np.uint64)
    out = (a.astype(np.uint64) << kk).astype(I64)
    return np.where(bad, I64(0), out).astype(I64)


def shr(a, k) -> np.ndarray:
    """torch.bitwise_right_shift on int64 (intmath.py:83-100): arithmetic."""
    a = as64(a)
    k = as64(k)
    kk = np.where((k < 0) | (k >= 63), 63, k)
    return np.right_shift(a, kk).astype(I64)


def floor_div(a, b):
    """intmath.py:49-59 — Python floor division (b != 0)."""
    if isinstance(a, (int, np.integer)) and isinstance(b, (int, np.integer)):
        return int(a) // int(b)
    return np.floor_divide(as64(a), as64(b)).astype(I64)


def round_half_away_div(a, b):
    """intmath.py:62-80 — sign(a) * floor((|a| + floor(b/2)) / b), b > 0.

    Tensor branch: sign = where(a<0,-1,1); mag = |a| (wraps at INT64_MIN);
    half = floor_div(b, 2); result = sign * floor_div(mag + half, b)."""
    if isinstance(a, (int, np.integer)) and isinstance(b, (int, np.integer)):
        a, b = int(a), int(b)
        if b <= 0:
            raise ValueError("b must be > 0")
        sign = -1 if a < 0 else 1
        return sign * ((abs(a) + b // 2) // b)
    a = as64(a)
    b = as64(b)
    sign = np.where(a < 0, I64(-1), I64(1))
    mag = np.abs(a)
    half = np.floor_divide(b, 2)
    return (sign * np.floor_divide(mag + half, b)).astype(I64)


rhad = round_half_away_div


def ashr(a, k: int):
    """intmath.py:83-93 (python-int shift amount)."""
    if isinstance(a, (int, np.integer)):
        return int(a) >> k
    return shr(a, k)


def rshift_round(a, k: int):
    """intmath.py:120-131 — (a + 2^(k-1)) >> k; k == 0 is the identity."""
    if k == 0:
        return a
    if isinstance(a, (int, np.integer)):
        return (int(a) + (1 << (k - 1))) >> k
    return shr(as64(a) + I64(1 << (k - 1)), k)


def rshift_round_t(a, k):
    """intmath.py:134-147 — per-element shift amounts; k == 0 entries unchanged.

    half = 1 << (max(k,1)-1) with torch's lshift clamp; rounded =
    (a + half) >> max(k,1) with torch's rshift clamp."""
    a = as64(a)
    k = np.broadcast_to(as64(k), a.shape)
    kpos = np.maximum(k, 1)
    half = shl(np.ones_like(a), kpos - 1)
    rounded = shr(a + half, kpos)
    return np.where(k == 0, a, rounded).astype(I64)


def clamp_i8(a) -> np.ndarray:
    """intmath.py:150-153."""
    return np.clip(as64(a), -128, 127).astype(I8)


def to_i32(a) -> np.ndarray:
    """torch ``.to(torch.int32)`` on int64: truncation modulo 2^32."""
    return as64(a).astype(I32)


def ilog2(a):
    """intmath.py:164-177 via int_prims.py:47-55 (_ilog2_loop).

    The tensor loop returns floor(log2 a) for a >= 1 and 0 for a <= 1
    (no hit fires for a < 2, including negative values)."""
    if isinstance(a, (int, np.integer)):
        a = int(a)
        if a < 1:
            raise ValueError("ilog2_floor requires a >= 1")
        return a.bit_length() - 1
    v = as64(a).copy()
    r = np.zeros_like(v)
    for s in (32, 16, 8, 4, 2, 1):
        hit = v >= (1 << s)
        r = r + hit.astype(I64) * s
        v = np.right_shift(v, hit.astype(I64) * s)
    return r


def isqrt(a):
    """intmath.py:180-202 via int_prims.py:31-44 (_isqrt_loop): 32 steps of
    the bitwise method from d = 2^62; negative inputs give 0."""
    if isinstance(a, (int, np.integer)):
        a = int(a)
        if a < 0:
            raise ValueError("isqrt requires a >= 0")
        x, c, d = a, 0, 1 << 62
        while d > a:
            d >>= 2
        while d != 0:
            if x >= c + d:
                x -= c + d
                c = (c >> 1) + d
            else:
                c >>= 1
            d >>= 2
        return c
    n = as64(a)
    rem = n.copy()
    c = np.zeros_like(n)
    d = 1 << 62
    for _ in range(32):
        t = c + I64(d)
        ge = rem >= t
        rem = np.where(ge, rem - t, rem)
        c = np.right_shift(c, 1) + np.where(ge, I64(d), I64(0))
        d >>= 2
    return c
