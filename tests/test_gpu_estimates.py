"""The fp64-estimate helpers of csrc/intops.h, run on the device one element
at a time (detllm_op_scalar ops 8-15) against exact Python integers at the
edges of the operand bounds their callers check.

Each helper returns an integer as the truncation of a biased fp64 (or fp32)
estimate; the host build is tested in test_intops_host.py. These cases pin
the device arithmetic itself (v_fma_f64, v_div_* and v_sqrt_f64 as the
compiler emits them for gfx950): quotients next to every rounding boundary,
operands just inside each stated bound, and the int8 saturation edges."""

import math
import random

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
I64 = torch.int64


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from idempotent_llm_amd import _lib
    _lib.load()


def run(op, a, b=None, c=None):
    from idempotent_llm_amd._lib import call
    n = len(a)
    t = lambda v: torch.tensor(v, dtype=I64, device="cuda") if v is not None else None
    o1 = torch.empty(n, dtype=I64, device="cuda")
    o2 = torch.empty(n, dtype=I64, device="cuda")
    call("detllm_op_scalar", op, t(a), t(b), t(c), n, o1, o2)
    return o1.cpu().tolist()


def rhad(a, d):
    q = (abs(a) + d // 2) // d
    return -q if a < 0 else q


def clamp8(x):
    return max(-128, min(127, x))


def dexp(n, t):
    """ops/di_exp.py:27-37 for x = -n <= 0 with constant tpos t."""
    q, rem = divmod(n, t)
    return (t - ((rem + 1) >> 1)) >> min(q, 62)


def _boundary_operands(rng, d, s, m_max, count):
    """m with m s + floor(d/2) next to a multiple of d (the truncation edges)."""
    out = []
    for _ in range(count):
        k = rng.randrange(0, max(1, (m_max * s) // d) + 1)
        base = (k * d - d // 2) // s
        for dm in (-1, 0, 1):
            m = base + dm
            if 0 <= m <= m_max:
                out.append(m)
    return out


def test_rhad_est_and_signed_forms():
    """op 8 rhad(m s, d) and op 9 its signed form, for 2 m s + d < 2^51 and
    quotients below 2^32 (int8 quantisation s = 127, RMSNorm s = 2^20,
    attention probabilities s = 2^14, the merge s = 1)."""
    rng = random.Random(5)
    A, B, C = [], [], []
    for s in (1, 127, 1 << 14, 1 << 20):
        for e in list(range(0, 50, 3)) + [49, 50]:
            d = max(1, (1 << e) + rng.randrange(-3, 4))
            if d >= 1 << 51:
                continue
            # 2 m s + d < 2^51 and a quotient (m s + floor(d/2)) // d below 2^32
            m_max = min(((1 << 51) - d - 1) // (2 * s), ((1 << 32) * d - d // 2 - 1) // s)
            if m_max < 0:
                continue
            ms = _boundary_operands(rng, d, s, m_max, 6) + [0, m_max, rng.randrange(m_max + 1)]
            for m in ms:
                A.append(m); B.append(d); C.append(s)
    want = [rhad(a * c, b) for a, b, c in zip(A, B, C)]
    assert run(8, A, B, C) == want
    # the signed form returns int32: quotients below 2^31, both signs
    keep = [i for i, w in enumerate(want) if w < 1 << 31]
    A9 = [v for i in keep for v in (A[i], -A[i])]
    B9 = [B[i] for i in keep for _ in (0, 1)]
    C9 = [C[i] for i in keep for _ in (0, 1)]
    want = [rhad(a * c if a >= 0 else -(-a * c), b) for a, b, c in zip(A9, B9, C9)]
    assert run(9, A9, B9, C9) == want


def test_rhad_est_i8_saturation_edges():
    """op 10 clamp_i8(rhad(n, d)) for 2 |n| + d < 2^51: quotients 126..129,
    254..256 and far beyond, both signs."""
    rng = random.Random(6)
    A, B = [], []
    for e in (0, 1, 5, 17, 30, 40, 44, 45):
        d = (1 << e) + rng.randrange(0, 3)
        for q in (0, 1, 126, 127, 128, 129, 254, 255, 256, 1000):
            for r in (-(d // 2) - 1, -(d // 2), 0, (d - 1) // 2, (d + 1) // 2 - 1, d // 2):
                n = q * d + r
                if n < 0 or 2 * n + d >= 1 << 51:
                    continue
                A += [n, -n]
                B += [d, d]
    want = [clamp8(rhad(n, d)) for n, d in zip(A, B)]
    assert run(10, A, B) == want


def test_rhad_est_corr_signed_near_2p53():
    """op 11 sign(a) rhad(|a| s, d) with the remainder step: s |a| + d up to
    just below 2^53, quotients below 2^31 (the merge's 46-bit rows), and
    |a| <= d < 2^53 at s = 127 (the fp64 row quantiser's large rows)."""
    rng = random.Random(7)
    A, B, C = [], [], []
    for s in (1, 127):
        for e in (20, 22, 30, 40):
            d = (1 << e) + rng.randrange(1, 1000)
            a_max = min(((1 << 53) - d - 1) // s, ((1 << 31) - 2) * d // s)
            for a in _boundary_operands(rng, d, s, a_max, 8) + [a_max, a_max - 1]:
                for sg in (1, -1):
                    A.append(sg * a); B.append(d); C.append(s)
    # the fp64 row quantiser's large rows: s = 127, |a| <= d < 2^53
    for e in (43, 46, 50, 52):
        d = (1 << e) + rng.randrange(1, 1 << 20)
        for a in _boundary_operands(rng, d, 127, d, 8) + [d, d - 1]:
            for sg in (1, -1):
                A.append(sg * a); B.append(d); C.append(127)
    for d in ((1 << 53) - 1, (1 << 53) - 3):
        for a in (d, d - 1, d // 2, d // 127):
            for sg in (1, -1):
                A.append(sg * a); B.append(d); C.append(127)
    want = [rhad(a * c if a >= 0 else -((-a) * c), b) for a, b, c in zip(A, B, C)]
    assert run(11, A, B, C) == want


def test_dexp_est_bounds():
    """op 12 DI-Exp of -n for 0 <= n < 2^22 and 1 <= t < 2^23, including
    n = 2^22 - 1, t = 2^23 - 1, multiples of t and their neighbours."""
    rng = random.Random(8)
    A, B = [], []
    for t in (1, 2, 3, 127, 4096, 65535, (1 << 22) - 1, 1 << 22, (1 << 23) - 1):
        ns = {0, 1, (1 << 22) - 1, (1 << 22) - 2}
        for k in range(0, 40):
            for dn in (-1, 0, 1):
                ns.add(k * t + dn)
        ns |= {rng.randrange(1 << 22) for _ in range(30)}
        for n in sorted(ns):
            if 0 <= n < 1 << 22:
                A.append(n); B.append(t)
    assert run(12, A, B) == [dexp(n, t) for n, t in zip(A, B)]


def test_dexp_est_sp_bounds():
    """op 13 the same DI-Exp taken from sp = t - n (the attention's score
    offset form), |sp| < 2^23."""
    rng = random.Random(9)
    A, B = [], []
    for t in (1, 5, 1000, (1 << 22) + 3, (1 << 23) - 1):
        for n in {0, 1, t - 1, t, t + 1, 2 * t, (1 << 22) - 1} | {rng.randrange(1 << 22)
                                                                  for _ in range(20)}:
            sp = t - n
            if 0 <= n < 1 << 22 and abs(sp) < 1 << 23:
                A.append(sp); B.append(t)
    assert run(13, A, B) == [dexp(t - sp, t) for sp, t in zip(A, B)]


def test_di_exp_tpos_fast_vs_integer_form():
    """op 14 the DI-Exp constant max(rhad(2^k, m_f), 1), m_f = m + (m >> 1)
    - (m >> 4) (model.py:355-358), over normalised mantissas and k in
    [0, 46] (the estimate) and past it (the integer path)."""
    rng = random.Random(10)
    A, B = [], []
    for k in list(range(0, 48)) + [50, 60, 62]:
        for m in (1 << 15, (1 << 16) - 1, 43690, 21846, rng.randrange(1 << 15, 1 << 16), 1, 7):
            A.append(m); B.append(k)
    want = []
    for m, k in zip(A, B):
        mf = m + (m >> 1) - (m >> 4)
        want.append(max(rhad(1 << k, mf if mf else 1), 1))
    assert run(14, A, B) == want


def test_isqrt_est_near_squares():
    """op 15 floor(sqrt(n)) for 0 <= n < 2^62 at r^2 - 1, r^2, r^2 + 1."""
    rng = random.Random(11)
    A = [0, 1, 2, 3, (1 << 62) - 1, (1 << 62) - 2]
    for r in [1, 2, 3, (1 << 31) - 1, (1 << 26) + 1, 3037000499 // 2] + \
            [rng.randrange(1, 1 << 31) for _ in range(60)]:
        for dn in (-1, 0, 1):
            n = r * r + dn
            if 0 <= n < 1 << 62:
                A.append(n)
    assert run(15, A) == [math.isqrt(n) for n in A]
