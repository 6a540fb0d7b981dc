"""Pin the oracle's integer primitives against closed forms and brute force.

Values restated from the reference's KATs (tests/test_intmath.py:21-197) and
checked against Python's own integer semantics, ``math.isqrt`` and
``int.bit_length`` — never against the oracle's own formula."""

import math

import numpy as np
import pytest

from oracle import intmath as im

I64 = np.int64


def a64(*v):
    return np.array(v, dtype=I64)


def test_floor_div_python_semantics():
    a = np.arange(-100, 100, dtype=I64)
    for b in (1, 2, 3, 7, 128):
        assert im.floor_div(a, b).tolist() == [x // b for x in range(-100, 100)]
    assert im.floor_div(-7, 2) == -4 and im.floor_div(-8, 2) == -4 and im.floor_div(-1, 4) == -1


def test_rhad_ties_away_from_zero():
    assert im.rhad(3, 2) == 2 and im.rhad(-3, 2) == -2
    assert im.rhad(5, 2) == 3 and im.rhad(-5, 2) == -3
    assert im.rhad(5, 4) == 1 and im.rhad(-5, 4) == -1 and im.rhad(7, 4) == 2
    with pytest.raises(ValueError):
        im.rhad(5, 0)


def test_rhad_tensor_matches_exact_rational_rounding():
    from fractions import Fraction
    a = np.arange(-1000, 1000, dtype=I64)
    for b in (1, 2, 3, 8, 100, 127):
        got = im.rhad(a, np.full_like(a, b)).tolist()
        want = []
        for x in range(-1000, 1000):
            q = Fraction(abs(x), b)
            r = math.floor(q + Fraction(1, 2))
            want.append(-r if x < 0 else r)
        assert got == want


def test_shifts_torch_clamping():
    a = a64(-5, 5, -(1 << 62), 1 << 62)
    assert im.shr(a, 1).tolist() == [-3, 2, -(1 << 61), 1 << 61]
    for k in (63, 64, 100, -1):
        assert im.shr(a, k).tolist() == [-1, 0, -1, 0]
    assert im.shl(a, 1).tolist() == [-10, 10, -(1 << 63), -(1 << 63)]
    for k in (64, 65, -1):
        assert im.shl(a, k).tolist() == [0, 0, 0, 0]
    # wrap modulo 2^64
    assert im.shl(a64(3), 63).tolist() == [-(1 << 63)]


def test_rshift_round_formula():
    assert im.rshift_round(3, 1) == 2 and im.rshift_round(-3, 1) == -1
    assert im.rshift_round(5, 2) == 1 and im.rshift_round(6, 2) == 2
    assert im.rshift_round(-6, 2) == -1 and im.rshift_round(7, 0) == 7
    a = np.arange(-1000, 1000, dtype=I64)
    for k in (1, 2, 7, 15):
        assert im.rshift_round(a, k).tolist() == [(x + (1 << (k - 1))) >> k
                                                  for x in range(-1000, 1000)]


def test_rshift_round_t_per_element():
    a = a64(-1000, -6, -3, 0, 3, 6, 1000)
    k = a64(3, 2, 1, 0, 1, 2, 3)
    want = [x if s == 0 else (x + (1 << (s - 1))) >> s for x, s in zip(a.tolist(), k.tolist())]
    assert im.rshift_round_t(a, k).tolist() == want


def test_clamp_i8():
    got = im.clamp_i8(a64(-1000, -129, -128, -1, 0, 126, 127, 128, 1000))
    assert got.dtype == np.int8
    assert got.tolist() == [-128, -128, -128, -1, 0, 126, 127, 127, 127]


def test_ilog2_exhaustive_small_and_large():
    a = np.arange(1, 1 << 16, dtype=I64)
    assert im.ilog2(a).tolist() == [x.bit_length() - 1 for x in range(1, 1 << 16)]
    vals = [1, (1 << 30) - 1, 1 << 30, (1 << 31) - 1, 1 << 40, (1 << 62) + 123, (1 << 63) - 1]
    assert im.ilog2(a64(*vals)).tolist() == [v.bit_length() - 1 for v in vals]
    # the reference's tensor loop yields 0 below 1 (no hit fires)
    assert im.ilog2(a64(0, -5)).tolist() == [0, 0]
    with pytest.raises(ValueError):
        im.ilog2(0)


def test_isqrt_against_math():
    n = np.arange(0, 70000, dtype=I64)
    assert im.isqrt(n).tolist() == [math.isqrt(x) for x in range(70000)]
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.integers(0, 1 << 62, 20000, dtype=I64),
                        a64(0, 1, 2, 3, 4, (1 << 31) - 1, 1 << 31, (1 << 52) + 7,
                            (1 << 62) - 1, (1 << 63) - 1)])
    assert im.isqrt(v).tolist() == [math.isqrt(int(x)) for x in v]
    r = np.arange(0, 100000, 977, dtype=I64)
    assert (im.isqrt(r * r) == r).all()
    assert im.isqrt(a64(-1, -(1 << 40))).tolist() == [0, 0]
    for x in (0, 1, 2, 3, (1 << 62) - 1):
        assert im.isqrt(x) == math.isqrt(x)


def test_to_i32_truncates():
    assert im.to_i32(a64((1 << 40) + (1 << 31) + 5)).tolist() == [-2147483643]
