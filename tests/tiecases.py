"""Logit rows with real ties for greedy_pick (src/detllm/model.py:482-490:
argmax of logits * head_m in int64, lowest token id among the maxima).

``tie_cases()`` returns (rows int32 [R, V], head_m int64 [V]) with V = 5000,
so the rows span three 2048-id chunks of the device arg-max (the last one
partial). head_m[i] = 20000 + i % 97 repeats every 97 ids, so equal logits at
ids 97 apart tie exactly; other rows tie through crossed mantissas
(logits[a] = head_m[b] * t, logits[b] = head_m[a] * t). Rows:

  0  two-way tie inside chunk 0 (ids 5 and 1000)
  1  tie across the chunk boundary (ids 2047 and 2048)
  2  tie between the first chunk and the last, partial one (100 and 4999)
  3  three-way tie over three chunks (ids 2100, 2100 + 97 * 21, 2100 - 97 * 21)
  4  all-zero row: every product is 0, the pick is id 0
  5  a many-way tie over every chunk (ids 97 k, k >= 1, all = -20000)
  6  tie between two ids one lane visits in turn (4099, 4099 + 256)
  7  int32 extremes: INT32_MAX at ids 10 and 107 (same mantissa), INT32_MIN
     elsewhere in places
  8  a unique maximum at the highest id (no tie)
  9  tie between the highest id and a lower one in the same chunk (4902, 4999)
 10  tie between two lanes of one wave (4100, 4130)

``brute_pick`` is the definition itself in Python integers.
"""

from __future__ import annotations

import numpy as np

V = 5000


def _head_m() -> np.ndarray:
    return (20000 + np.arange(V, dtype=np.int64) % 97).astype(np.int64)


def tie_cases():
    hm = _head_m()
    rng = np.random.default_rng(2024)
    rows = []

    def base():
        # products of these stay below 2^14 * 2^15 < every planted maximum
        return rng.integers(-(1 << 14), 1 << 14, V).astype(np.int64)

    def cross(r, a, b, t=8):
        r[a] = hm[b] * t
        r[b] = hm[a] * t
        return r

    rows.append(cross(base(), 5, 1000))
    rows.append(cross(base(), 2047, 2048))
    rows.append(cross(base(), 100, 4999))
    r = base()
    ids3 = [2100, 2100 + 97 * 21, 2100 - 97 * 21]
    assert len({hm[i] for i in ids3}) == 1
    r[ids3] = 50000
    rows.append(r)
    rows.append(np.zeros(V, np.int64))
    r = np.full(V, -1, np.int64)
    r[:97] = -2
    rows.append(r)
    rows.append(cross(base(), 4099, 4099 + 256))
    r = base()
    r[::3] = -(1 << 31)
    r[[10, 107]] = (1 << 31) - 1
    rows.append(r)
    r = base()
    r[V - 1] = 70000
    rows.append(r)
    rows.append(cross(base(), 4902, 4999))
    rows.append(cross(base(), 4100, 4130))
    out = np.stack(rows).astype(np.int32)
    return out, hm


def brute_pick(rows: np.ndarray, head_m: np.ndarray) -> list[int]:
    picks = []
    hm = [int(x) for x in head_m]
    for row in rows:
        prods = [int(v) * h for v, h in zip(row.tolist(), hm)]
        mx = max(prods)
        picks.append(min(i for i, p in enumerate(prods) if p == mx))
    return picks


# the pick of each row, by construction (brute_pick must agree)
EXPECTED = [5, 2047, 100, 2100 - 97 * 21, 0, 97, 4099, 10, V - 1, 4902, 4100]
