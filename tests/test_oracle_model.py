"""Pin the oracle's IntQwen3 restatement and GEMMs.

* GEMMs: naive loops / plain int64 products (the reference's
  tests/test_ops.py:52-78 restated).
* Model: tokens, logits and demo chain hashes written by the reference's own
  IntQwen3(backend="reference") on seeded random-init artifacts
  (tests/golden/model_*.json), including batch invariance with right-padded
  co-prompts and the split-prefill path.
"""

import json
import os

import numpy as np
import pytest

from idempotent_llm_amd import artifact as art
from idempotent_llm_amd.hashchain import chain_hashes, token_chain
from oracle import gemm
from oracle.model import IntQwen3Oracle

HERE = os.path.dirname(os.path.abspath(__file__))
I64 = np.int64


def test_int_gemm_matches_naive_loop():
    rng = np.random.default_rng(0)
    a = rng.integers(-128, 128, (7, 33)).astype(np.int8)
    b = rng.integers(-128, 128, (33, 5)).astype(np.int8)
    got = gemm.int_gemm(a, b)
    assert got.dtype == np.int32
    for i in range(7):
        for j in range(5):
            assert int(got[i, j]) == sum(int(a[i, k]) * int(b[k, j]) for k in range(33))


def test_exact_f32_chunked_gemm_worst_case():
    # all -128 operands: every partial sum reaches the f32 exactness limit
    a = np.full((3, 3072), -128, np.int8)
    b = np.full((3072, 4), -128, np.int8)
    got = gemm.exact_matmul_f32(a, b.astype(np.float32))
    assert (got == 3072 * 128 * 128).all()
    rng = np.random.default_rng(1)
    a = rng.integers(-128, 128, (5, 2048)).astype(np.int8)
    b = rng.integers(-128, 128, (2048, 9)).astype(np.int8)
    want = a.astype(I64) @ b.astype(I64)
    assert np.array_equal(gemm.exact_matmul_f32(a, b.astype(np.float32)), want)


def test_u8_and_u16_tricks_exact():
    rng = np.random.default_rng(7)
    p = rng.integers(0, 129, (9, 21)).astype(np.int32)
    v = rng.integers(-128, 128, (21, 6)).astype(np.int8)
    got = gemm.int_gemm_u8i8(p, v)
    assert got.dtype == I64   # backends.py:148-149: the int32 colsum promotes
    assert np.array_equal(got, p.astype(I64) @ v.astype(I64))
    p = rng.integers(0, (1 << 14) + 1, (9, 300)).astype(np.int32)
    v = rng.integers(-128, 128, (300, 6)).astype(np.int8)
    got = gemm.int_gemm_u16i8(p, v)
    assert got.dtype == I64
    assert np.array_equal(got, p.astype(I64) @ v.astype(I64))


def _load(name):
    with open(os.path.join(HERE, "golden", f"model_{name}.json")) as f:
        return json.load(f)


@pytest.fixture(scope="module", params=["tiny", "mid"])
def case(request, tmp_path_factory):
    rec = _load(request.param)
    d = str(tmp_path_factory.mktemp(request.param))
    art.make_artifact(d, rec["dims"], rec["seed"])
    assert art.artifact_digest(d) == rec["artifact_sha256"], "artifact generator drifted"
    return rec, IntQwen3Oracle(d)


def test_prefill_logits(case):
    rec, m = case
    ids = np.array(rec["prompt"], dtype=I64)[None]
    pos = np.arange(ids.shape[1], dtype=I64)[None]
    logits, xm, xk, _ = m.forward(ids, pos)
    assert logits.dtype == np.int32
    assert chain_hashes(logits[0]) == rec["prefill_chain"]
    assert logits[0, -1].tolist() == rec["prefill_last_row"]
    assert xm[0, :, 0].tolist() == rec["prefill_xm"] and xk[0, :, 0].tolist() == rec["prefill_xk"]


def test_generate_b1(case):
    rec, m = case
    ids = np.array(rec["prompt"], dtype=I64)[None]
    toks, steps = m.generate(ids, len(rec["b1_tokens"]))
    assert toks[0].tolist() == rec["b1_tokens"]
    assert chain_hashes([s[0] for s in steps]) == rec["b1_logit_chain"]
    assert token_chain(toks[0]) == rec["b1_token_chain"]


def test_generate_padded_batch(case):
    rec, m = case
    ids = np.array(rec["batch_ids"], dtype=I64)
    valid = np.array(rec["batch_valid"], dtype=bool)
    toks, steps = m.generate(ids, len(rec["b1_tokens"]), chunk_valid=valid)
    assert toks.tolist() == rec["batch_tokens"]
    for b in range(ids.shape[0]):
        assert chain_hashes([s[b] for s in steps]) == rec["batch_row_chains"][b]
    assert rec["batch_row_chains"][0] == rec["b1_logit_chain"]   # batch invariance


def test_head_rows_select_the_full_logits_rows(case):
    """forward(head_rows=r) computes the LM head at position r[b] of each row
    only: the same rows (and row scales) as the full [B, T, vocab] logits
    against the reference-written padded-batch goldens."""
    rec, m = case
    ids = np.array(rec["batch_ids"], dtype=I64)
    valid = np.array(rec["batch_valid"], dtype=bool)
    B, T = ids.shape
    pos = np.broadcast_to(np.arange(T, dtype=I64), (B, T))
    full, fxm, fxk, _ = m.forward(ids, pos, None, valid)
    last = np.maximum(valid.sum(axis=1) - 1, 0)
    sel, sxm, sxk, _ = m.forward(ids, pos, None, valid, head_rows=last)
    rows = np.arange(B)
    assert sel.shape == (B, full.shape[-1])
    assert np.array_equal(sel, full[rows, last])
    assert np.array_equal(sxm, fxm[rows, last]) and np.array_equal(sxk, fxk[rows, last])
    for b in range(B):    # the first step of the reference's padded-batch chains
        assert chain_hashes([sel[b]])[0] == rec["batch_row_chains"][b][0]


def test_split_prefill(case):
    rec, m = case
    ids = np.array(rec["prompt"], dtype=I64)
    T = len(ids)
    half = T // 2
    pos = np.arange(T, dtype=I64)[None]
    full, _, _, _ = m.forward(ids[None], pos)
    _, _, _, cache = m.forward(ids[None, :half], pos[:, :half])
    rows = []
    for t in range(half, T):
        lg, _, _, cache = m.forward(ids[None, t:t + 1], np.array([[t]], I64), cache)
        rows.append(lg[0, 0])
    assert chain_hashes(rows) == rec["split_tail_chain"]
    assert chain_hashes(rows) == chain_hashes(full[0, half:])   # prefill/decode invariance


def test_greedy_pick_ties(case):
    rec, m = case
    rows = np.array(rec["tie_rows"], dtype=np.int32)
    assert m.greedy_pick(rows).tolist() == rec["tie_picks"]


def _ns_pick(head_m):
    """The oracle's greedy_pick bound to a given head_m (model.py:482-490)."""
    from types import SimpleNamespace
    return lambda rows: IntQwen3Oracle.greedy_pick(
        SimpleNamespace(head_m=head_m, vocab=head_m.shape[0]), rows)


def test_greedy_pick_real_ties_vs_brute_force():
    """Rows with real ties (inside a 2048-id chunk, across chunk boundaries,
    many-way, all-zero, int32 extremes): the oracle's pick equals the lowest
    id among the maxima computed in Python integers."""
    from tiecases import EXPECTED, brute_pick, tie_cases
    rows, hm = tie_cases()
    prods = rows.astype(object) * hm.astype(object)
    n_max = [(p == p.max()).sum() for p in prods]
    assert sum(n > 1 for n in n_max) == len(EXPECTED) - 1   # every row but one ties
    assert brute_pick(rows, hm) == EXPECTED
    assert _ns_pick(hm)(rows).tolist() == EXPECTED


def test_tie_rows_reject_a_flipped_tie_rule():
    """A planted mistake in the oracle (highest id among the maxima, or the
    first maximum of the last 2048-id chunk) fails on these rows."""
    from tiecases import EXPECTED, tie_cases
    rows, hm = tie_cases()
    scaled = rows.astype(I64) * hm

    def highest(s):
        mx = s.max(axis=-1, keepdims=True)
        return np.where(s == mx, np.arange(s.shape[1]), -1).max(axis=-1).tolist()

    def chunk_last_wins(s, chunk=2048):
        out = []
        for row in s:
            best_v, best_i = None, None
            for c0 in range(0, row.shape[0], chunk):
                seg = row[c0:c0 + chunk]
                i = int(np.argmax(seg)) + c0
                if best_v is None or row[i] >= best_v:   # ">=": later chunk wins ties
                    best_v, best_i = row[i], i
            out.append(best_i)
        return out

    assert highest(scaled) != EXPECTED
    assert chunk_last_wins(scaled) != EXPECTED
