"""GPU parity of the full IntQwen3 rocm runtime: logits, tokens and the demo
chain hashes must equal those the reference's CPU backend wrote
(tests/golden/model_*.json) — eager, graph-captured, right-padded batches,
split prefill, greedy ties — plus the determinism invariances of the
reference's tests/test_determinism.py, all exact."""

import json
import os

import numpy as np
import pytest
import torch

from idempotent_llm_amd import artifact as art
from idempotent_llm_amd.hashchain import chain_hashes, token_chain

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
I64 = torch.int64


def _load(name):
    with open(os.path.join(HERE, "golden", f"model_{name}.json")) as f:
        return json.load(f)


@pytest.fixture(scope="module", params=["tiny", "mid"])
def case(request, tmp_path_factory):
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from idempotent_llm_amd.model import IntQwen3
    rec = _load(request.param)
    d = str(tmp_path_factory.mktemp(request.param))
    art.make_artifact(d, rec["dims"], rec["seed"])
    assert art.artifact_digest(d) == rec["artifact_sha256"], "artifact generator drifted"
    print(f"[model case {request.param}]", flush=True)
    return rec, IntQwen3(d, backend="rocm"), d


def _ids(rec):
    return torch.tensor(rec["prompt"], dtype=I64, device="cuda")


def test_prefill_logits_and_guard(case):
    rec, m, _ = case
    ids = _ids(rec)[None]
    pos = torch.arange(ids.shape[1], device="cuda")[None]
    logits, xm, xk, _ = m.forward(ids, pos, guard=True)
    assert logits.dtype == torch.int32
    assert chain_hashes(logits[0]) == rec["prefill_chain"]
    assert logits[0, -1].tolist() == rec["prefill_last_row"]
    assert xm[0, :, 0].tolist() == rec["prefill_xm"]
    assert xk[0, :, 0].tolist() == rec["prefill_xk"]


def test_generate_b1_eager(case):
    rec, m, _ = case
    toks, steps = m.generate(_ids(rec)[None], len(rec["b1_tokens"]))
    assert toks[0].tolist() == rec["b1_tokens"]
    assert chain_hashes([s[0] for s in steps]) == rec["b1_logit_chain"]
    assert token_chain(toks[0]) == rec["b1_token_chain"]


def test_generate_b1_graphed(case):
    rec, m, _ = case
    toks, steps = m.generate(_ids(rec)[None], len(rec["b1_tokens"]), use_graph=True)
    assert toks[0].tolist() == rec["b1_tokens"]
    assert chain_hashes([s[0] for s in steps]) == rec["b1_logit_chain"]


@pytest.mark.parametrize("use_graph", [False, True])
def test_padded_batch(case, use_graph):
    rec, m, _ = case
    ids = torch.tensor(rec["batch_ids"], dtype=I64, device="cuda")
    valid = torch.tensor(rec["batch_valid"], dtype=torch.bool, device="cuda")
    toks, steps = m.generate(ids, len(rec["b1_tokens"]), chunk_valid=valid, use_graph=use_graph)
    assert toks.tolist() == rec["batch_tokens"]
    for b in range(ids.shape[0]):
        assert chain_hashes([s[b] for s in steps]) == rec["batch_row_chains"][b]


def test_split_prefill(case):
    rec, m, _ = case
    ids = _ids(rec)
    T = ids.shape[0]
    half = T // 2
    pos = torch.arange(T, device="cuda")[None]
    full, _, _, _ = m.forward(ids[None], pos)
    _, _, _, cache = m.forward(ids[None, :half], pos[:, :half])
    rows = []
    for t in range(half, T):
        lg, _, _, cache = m.forward(ids[None, t:t + 1], torch.tensor([[t]], device="cuda"), cache)
        rows.append(lg[0, 0])
    assert chain_hashes(rows) == rec["split_tail_chain"]
    for t in range(half, T):
        assert torch.equal(rows[t - half], full[0, t])


def test_greedy_pick_ties(case):
    rec, m, _ = case
    rows = torch.tensor(rec["tie_rows"], dtype=torch.int32, device="cuda")
    assert m.greedy_pick(rows).tolist() == rec["tie_picks"]


def test_run_to_run(case):
    rec, m, _ = case
    base_t, base_l = m.generate(_ids(rec)[None], 8, use_graph=True)
    for _ in range(3):
        t, lg = m.generate(_ids(rec)[None], 8, use_graph=True)
        assert torch.equal(t, base_t)
        for a, b in zip(lg, base_l):
            assert torch.equal(a, b)


def test_graph_growth_matches_oracle(case):
    """Prompt in bucket 256, decode past 256 slots: the graph is re-captured
    after the cache grows; every step equals the oracle (graphed.py:76-93)."""
    rec, m, d = case
    if rec["dims"]["hidden"] != 256:
        pytest.skip("tiny model only (oracle speed)")
    from oracle.model import IntQwen3Oracle
    steps = 250
    ids = _ids(rec)[None]
    tg, lg = m.generate(ids, steps, use_graph=True)
    te, le = IntQwen3Oracle(d).generate(ids.cpu().numpy(), steps)
    assert tg.cpu().numpy().tolist() == te.tolist()
    assert chain_hashes(lg) == chain_hashes(le)


def test_split_attention_decode_matches_oracle(case, monkeypatch):
    """Decode through the split-S attention (threshold lowered so that rows
    past 256 slots split into 256-slot chunks; the merge sums the partials):
    eager and graphed generation equal the oracle for 250 steps, and a batch
    of 3 gives the same logits split and unsplit."""
    rec, m, d = case
    if rec["dims"]["hidden"] != 256:
        pytest.skip("tiny model only (oracle speed)")
    import idempotent_llm_amd.model as mdl
    from oracle.model import IntQwen3Oracle
    steps = 250
    ids = _ids(rec)[None]
    te, le = IntQwen3Oracle(d).generate(ids.cpu().numpy(), steps)
    monkeypatch.setattr(mdl, "SPLIT_MIN_SLOTS", 0)
    assert m._split_plan(1, 512) is not None
    for use_graph in (False, True):
        tg, lg = m.generate(ids, steps, use_graph=use_graph)
        assert tg.cpu().numpy().tolist() == te.tolist(), use_graph
        assert chain_hashes(lg) == chain_hashes(le), use_graph
    ids3 = ids.repeat(3, 1)
    ids3[1, -1] = 7
    runs = []
    for thr in (0, 1 << 30):
        monkeypatch.setattr(mdl, "SPLIT_MIN_SLOTS", thr)
        runs.append(m.generate(ids3, 40 + 256 - ids.shape[1], use_graph=True))
    assert torch.equal(runs[0][0], runs[1][0])
    for a, b in zip(runs[0][1], runs[1][1]):
        assert torch.equal(a, b)


def test_step_greedy_matches_step_then_pick(case):
    """GraphedDecode.step_greedy (the pick captured in the step's graph, ids
    fed back on the device) gives the tokens and logits of
    greedy_pick(step(cur)) at batch 3, across a cache bucket growth for the
    tiny model (re-capture of both graphs)."""
    from idempotent_llm_amd.graphed import GraphedDecode
    rec, m, _ = case
    ids = _ids(rec)[None].repeat(3, 1)
    ids[1, -1] = 7
    ids[2, -2:] = 11
    B, T = ids.shape
    steps = 260 - T if rec["dims"]["hidden"] == 256 else 12
    pos = torch.arange(T, device="cuda").expand(B, T)
    lens = torch.full((B,), T, dtype=I64, device="cuda")
    runs = []
    for mode in ("step", "greedy"):
        logits, _, _, cache = m.forward(ids, pos)
        gd = GraphedDecode(m, cache, lens)
        cur = m.greedy_pick(logits[:, -1])
        toks, lgs = [], []
        for i in range(steps):
            if mode == "step":
                lg = gd.step(cur)
                cur = m.greedy_pick(lg)
            else:
                cur = gd.step_greedy(cur if i == 0 else None)
                lg = gd.out_pick[:, 0]
            toks.append(cur.clone())
            lgs.append(lg.clone())
        runs.append((torch.stack(toks), torch.stack(lgs)))
    assert torch.equal(runs[0][0], runs[1][0])
    assert torch.equal(runs[0][1], runs[1][1])


@pytest.mark.parametrize("chunk", [2048, 64, 1, 5000])
def test_greedy_pick_real_ties_on_device(chunk):
    """detllm_greedy_pick (the pick of IntQwen3.greedy_pick and of the graphed
    step) on rows with real ties inside and across arg-max chunks, with the
    chunk size varied so the cross-chunk combine sees 1 to 5000 partials:
    the lowest id among the maxima, as brute force in Python integers."""
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from idempotent_llm_amd._lib import call
    from tiecases import EXPECTED, brute_pick, tie_cases
    print(f"[greedy ties chunk={chunk}]", flush=True)
    rows, hm = tie_cases()
    assert brute_pick(rows, hm) == EXPECTED
    R, V = rows.shape
    nch = -(-V // chunk)
    pv = torch.empty(R, nch, dtype=I64, device="cuda")
    pi = torch.empty(R, nch, dtype=I64, device="cuda")
    out = torch.full((R,), -1, dtype=I64, device="cuda")
    call("detllm_greedy_pick", torch.from_numpy(rows).cuda(), torch.from_numpy(hm).cuda(),
         R, V, chunk, pv, pi, out)
    assert out.tolist() == EXPECTED


# ---------------------------------------------------------------- index errors

def test_out_of_range_indices_raise_like_the_reference(case):
    """embed_e8[ids] and cos_t[positions] raise IndexError in the reference
    (model.py:244-246, ops/rope.py:48-49); negative indices wrap as torch's
    indexing does."""
    rec, m, _ = case
    V, P = rec["dims"]["vocab"], rec["dims"]["max_pos"]
    ids = _ids(rec)[None]
    T = ids.shape[1]
    pos = torch.arange(T, device="cuda")[None]
    # host tensors: checked before the launch
    with pytest.raises(IndexError):
        m.forward(torch.tensor([[V]]), torch.tensor([[0]]))
    with pytest.raises(IndexError):
        m.forward(torch.tensor([[1]]), torch.tensor([[P]]))
    with pytest.raises(IndexError):
        m.generate(ids, P)                 # runs past the RoPE table
    # right-padded rows decode at their own lengths (pos = lens + step - 1),
    # so the last position is max(lens) + max_new - 2, not T0 + max_new - 2:
    # a run ending at position P - 1 completes, one step more raises
    ids2 = ids.expand(2, T).contiguous()
    cv = torch.ones(2, T, dtype=torch.bool, device="cuda")
    cv[0, T - 3:] = False
    cv[1, T - 5:] = False
    n_ok = P - (T - 3) + 1
    toks, _ = m.generate(ids2, n_ok, chunk_valid=cv, use_graph=True)
    assert toks.shape == (2, n_ok)
    with pytest.raises(IndexError, match="position"):
        m.generate(ids2, n_ok + 1, chunk_valid=cv, use_graph=True)
    # a cache holds a fixed number of rows: another batch size is refused on
    # the host before any kernel could index its page tables past their rows
    _, _, _, cache = m.forward(ids2, pos.expand(2, T))
    with pytest.raises(ValueError, match="rows"):
        m.forward(ids.expand(3, T).contiguous(), pos.expand(3, T) + T, cache)
    with pytest.raises(RuntimeError, match="rows"):
        m.forward(ids[:, :1], pos[:, :1] + T, cache)
    # device tensors: flagged by the kernels, raised at the next check
    bad = ids.clone()
    bad[0, 3] = V + 5
    m.forward(bad, pos)
    with pytest.raises(IndexError, match="token id"):
        m.raise_if_device_error()
    m.forward(ids, pos + P)
    with pytest.raises(IndexError, match="position"):
        m.raise_if_device_error()
    m.raise_if_device_error()              # the word was cleared
    # negative ids and positions wrap (torch semantics)
    wrapped = ids.clone()
    wrapped[0, 2] = ids[0, 2] - V
    a, _, _, _ = m.forward(ids, pos)
    b, _, _, _ = m.forward(wrapped, pos)
    m.raise_if_device_error()
    assert torch.equal(a, b)


# ---------------------------------------------------------------- seams

def test_seams_are_honoured(case):
    """_attn_scores / _attn_context / _lm_head (model.py:430-432, :469-478)
    are override points: a subclass that calls the defaults gets the fused
    path's bits through the unfused seam path, and an override that changes
    the result changes the logits."""
    from idempotent_llm_amd.model import IntQwen3
    rec, m, d = case
    calls = []

    class Spy(IntQwen3):
        def _attn_scores(self, q8, qm, qk, K8r, L, group, aux=None):
            calls.append(("scores", aux["li"], tuple(q8.shape)))
            assert aux["q"].dtype == torch.int64 and aux["kk"].dtype == torch.int64
            return super()._attn_scores(q8, qm, qk, K8r, L, group, aux)

        def _attn_context(self, probs, V8r, L, aux=None):
            calls.append(("context", aux["li"]))
            return super()._attn_context(probs, V8r, L, aux)

    spy = Spy(d, backend="rocm")
    ids = _ids(rec)[None]
    pos = torch.arange(ids.shape[1], device="cuda")[None]
    want, _, _, _ = m.forward(ids, pos)
    got, _, _, _ = spy.forward(ids, pos)
    assert torch.equal(got, want)
    n_layers = rec["dims"]["n_layers"]
    assert [c[1] for c in calls if c[0] == "scores"] == list(range(n_layers))
    assert chain_hashes(got[0]) == rec["prefill_chain"]

    class ZeroHead(IntQwen3):
        def _lm_head(self, x8, xm, xk):
            return torch.zeros(*x8.shape[:-1], self.vocab, dtype=torch.int32, device=x8.device)

    z, _, _, _ = ZeroHead(d, backend="rocm").forward(ids, pos)
    assert int(z.abs().max()) == 0


def test_qk_head_pipeline_matches_fused_q8(case):
    """The op-kernel _qk_head_pipeline (model.py:200-216) feeding the seams'
    diagnostics gives, after QK smoothing and quant_i8_pertoken
    (model.py:317-323), the q8 the fused epilogue produced."""
    from idempotent_llm_amd import dyadic as dy
    from idempotent_llm_amd.model import IntQwen3
    rec, m, d = case
    seen = {}

    class Grab(IntQwen3):
        def _attn_scores(self, q8, qm, qk, K8r, L, group, aux=None):
            if aux["li"] == 0:
                seen.update(q8=q8.clone(), qm=qm.clone(), qk=qk.clone(), q=aux["q"],
                            qkk=aux["qkk"], L=L, group=group)
            return super()._attn_scores(q8, qm, qk, K8r, L, group, aux)

    g = Grab(d, backend="rocm")
    ids = _ids(rec)[None]
    g.forward(ids, torch.arange(ids.shape[1], device="cuda")[None])
    L, grp = seen["L"], seen["group"]
    qs = L.qs_m.view(g.n_kv, g.hd).repeat_interleave(grp, dim=0)
    q = seen["q"] * qs[None, :, None, :]
    one = torch.ones(*q.shape[:-1], 1, dtype=I64, device="cuda")
    q8, qm, qk = dy.quant_i8_pertoken(q, one, one * 0 + seen["qkk"] + L.qs_k)
    assert torch.equal(q8, seen["q8"])
    assert torch.equal(qm, seen["qm"]) and torch.equal(qk, seen["qk"])


def test_graphed_modes_and_signature(case):
    """GraphedDecode(model, cache, lens, mode, layer_compile) (graphed.py:44-45):
    mode "capture" and "layers" give the same tokens and logits."""
    from idempotent_llm_amd.graphed import GraphedDecode
    rec, m, _ = case
    ids = _ids(rec)[None]
    T = ids.shape[1]
    pos = torch.arange(T, device="cuda")[None]
    lens = torch.full((1,), T, dtype=I64, device="cuda")
    runs = []
    for mode in ("capture", "layers"):
        lg, _, _, cache = m.forward(ids, pos)
        gd = GraphedDecode(m, cache, lens, mode=mode, layer_compile=True)
        cur = m.greedy_pick(lg[:, -1])
        out = []
        for _ in range(6):
            lg1 = gd.step(cur).clone()
            cur = m.greedy_pick(lg1)
            out.append(lg1)
        runs.append(torch.stack(out))
    assert torch.equal(runs[0], runs[1])
    with pytest.raises(ValueError):
        GraphedDecode(m, m.forward(ids, pos)[3], lens, mode="bogus")


def test_logits_digest_matches_host_formula(case):
    """detllm_logits_digest against the same sum computed in Python."""
    from idempotent_llm_amd.demo import logits_digest
    rec, m, _ = case
    rows = torch.tensor(np.stack([rec["prefill_last_row"], [0] * len(rec["prefill_last_row"])]),
                        dtype=torch.int32, device="cuda")
    got = logits_digest(rows).cpu().tolist()
    M = (1 << 64) - 1

    def mix(z):
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        return z ^ (z >> 31)

    for r, g in zip(rows.cpu().numpy(), got):
        want = sum(mix((i << 32) | (int(x) & 0xFFFFFFFF)) for i, x in enumerate(r)) & M
        assert g & M == want
