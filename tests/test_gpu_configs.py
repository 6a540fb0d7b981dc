"""The benchmark configurations c1–c4 on the GPU, exact against the CPU oracle
(which the reference's golden vectors pin) or, where the oracle would need
minutes, through the invariances the reference's tests check
(tests/test_determinism.py): batch composition, prefill/decode split,
query chunking, graph == eager.

Inputs follow the recipes of the benchmark configurations: splitmix64
streams and Irwin-Hall Gaussians (idempotent_llm_amd.artifact), seeds 1–4."""

import numpy as np
import pytest
import torch

from idempotent_llm_amd import artifact as art
from idempotent_llm_amd.hashchain import chain_hashes
from oracle import dyadic as ody
from oracle import gemm as ogemm
from oracle import ops as oops

pytestmark = pytest.mark.gpu
I64 = torch.int64


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from idempotent_llm_amd import _lib
    _lib.load()


def g(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def eq(got, want, what=""):
    got = got.cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    assert np.array_equal(got.astype(np.int64), want.astype(np.int64)), what


# ---------------------------------------------------------------- c1: MLP block

def test_c1_mlp_block_2048_tokens():
    """_norm_quant -> gate|up GEMM -> requant_i32_common(14) x2 -> di_swiglu ->
    quant_i8_pertoken -> down GEMM -> requant_i32_common(20) -> residual_add
    (model.py:414-427) on 2048 tokens, identity smoothing."""
    from idempotent_llm_amd._lib import call
    from idempotent_llm_amd.backends import gemm_nt
    print("[c1 MLP block T=2048]", flush=True)
    T, H, I = 2048, 1024, 3072
    h = art.gauss_int(1, "c1.h", (T, H), 1 << 12).astype(np.int32)
    k_res = np.full((T, 1), 24, np.int64)
    Wg = art.rand_i8(1, "c1.gate", (H, I))
    Wu = art.rand_i8(1, "c1.up", (H, I))
    Wd = art.rand_i8(1, "c1.down", (I, H))
    gm = art.uniform_int(1, "c1.gate_m", (I,), 1 << 14, 1 << 15)
    um = art.uniform_int(1, "c1.up_m", (I,), 1 << 14, 1 << 15)
    dm = art.uniform_int(1, "c1.down_m", (H,), 1 << 14, 1 << 15)
    ones_h, ones_i = np.ones(H, np.int64), np.ones(I, np.int64)
    # oracle (model.py:414-427 with ms_m = ds_m = 1, ms_k = ds_k = 0)
    y = oops.di_rmsnorm(h).astype(np.int64) * ones_h
    x8, xm, xk = ody.quant_i8_pertoken(y, np.ones((T, 1), np.int64), np.full((T, 1), 20))
    gate, ogm, ogk = ody.requant_i32_common(ogemm.int_gemm(x8, Wg), xm, xk, gm, 20, 14)
    up, oum, ouk = ody.requant_i32_common(ogemm.int_gemm(x8, Wu), xm, xk, um, 20, 14)
    ys, ym, yk = oops.di_swiglu(gate, ogm, ogk, up, oum, ouk)
    y8, y8m, y8k = ody.quant_i8_pertoken(ys * ones_i, ym, yk + 0)
    d, ddm, ddk = ody.requant_i32_common(ogemm.int_gemm(y8, Wd), y8m, y8k, dm, 20, 20)
    h_out, k_out = ody.residual_add(h, k_res, d, ddm, ddk)
    # GPU: the model's fused kernels
    hg = g(h)
    kg = g(k_res[:, 0].copy())
    x8g = torch.empty(T, H, dtype=torch.int8, device="cuda")
    xmg = torch.empty(T, dtype=I64, device="cuda")
    xkg = torch.empty(T, dtype=I64, device="cuda")
    call("detllm_norm_quant", hg, T, H, g(ones_h), 0, x8g, xmg, xkg)
    eq(x8g, x8, "x8"); eq(xmg, xm[:, 0], "xm"); eq(xkg, xk[:, 0], "xk")
    Wgu = g(np.concatenate([Wg, Wu], axis=1).T.copy())
    P = gemm_nt(x8g, Wgu)
    y8g = torch.empty(T, I, dtype=torch.int8, device="cuda")
    ymg = torch.empty(T, dtype=I64, device="cuda")
    ykg = torch.empty(T, dtype=I64, device="cuda")
    call("detllm_swiglu_quant", P, 1, 0, T, I, xmg, xkg, g(gm), 20, g(um), 20, g(ones_i), 0,
         y8g, ymg, ykg, None, 0, 0, 0, 0)
    eq(y8g, y8, "y8"); eq(ymg, y8m[:, 0], "ym"); eq(ykg, y8k[:, 0], "yk")
    Pd = gemm_nt(y8g, g(Wd.T.copy()))
    call("detllm_residual_normq", Pd, 1, 0, T, H, ymg, ykg, g(dm), 20, 20, hg, kg, None, 0,
         None, None, None, None, 0, 0, 0, 0)
    eq(hg, h_out, "h"); eq(kg, k_out[:, 0], "k_res")


# ------------------------------------------------------- c2: attention prefill

def _c2_inputs(T):
    nq, nkv, hd = 16, 8, 128
    q = np.clip(art.gauss_int(2, "c2.q", (1, nq, T, hd), 32), -127, 127)
    k = np.clip(art.gauss_int(2, "c2.k", (1, nkv, T, hd), 32), -127, 127)
    v = np.clip(art.gauss_int(2, "c2.v", (1, nkv, T, hd), 32), -127, 127).astype(np.int8)
    cos_t, sin_t = oops.build_rope_tables(hd, 4096, 1e6)
    return q, k, v, cos_t, sin_t


def _c2_oracle(T, p_out_bits=15):
    q, k, v, cos_t, sin_t = _c2_inputs(T)
    pos = np.arange(T)
    q8, qm, qk = ody.quant_i8_pertoken(oops.apply_int_rope(q, cos_t, sin_t, pos), 1, 0)
    k8 = ody.requant_i8_static(oops.apply_int_rope(k, cos_t, sin_t, pos), 1, 0, 1, 0, 1, 0)
    sm, sk = ody.norm_scale(qm * 46341, qk + 19)
    causal = np.arange(T)[None, :] <= np.arange(T)[:, None]
    ctx = np.empty((1, 16, T, 128), np.int64)
    for hq in range(16):
        sc = ogemm.int_gemm(q8[:, hq], np.ascontiguousarray(k8[:, hq // 2].transpose(0, 2, 1)))
        p = oops.di_softmax(sc, sm[:, hq], sk[:, hq], causal[None], p_out_bits=p_out_bits)
        if p_out_bits == 15:
            ctx[:, hq] = ogemm.int_gemm_u16i8(p, v[:, hq // 2])
        else:
            ctx[:, hq] = ogemm.int_gemm_u8i8(p, v[:, hq // 2])
    att = ctx.transpose(0, 2, 1, 3).reshape(T, 16 * 128)
    out = ody.requant_i8_rowcol(att, np.ones((T, 1), np.int64), np.zeros((T, 1), np.int64),
                                np.ones(16 * 128, np.int64), 14)
    return (q8, k8, v, sm, sk), ctx, out


def _c2_gpu(T, chunk=None):
    """Q/K through the op kernels, then the MFMA prefill attention kernel on a
    [1, 8, cap, 128] K / [1, 8, 128, cap] V^T cache; queries in chunks of
    `chunk` (S_past advancing) when given."""
    from idempotent_llm_amd import dyadic as dd
    from idempotent_llm_amd import ops as dops
    from idempotent_llm_amd._lib import call
    q, k, v, cos_t, sin_t = _c2_inputs(T)
    pos = torch.arange(T, device="cuda")
    q8, qm, qk = dd.quant_i8_pertoken(dops.apply_int_rope(g(q), g(cos_t), g(sin_t), pos), 1, 0)
    k8 = dd.requant_i8_static(dops.apply_int_rope(g(k), g(cos_t), g(sin_t), pos), 1, 0, 1, 0, 1, 0)
    sm, sk = dd.norm_scale(qm * 46341, qk + 19)
    _, tpos = dops.di_exp(torch.zeros_like(sm), sm, sk)
    from pagedcache import paged
    cap = (T + 255) // 256 * 256
    kc = torch.zeros(1, 8, cap, 128, dtype=torch.int8, device="cuda")
    vc = torch.zeros(1, 8, 128, cap, dtype=torch.int8, device="cuda")
    kc[:, :, :T] = k8
    vc[..., :T] = g(v).transpose(2, 3)
    valid = torch.zeros(1, cap, dtype=torch.bool, device="cuda")
    valid[:, :T] = True
    kp, vp, table, width, valid = paged(kc, vc, valid, seed=T)
    out = torch.empty(1, T, 16 * 128, dtype=I64, device="cuda")
    step = chunk or T
    for t0 in range(0, T, step):
        t1 = min(T, t0 + step)
        q8c = q8[:, :, t0:t1].contiguous()
        tc = tpos[:, :, t0:t1, 0].contiguous()
        oc = torch.empty(1, t1 - t0, 16 * 128, dtype=I64, device="cuda")
        call("detllm_attn_prefill", q8c, tc, kp, vp, table, width, valid.view(torch.uint8),
             width * 128, 1, t1 - t0, t0, 16, 8, oc)
        out[:, t0:t1] = oc
    res = dd.requant_i8_rowcol(out[0], 1, 0, torch.ones(2048, dtype=I64, device="cuda"), 14)
    return (q8, k8, sm, sk), out, res


@pytest.mark.parametrize("T", [512, 2048])
def test_c2_attention_prefill_vs_oracle(T):
    """Config c2 (seq 2048, causal, 16q/8kv x 128, RoPE theta 1e6, 15-bit
    probabilities, hi/lo P.V, rowcol requant to int8), exact."""
    print(f"[c2 attention prefill T={T}]", flush=True)
    (q8, k8, v, sm, sk), ctx, (o8, om, ok) = _c2_oracle(T)
    (gq8, gk8, gsm, gsk), gctx, (g8, gm, gk) = _c2_gpu(T)
    eq(gq8, q8, "q8"); eq(gk8, k8, "k8"); eq(gsm, sm, "sm"); eq(gsk, sk, "sk")
    eq(gctx[0], ctx[0].transpose(1, 0, 2).reshape(T, 2048), "context")
    eq(g8, o8, "out8"); eq(gm, om, "out m"); eq(gk, ok, "out k")


def test_c2_query_chunking_invariance():
    """Queries in chunks of 256 against the same cache give the same bits as
    one 2048-query launch (model.py:383-401: every op is per query row)."""
    print("[c2 chunking]", flush=True)
    _, full, _ = _c2_gpu(2048)
    _, chunked, _ = _c2_gpu(2048, chunk=256)
    assert torch.equal(full, chunked)


def test_c2_int8_probability_variant():
    """p_out_bits = 8 probabilities in [0, 128] with the u8 trick
    (backends.py:138-149), the literal "int8 probabilities" reading of c2."""
    from idempotent_llm_amd import dyadic as dd
    from idempotent_llm_amd import ops as dops
    from idempotent_llm_amd.backends import int_gemm_u8i8
    print("[c2 int8 probabilities]", flush=True)
    T = 256
    (q8, k8, v, sm, sk), ctx, _ = _c2_oracle(T, p_out_bits=8)
    causal = torch.arange(T, device="cuda")[None, :] <= torch.arange(T, device="cuda")[:, None]
    for hq in (0, 7, 15):
        sc = ogemm.int_gemm(q8[:, hq], np.ascontiguousarray(k8[:, hq // 2].transpose(0, 2, 1)))
        p = dops.di_softmax(g(sc), g(sm[:, hq]), g(sk[:, hq]), causal[None], p_out_bits=8)
        assert int(p.max()) <= 128 and int(p.min()) >= 0
        eq(int_gemm_u8i8(p, g(v[:, hq // 2]), "rocm"), ctx[:, hq], f"head {hq}")


# ------------------------------------------------------- c3: full model decode

@pytest.fixture(scope="module")
def full_model(tmp_path_factory):
    from idempotent_llm_amd.model import IntQwen3
    d = str(tmp_path_factory.mktemp("qwen3_0p6b"))
    print("[full model: artifact]", flush=True)
    art.make_artifact(d, art.QWEN3_0_6B, seed=3)
    return d, IntQwen3(d, backend="rocm")


def _c3_fixture():
    import json
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "c3_chains.json")
    with open(path) as f:
        return json.load(f)


@pytest.mark.parametrize("config", ["b1", "b8", "split"])
def test_c3_every_step_vs_oracle_fixture(full_model, config):
    """Config c3 as configured: 64-token prompt (seed 30), 512 greedy steps
    (prefill + 511 graphed decodes) at batch 1, batch 8 (every row) and split
    prefill, run by the determinism harness (scripts/demo.py:101-164). The
    tokens and the demo chain hashes of every step of every row equal the
    CPU oracle's (tests/golden/c3_chains.json, make_c3_fixture.py)."""
    from idempotent_llm_amd.demo import run_int8
    d, m = full_model
    fx = _c3_fixture()
    assert art.artifact_digest(d) == fx["artifact_sha256"], "artifact generator drifted"
    V = art.QWEN3_0_6B["vocab"]
    prompt = art.prompt_ids(fx["prompt_seed"], fx["prompt_len"], V)
    co = art.co_prompts(fx["co_prompt_seed"], 7, V)
    steps = fx["steps"]
    print(f"[c3 {config}: {steps} steps vs oracle fixture]", flush=True)
    tcs, lcs = run_int8(m, f"int8-rocm-{config}", steps, prompt, co, all_rows=True)
    want = fx[config] if config == "b8" else [fx[config]]
    assert len(tcs) == len(want)
    for r, (tc, lc, w) in enumerate(zip(tcs, lcs, want)):
        first_bad = next((i for i, (a, b) in enumerate(zip(lc.steps, w["logit_chain"]))
                          if a != b), None)
        assert first_bad is None, f"row {r}: logits diverge from the oracle at step {first_bad}"
        assert tc.steps == w["token_chain"], f"row {r}: tokens"
        assert len(lc.steps) == steps


def test_c3_batch8_row0_equals_batch1_512_steps(full_model):
    """b8 = the b1 prompt plus 7 seeded co-prompts, right-padded
    (scripts/demo.py:90-124): row 0's tokens and logits at every one of 512
    graphed steps equal the b1 run's."""
    _, m = full_model
    print("[c3 b8 vs b1, 512 steps]", flush=True)
    V = art.QWEN3_0_6B["vocab"]
    p0 = art.prompt_ids(30, 64, V)
    ids, valid = art.right_pad([p0] + art.co_prompts(31, 7, V))
    t1, l1 = m.generate(torch.from_numpy(p0)[None].cuda(), 512, use_graph=True)
    t8, l8 = m.generate(torch.from_numpy(ids).cuda(), 512, use_graph=True,
                        chunk_valid=torch.from_numpy(valid).cuda())
    assert torch.equal(t8[0], t1[0])
    for a, b in zip(l8, l1):
        assert torch.equal(a[0], b[0])


# ----------------------------------------------------- c4: batch-32 stress

def _graphed_run(m, ids, valid, steps, on_step):
    """IntQwen3.generate(use_graph=True) (model.py:492-522) with a per-step
    callback instead of keeping every step's logits."""
    from idempotent_llm_amd.graphed import GraphedDecode
    B, T = ids.shape
    pos = torch.arange(T, device="cuda").expand(B, T)
    lens = valid.sum(dim=1)
    logits, _, _, cache = m._forward(ids, pos, None, valid, (lens - 1).clamp(min=0))
    cur = m.greedy_pick(logits)
    on_step(0, logits, cur)
    gd = GraphedDecode(m, cache, lens)
    for i in range(1, steps):
        lg = gd.step(cur)
        cur = m.greedy_pick(lg)
        on_step(i, lg, cur)


def test_c4_batch32_to_4096_slots(full_model):
    """32 prompts of seeded lengths in [16, 1024], right-padded, prefill, then
    graphed decode until the cache holds 4096 slots (the graph is re-captured
    when the cache bucket grows). Row 0's token and logits at every step
    equal its batch-1 run's."""
    _, m = full_model
    lens = art.uniform_int(4, "c4.lens", (32,), 16, 1025)
    prompts = [art.uniform_int(4, f"c4.prompt.{i}", (int(n),), 100, 50000)
               for i, n in enumerate(lens)]
    ids, valid = art.right_pad(prompts)
    T_pad = ids.shape[1]
    steps = 4096 - T_pad
    print(f"[c4 b32 T_pad={T_pad} steps={steps}]", flush=True)
    ref_l, ref_t = [], []
    _graphed_run(m, torch.from_numpy(prompts[0])[None].cuda(),
                 torch.ones(1, len(prompts[0]), dtype=torch.bool, device="cuda"), steps,
                 lambda i, lg, cur: (ref_l.append(lg[0].clone()), ref_t.append(cur[0].clone())))
    bad = []

    def check(i, lg, cur):
        if not (torch.equal(lg[0], ref_l[i]) and torch.equal(cur[0], ref_t[i])):
            bad.append(i)

    _graphed_run(m, torch.from_numpy(ids).cuda(), torch.from_numpy(valid).cuda(), steps, check)
    assert not bad, bad[:10]


def _c4_prompts():
    lens = art.uniform_int(4, "c4.lens", (32,), 16, 1025)
    return [art.uniform_int(4, f"c4.prompt.{i}", (int(n),), 100, 50000)
            for i, n in enumerate(lens)]


@pytest.mark.parametrize("graphed", [True, False], ids=["graphed", "eager"])
def test_c4_prefix_vs_oracle_fixture(full_model, graphed):
    """Config c4's batch of 32 ragged prompts (seeded lengths in [16, 1024],
    right-padded) against the CPU oracle on a prefix of the run: the prefill
    and the first decodes of every row (the full run to 4096 slots would take
    the oracle days). Tokens and the demo chain hashes of the logits at every
    step of every row equal tests/golden/c4_prefix.json (make_c4_fixture.py)."""
    import json
    import os
    d, m = full_model
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                           "c4_prefix.json")) as f:
        fx = json.load(f)
    assert art.artifact_digest(d) == fx["artifact_sha256"], "artifact generator drifted"
    prompts = _c4_prompts()
    assert [len(p) for p in prompts] == fx["lens"]
    ids, valid = art.right_pad(prompts)
    assert ids.shape[1] == fx["padded_len"]
    steps = fx["steps"]
    print(f"[c4 prefix vs oracle: B=32 T={ids.shape[1]} steps={steps} graphed={graphed}]",
          flush=True)
    toks, lg = m.generate(torch.from_numpy(ids).cuda(), steps, use_graph=graphed,
                          chunk_valid=torch.from_numpy(valid).cuda())
    rows = [[r.cpu().numpy() for r in step] for step in lg]
    for b, w in enumerate(fx["rows"]):
        assert toks[b].tolist() == w["tokens"], f"row {b}: tokens"
        assert chain_hashes([rows[s][b] for s in range(steps)]) == w["logit_chain"], f"row {b}"


def test_4k_prompt_long_context(full_model):
    """tests/test_determinism.py:127-161 on the full-size model with a
    4096-token prompt (seeded ids: the reference tokenises wikitext, a
    network fetch): run-to-run equality of 5 greedy steps (eager, and the
    graphed decode equal to it); batch invariance at bs 2 with a 100-token
    co-prompt; and prefill of 4095 tokens then one decode equal to the full
    prefill's last row (the decode scans 4096 slots: split-S attention)."""
    _, m = full_model
    V = art.QWEN3_0_6B["vocab"]
    ids = torch.from_numpy(art.prompt_ids(40, 4096, V)).cuda()
    T = ids.shape[0]
    print("[4k prompt: run-to-run]", flush=True)
    t1, l1 = m.generate(ids[None], 5)
    t2, l2 = m.generate(ids[None], 5)
    tg, lgr = m.generate(ids[None], 5, use_graph=True)
    assert torch.equal(t1, t2) and torch.equal(t1, tg)
    for a, b, c in zip(l1, l2, lgr):
        assert torch.equal(a, b) and torch.equal(a, c)
    print("[4k prompt: bs-2 batch invariance]", flush=True)
    bids = torch.zeros(2, T, dtype=torch.int64, device="cuda")
    valid = torch.zeros(2, T, dtype=torch.bool, device="cuda")
    bids[0] = ids
    valid[0] = True
    bids[1, :100] = ids[:100]
    valid[1, :100] = True
    tb, lb = m.generate(bids, 5, chunk_valid=valid)
    assert torch.equal(tb[0], t1[0])
    for a, b in zip(lb, l1):
        assert torch.equal(a[0], b[0])
    print("[4k prompt: prefill 4095 + decode 1 == full prefill]", flush=True)
    pos = torch.arange(T, device="cuda")[None]
    full, _, _, _ = m.forward(ids[None], pos)
    _, _, _, c = m.forward(ids[None, :-1], pos[:, :-1])
    lg2, _, _, c = m.forward(ids[None, -1:], pos[:, -1:], c)
    assert torch.equal(full[0, -1], lg2[0, 0])
    assert torch.equal(full[0, -1], l1[0][0])
    m.raise_if_device_error()


def test_c4_split_prefill_batch32(full_model):
    """Split prefill of config c4's ragged batch of 32 (seeded lengths in
    [16, 1024]): the first half of the padded length at once, then token by
    token (padding slots stay invalid); the logits of every valid position
    equal the one-shot prefill's (tests/test_determinism.py:96-113, for a
    batch)."""
    _, m = full_model
    lens = art.uniform_int(4, "c4.lens", (32,), 16, 1025)
    prompts = [art.uniform_int(4, f"c4.prompt.{i}", (int(n),), 100, 50000)
               for i, n in enumerate(lens)]
    ids, valid = art.right_pad(prompts)
    B, T = ids.shape
    print(f"[c4 split prefill B={B} T={T}]", flush=True)
    ids_g, valid_g = torch.from_numpy(ids).cuda(), torch.from_numpy(valid).cuda()
    pos = torch.arange(T, device="cuda").expand(B, T)
    full, _, _, _ = m.forward(ids_g, pos, chunk_valid=valid_g)
    half = T // 2
    lg, _, _, cache = m.forward(ids_g[:, :half], pos[:, :half], chunk_valid=valid_g[:, :half])
    mism = []
    for t in range(half):
        ok = torch.equal(lg[:, t][valid_g[:, t]], full[:, t][valid_g[:, t]])
        if not ok:
            mism.append(t)
    for t in range(half, T):
        lg, _, _, cache = m.forward(ids_g[:, t:t + 1], pos[:, t:t + 1], cache,
                                    chunk_valid=valid_g[:, t:t + 1])
        if not torch.equal(lg[:, 0][valid_g[:, t]], full[:, t][valid_g[:, t]]):
            mism.append(t)
    assert not mism, mism[:10]
