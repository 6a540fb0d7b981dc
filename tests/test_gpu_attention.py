"""GPU checks of the decode attention paths through the C-ABI: the fused
Q/K/V-epilogue + attention kernel (detllm_qkv_attn_decode) against the two
separate launches it replaces (detllm_qkv_epilogue, detllm_attn_decode),
which the model goldens pin to the reference CPU path. Exact equality of the
attention output and of every cache byte, for random cache contents, ragged
validity masks, scanned-slot bounds given on the host or on the device, and
score rows that need the global scratch."""

import numpy as np
import pytest
import torch

from idempotent_llm_amd import artifact as art
from pagedcache import paged, unpaged

pytestmark = pytest.mark.gpu
I64 = torch.int64


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from idempotent_llm_amd import _lib
    _lib.load()


def _layer_params(dims, seed):
    t, cfg = art.make_artifact_tensors(dims, seed)
    p, Lc = "layers.0.", cfg["layers"][0]
    d = lambda n: torch.from_numpy(np.ascontiguousarray(t[p + n])).cuda()
    g = dict(q_m=d("q.m"), q_k=Lc["q"]["k"], k_m=d("k.m"), k_k=Lc["k"]["k"], v_m=d("v.m"),
             v_k=Lc["v"]["k"], q_norm_m=d("q_norm.m"), q_norm_k=Lc["q_norm_k"],
             k_norm_m=d("k_norm.m"), k_norm_k=Lc["k_norm_k"],
             qs_m=d("qs_m").reshape(-1).contiguous(), qs_k=Lc["qs_k"],
             kq_m=d("kq_m").reshape(-1).contiguous(), kq_k=d("kq_k").reshape(-1).contiguous(),
             ks_m=d("ks_m"), ks_k=d("ks_k"), vq_m=d("vq_m"), vq_k=d("vq_k"),
             cos=torch.from_numpy(t["rope.cos"]).cuda(), sin=torch.from_numpy(t["rope.sin"]).cuda())
    return g


def _run(dims, B, cap, S, slot, device_bounds, seed):
    from idempotent_llm_amd._lib import call
    prm = _layer_params(dims, seed)
    nq, nkv, hd = dims["n_q_heads"], dims["n_kv_heads"], 128
    rnd = torch.Generator().manual_seed(seed)
    ns = 2
    P = torch.randint(-(1 << 19), 1 << 19, (ns, B, (nq + 2 * nkv) * hd), generator=rnd,
                      dtype=torch.int32).cuda()
    xm = torch.randint(1 << 15, 1 << 16, (B,), generator=rnd, dtype=I64).cuda()
    xk = torch.randint(22, 30, (B,), generator=rnd, dtype=I64).cuda()
    pos = torch.randint(0, dims["max_pos"], (B,), generator=rnd, dtype=I64).cuda()
    k0 = torch.randint(-128, 128, (B, nkv, cap, hd), generator=rnd, dtype=torch.int8).cuda()
    v0 = torch.randint(-128, 128, (B, nkv, hd, cap), generator=rnd, dtype=torch.int8).cuda()
    valid = (torch.rand(B, cap, generator=rnd) < 0.8).cuda()
    valid[:, slot] = True
    k0, v0, table, width, valid = paged(k0, v0, valid, seed=seed)
    vbytes = valid.view(torch.uint8)
    cap = width * 128
    G = nq // nkv
    Spad = (S + 15) // 16 * 16
    scratch = (torch.empty(B, nq, Spad, dtype=torch.int32, device="cuda")
               if G * Spad * 4 > 48 * 1024 else None)
    slot_dev = torch.tensor([slot], dtype=I64, device="cuda") if device_bounds else None
    s_dev = torch.tensor([S], dtype=I64, device="cuda") if device_bounds else None
    S_host = cap if device_bounds else S
    common = (prm["q_m"], prm["q_k"], prm["k_m"], prm["k_k"], prm["v_m"], prm["v_k"],
              prm["q_norm_m"], prm["q_norm_k"], prm["k_norm_m"], prm["k_norm_k"], prm["qs_m"],
              prm["qs_k"], prm["kq_m"], prm["kq_k"], prm["ks_m"], prm["ks_k"], prm["vq_m"],
              prm["vq_k"], prm["cos"], prm["sin"], prm["cos"].shape[0])
    # separate launches
    ka, va = k0.clone(), v0.clone()
    q8 = torch.empty(B, nq, 1, hd, dtype=torch.int8, device="cuda")
    tpos = torch.empty(B, nq, 1, dtype=I64, device="cuda")
    out_a = torch.empty(B, nq * hd, dtype=I64, device="cuda")
    call("detllm_qkv_epilogue", P, ns, B * P.shape[2], B, 1, nq, nkv, xm, xk, pos, *common,
         q8, tpos, None, ka, va, table, width, slot_dev, slot, None, None)
    call("detllm_attn_decode", q8, tpos, ka, va, table, width, vbytes, cap, B, S_host, nq, nkv,
         s_dev, scratch, out_a, None)
    # fused launch
    kb, vb = k0.clone(), v0.clone()
    out_b = torch.empty(B, nq * hd, dtype=I64, device="cuda")
    call("detllm_qkv_attn_decode", P, ns, B * P.shape[2], B, nq, nkv, xm, xk, pos, *common,
         kb, vb, table, width, slot_dev, slot, vbytes, cap, S_host, s_dev, scratch, out_b, None)
    # with the merge statistics (detllm_qkv_attn_decode_ext): the same
    # cache and context, and per (row, kv head) the largest v and ~v over
    # v = context * om of the kv head's query heads (and 0), om spanning
    # products that wrap
    om = torch.randint(-(1 << 40), 1 << 40, (nq * hd,), generator=rnd, dtype=I64).cuda()
    kc, vc = k0.clone(), v0.clone()
    out_c = torch.empty(B, nq * hd, dtype=I64, device="cuda")
    ext = torch.full((B, nkv, 2), 99, dtype=I64, device="cuda")
    call("detllm_qkv_attn_decode_ext", P, ns, B * P.shape[2], B, nq, nkv, xm, xk, pos, *common,
         kc, vc, table, width, slot_dev, slot, vbytes, cap, S_host, s_dev, scratch, out_c, None,
         om, ext)
    torch.cuda.synchronize()
    assert torch.equal(ka, kb)
    assert torch.equal(va, vb)
    assert torch.equal(out_a, out_b)
    assert torch.equal(kc, kb) and torch.equal(vc, vb) and torch.equal(out_c, out_b)
    vv = (out_b.cpu() * om.cpu()).view(B, nkv, G * hd)   # int64 products wrap
    hi = torch.clamp(vv.max(dim=2).values, min=0)
    nm = torch.clamp((~vv).max(dim=2).values, min=-1)
    assert torch.equal(ext.cpu(), torch.stack([hi, nm], dim=2))
    assert not torch.equal(ka, k0)          # the step's K slot was written
    assert out_a.abs().sum().item() > 0


@pytest.mark.parametrize("S,device_bounds", [(1, False), (17, False), (300, True), (512, False)])
def test_fused_decode_equals_separate_launches(S, device_bounds):
    print(f"[fused decode S={S} device_bounds={device_bounds}]", flush=True)
    _run(art.MID, B=3, cap=512, S=S, slot=S - 1, device_bounds=device_bounds, seed=S)


def test_fused_decode_scratch_path():
    """Scores of a (row, kv-head) beyond the 48 KiB LDS budget (S = 6200,
    G = 2) go through the global scratch in both paths."""
    print("[fused decode scratch S=6200]", flush=True)
    _run(art.MID, B=2, cap=6400, S=6200, slot=6199, device_bounds=False, seed=5)


def test_fused_decode_group1():
    dims = dict(art.TINY, n_q_heads=2, n_kv_heads=2)
    print("[fused decode G=1]", flush=True)
    _run(dims, B=2, cap=256, S=100, slot=99, device_bounds=True, seed=9)


# ------------------------------------------------------------ prefill kernel

def _prefill_case(B, n_q, n_kv, T, S_past, cap, seed, sk_lo, sk_hi, zero_heads=(),
                  extreme_rows=(), dead_prefix=0, p_valid=0.75, sm_lo=1 << 15):
    """Random prefill inputs: q8/K/V bytes, per-row score scales (sm, sk) and
    the DI-Exp constant tpos they give, a ragged validity mask. zero_heads get
    q = 0 (every score 0: flat rows, the largest denominators); extreme_rows
    (b, h, t) get q = -128 against K rows of -128 (scores of 2^21); batch row
    1 has its first dead_prefix slots invalid (queries that see no slot)."""
    from oracle import ops as oops
    rng = np.random.default_rng(seed)
    S = S_past + T
    q8 = rng.integers(-128, 128, (B, n_q, T, 128), dtype=np.int8)
    for h in zero_heads:
        q8[:, h] = 0
    kc = rng.integers(-128, 128, (B, n_kv, cap, 128), dtype=np.int8)
    vc = rng.integers(-128, 128, (B, n_kv, 128, cap), dtype=np.int8)
    for (b, h, t) in extreme_rows:
        q8[b, h, t] = -128
        kc[b, h // (n_q // n_kv), :S:7] = -128
    sm = rng.integers(sm_lo, 1 << 16, (B, n_q, T, 1), dtype=np.int64)
    sk = rng.integers(sk_lo, sk_hi + 1, (B, n_q, T, 1), dtype=np.int64)
    tpos = oops.di_exp_tpos(sm, sk)
    valid = rng.random((B, cap)) < p_valid
    if B > 1 and dead_prefix:
        valid[1, :dead_prefix] = False
    return q8, kc, vc, valid, sm, sk, tpos


def _prefill_oracle(q8, kc, vc, valid, sm, sk, S_past):
    """model.py:382-402 on the CPU oracle: int8 scores, DI-Softmax over the
    slots s <= S_past + t that are valid, exact p.v."""
    from oracle import gemm as ogemm
    from oracle import ops as oops
    B, n_q, T, _ = q8.shape
    n_kv = kc.shape[1]
    S = S_past + T
    vis = (np.arange(S)[None, :] <= (S_past + np.arange(T))[:, None])
    out = np.zeros((B, T, n_q * 128), dtype=np.int64)
    for b in range(B):
        mask = vis & valid[b, None, :S]
        for h in range(n_q):
            kvh = h // (n_q // n_kv)
            sc = ogemm.int_gemm(q8[b, h], np.ascontiguousarray(kc[b, kvh, :S].T))
            p = oops.di_softmax(sc, sm[b, h], sk[b, h], mask)
            out[b, :, h * 128:(h + 1) * 128] = ogemm.matmul_i64(
                p, np.ascontiguousarray(vc[b, kvh, :, :S].T))
    return out


PREFILL_CASES = {
    # B, n_q, n_kv, T, S_past, cap, seed, sk range, extras
    "typical": (2, 4, 2, 150, 37, 192, 1, 29, 34, {}),
    "wide_tpos": (2, 4, 2, 150, 37, 192, 2, 0, 62, dict(dead_prefix=40)),
    "flat_big_den": (1, 4, 1, 200, 0, 208, 3, 46, 60, dict(zero_heads=(0, 2), p_valid=1.0)),
    "extreme_scores": (2, 2, 2, 96, 5, 112, 4, 28, 40,
                       dict(extreme_rows=((0, 0, 3), (1, 1, 95), (0, 1, 50)))),
    "one_tile": (1, 2, 1, 64, 0, 64, 5, 30, 33, {}),
    "single_query": (3, 2, 2, 1, 300, 304, 6, 25, 45, dict(dead_prefix=301)),
    # tpos just below 2^23 on every row, flat rows over 4096 slots: sums of
    # exps beyond 2^34 next to small ones
    "big_tpos_long_rows": (1, 2, 1, 64, 4032, 4096, 7, 39, 39,
                           dict(zero_heads=(0,), sm_lo=60000, p_valid=1.0)),
}


@pytest.mark.parametrize("name", list(PREFILL_CASES))
def test_prefill_attention_vs_oracle(name):
    """detllm_attn_prefill (model.py:382-402) against the oracle's
    composition: int_gemm scores, di_softmax (ops/di_softmax.py:33-61) over
    valid & causal slots, exact p.v; tpos from the oracle's di_exp_tpos.
    Exact equality, including rows with no visible slot (all-zero context),
    tpos from 1 to about 2^46 in one wave, and denominators beyond 2^32."""
    from idempotent_llm_amd._lib import call
    B, n_q, n_kv, T, S_past, cap, seed, lo, hi, extra = PREFILL_CASES[name]
    print(f"[prefill attention {name}: B={B} n_q={n_q} n_kv={n_kv} T={T} S_past={S_past}]",
          flush=True)
    q8, kc, vc, valid, sm, sk, tpos = _prefill_case(B, n_q, n_kv, T, S_past, cap, seed, lo, hi,
                                                    **extra)
    want = _prefill_oracle(q8, kc, vc, valid, sm, sk, S_past)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    out = torch.full((B, T, n_q * 128), -7, dtype=I64, device="cuda")
    kp, vp, table, width, vmask = paged(kc, vc, valid, seed=seed)
    call("detllm_attn_prefill", d(q8), d(tpos[..., 0]), kp, vp, table, width,
         vmask.view(torch.uint8), width * 128, B, T, S_past, n_q, n_kv, out)
    got = out.cpu().numpy()
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} mismatches, first at {bad[0].tolist()}"
    if name == "flat_big_den":
        assert tpos[0, 0].max() > (1 << 32)  # den = sum of exps >= tpos * visible slots
    if name == "big_tpos_long_rows":
        assert tpos.max() < (1 << 23) and tpos.min() * 4033 > (1 << 34)


# ------------------------------------------------------------- decode kernel

DECODE_CASES = {
    # B, n_q, n_kv, S, cap, seed, sk range, extras  (one query at slot S - 1)
    "typical": (3, 4, 2, 300, 320, 11, 29, 34, {}),
    "wide_tpos": (2, 4, 2, 200, 208, 12, 0, 62, dict(dead_prefix=200)),
    "big_tpos_long_rows": (1, 2, 1, 4096, 4096, 13, 39, 39,
                           dict(zero_heads=(0,), sm_lo=60000, p_valid=1.0)),
    "single_slot": (2, 2, 2, 1, 16, 14, 25, 45, {}),
}


@pytest.mark.parametrize("name", list(DECODE_CASES))
def test_decode_attention_vs_oracle(name):
    """detllm_attn_decode (ops/fused_attn.py:47-142 semantics) against the
    oracle composition for one query per row at slot S - 1 (every valid slot
    below S visible): ragged masks, rows with no visible slot, tpos from 1 to
    about 2^46, flat rows whose denominators pass 2^34."""
    from idempotent_llm_amd._lib import call
    B, n_q, n_kv, S, cap, seed, lo, hi, extra = DECODE_CASES[name]
    print(f"[decode attention {name}: B={B} n_q={n_q} n_kv={n_kv} S={S}]", flush=True)
    q8, kc, vc, valid, sm, sk, tpos = _prefill_case(B, n_q, n_kv, 1, S - 1, cap, seed, lo, hi,
                                                    **extra)
    want = _prefill_oracle(q8, kc, vc, valid, sm, sk, S - 1)[:, 0]
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    G = n_q // n_kv
    Spad = (S + 15) // 16 * 16
    scratch = (torch.empty(B, n_q, Spad, dtype=torch.int32, device="cuda")
               if G * Spad * 4 > 48 * 1024 else None)
    out = torch.full((B, n_q * 128), -7, dtype=I64, device="cuda")
    kp, vp, table, width, vmask = paged(kc, vc, valid, seed=seed)
    call("detllm_attn_decode", d(q8[:, :, 0]), d(tpos[:, :, 0, 0]), kp, vp, table, width,
         vmask.view(torch.uint8), width * 128, B, S, n_q, n_kv, None, scratch, out, None)
    got = out.cpu().numpy()
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} mismatches, first at {bad[0].tolist()}"


# ------------------------------------------------------ split-S decode kernel

def _split(q8, tpos, kp, vp, table, width, vmask, B, S, n_q, n_kv, chunk, s_dev=None):
    """detllm_attn_decode_split -> its nsplit partial contexts (scratch and
    chunk maxima pre-filled with junk: every entry read must be written)."""
    from idempotent_llm_amd._lib import call
    ns = -(-S // chunk)
    scores = torch.full((B, n_q, ns * chunk), 0x7F7F7F7F, dtype=torch.int32, device="cuda")
    cmax = torch.full((B, n_q, ns), 0x7F7F7F7F, dtype=torch.int32, device="cuda")
    out = torch.full((ns, B, n_q * 128), -7, dtype=I64, device="cuda")
    call("detllm_attn_decode_split", q8, tpos, kp, vp, table, width, vmask.view(torch.uint8),
         width * 128, B, S, n_q, n_kv, s_dev, chunk, scores, cmax, out, None)
    return out


SPLIT_CASES = dict(DECODE_CASES)
# two rows of 4096 slots with ragged masks, one of them dead for its first
# 1000 slots (whole chunks with no visible slot)
SPLIT_CASES["long_ragged"] = (2, 4, 2, 4096, 4096, 15, 29, 34, dict(dead_prefix=1000))


@pytest.mark.parametrize("name", list(SPLIT_CASES))
@pytest.mark.parametrize("chunk", [256, "plan"])
def test_split_decode_vs_oracle(name, chunk):
    """detllm_attn_decode_split: the sum of the chunk partials against the
    oracle composition (the same cases as the one-block decode kernel, plus
    4096-slot ragged rows), at 256-slot chunks and at the planned chunking."""
    from idempotent_llm_amd._lib import attn_split_plan
    B, n_q, n_kv, S, cap, seed, lo, hi, extra = SPLIT_CASES[name]
    if chunk == "plan":
        chunk = attn_split_plan(B, S, n_q, n_kv)[0]
    print(f"[split decode {name}: B={B} n_q={n_q} n_kv={n_kv} S={S} chunk={chunk}]", flush=True)
    q8, kc, vc, valid, sm, sk, tpos = _prefill_case(B, n_q, n_kv, 1, S - 1, cap, seed, lo, hi,
                                                    **extra)
    want = _prefill_oracle(q8, kc, vc, valid, sm, sk, S - 1)[:, 0]
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    kp, vp, table, width, vmask = paged(kc, vc, valid, seed=seed)
    out = _split(d(q8[:, :, 0]), d(tpos[:, :, 0, 0]), kp, vp, table, width, vmask, B, S, n_q,
                 n_kv, chunk)
    got = out.sum(0).cpu().numpy()
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} mismatches, first at {bad[0].tolist()}"


@pytest.mark.parametrize("B,n_q,n_kv,S,s_dev", [
    (8, 16, 8, 4096, None),     # the c4 / long-context shape, planned and forced chunkings
    (8, 16, 8, 4096, 1000),     # device-bounded scan: chunks past 1000 slots contribute 0
    (1, 8, 1, 3000, None),      # G = 8 (chunks within 48 KiB of packed p)
    (3, 4, 4, 700, 700),        # G = 1, ragged last chunk
])
def test_split_decode_equals_one_block_kernel(B, n_q, n_kv, S, s_dev):
    """Random caches, queries and DI-Exp constants: the split partials sum to
    detllm_attn_decode's output for every chunking tried."""
    from idempotent_llm_amd._lib import attn_split_plan, call
    print(f"[split vs one-block decode B={B} n_q={n_q} n_kv={n_kv} S={S} s_dev={s_dev}]",
          flush=True)
    g = torch.Generator().manual_seed(S + B)
    cap = -(-S // 128) * 128
    q8 = torch.randint(-128, 128, (B, n_q, 128), generator=g, dtype=torch.int8).cuda()
    tpos = torch.randint(1, 1 << 22, (B, n_q), generator=g, dtype=I64).cuda()
    tpos[0, 0] = 1 << 40                      # the integer DI-Exp branch
    kc = torch.randint(-128, 128, (B, n_kv, cap, 128), generator=g, dtype=torch.int8)
    vc = torch.randint(-128, 128, (B, n_kv, 128, cap), generator=g, dtype=torch.int8)
    valid = torch.rand(B, cap, generator=g) < 0.7
    kp, vp, table, width, vmask = paged(kc, vc, valid, seed=B)
    sd = None if s_dev is None else torch.tensor([s_dev], dtype=I64, device="cuda")
    G = n_q // n_kv
    Spad = (S + 15) // 16 * 16
    scratch = (torch.empty(B, n_q, Spad, dtype=torch.int32, device="cuda")
               if G * Spad * 4 > 48 * 1024 else None)
    want = torch.empty(B, n_q * 128, dtype=I64, device="cuda")
    call("detllm_attn_decode", q8, tpos, kp, vp, table, width, vmask.view(torch.uint8),
         width * 128, B, S, n_q, n_kv, sd, scratch, want, None)
    chunks = {attn_split_plan(B, S, n_q, n_kv)[0], 256, 384}
    if G * 4096 * 4 <= 48 * 1024:
        chunks.add(4096)
    for ch in sorted(chunks):
        out = _split(q8, tpos, kp, vp, table, width, vmask, B, S, n_q, n_kv, ch, sd)
        assert torch.equal(out.sum(0), want), ch
        if s_dev is not None:
            first_empty = -(-s_dev // ch)
            assert (out[first_empty:] == 0).all()
    assert want.abs().sum().item() > 0


def test_split_decode_argument_errors():
    from idempotent_llm_amd._lib import call
    print("[split decode argument errors]", flush=True)
    B, n_q, n_kv, S = 1, 8, 1, 512
    q8 = torch.zeros(B, n_q, 128, dtype=torch.int8, device="cuda")
    tpos = torch.ones(B, n_q, dtype=I64, device="cuda")
    kc = torch.zeros(B, n_kv, S, 128, dtype=torch.int8)
    vc = torch.zeros(B, n_kv, 128, S, dtype=torch.int8)
    kp, vp, table, width, vmask = paged(kc, vc, torch.ones(B, S, dtype=torch.bool))
    sc = torch.empty(B, n_q, 4096, dtype=torch.int32, device="cuda")
    cm = torch.empty(B, n_q, 16, dtype=torch.int32, device="cuda")
    out = torch.empty(16, B, n_q * 128, dtype=I64, device="cuda")

    def run(chunk):
        call("detllm_attn_decode_split", q8, tpos, kp, vp, table, width,
             vmask.view(torch.uint8), width * 128, B, S, n_q, n_kv, None, chunk, sc, cm, out,
             None)

    with pytest.raises(RuntimeError, match="code -22"):
        run(200)          # not a multiple of the page
    with pytest.raises(RuntimeError, match="code -34"):
        run(2048)         # 8 heads x 2048 slots x 4 bytes of packed p > 48 KiB
    run(256)
    torch.cuda.synchronize()


@pytest.mark.parametrize("T", [100, 257])
def test_prefill_epilogue_kq_estimates(T):
    """The prefill Q/K/V epilogue (rows layout, R > 64) with the K channels'
    divisor estimates precomputed at load (detllm_kq_est) writes the same q8,
    DI-Exp constants and K/V cache bytes as deriving them per element."""
    from idempotent_llm_amd._lib import call
    dims = art.MID
    prm = _layer_params(dims, 3)
    nq, nkv, hd = dims["n_q_heads"], dims["n_kv_heads"], 128
    rnd = torch.Generator().manual_seed(T)
    B, cap = 1, 512
    P = torch.randint(-(1 << 19), 1 << 19, (1, B * T, (nq + 2 * nkv) * hd), generator=rnd,
                      dtype=torch.int32).cuda()
    xm = torch.randint(1 << 15, 1 << 16, (B * T,), generator=rnd, dtype=I64).cuda()
    xk = torch.randint(22, 30, (B * T,), generator=rnd, dtype=I64).cuda()
    pos = torch.arange(T, dtype=I64).cuda()
    common = (prm["q_m"], prm["q_k"], prm["k_m"], prm["k_k"], prm["v_m"], prm["v_k"],
              prm["q_norm_m"], prm["q_norm_k"], prm["k_norm_m"], prm["k_norm_k"], prm["qs_m"],
              prm["qs_k"], prm["kq_m"], prm["kq_k"], prm["ks_m"], prm["ks_k"], prm["vq_m"],
              prm["vq_k"], prm["cos"], prm["sin"], prm["cos"].shape[0])
    est = torch.empty(prm["kq_m"].numel(), 4, dtype=I64, device="cuda")
    call("detllm_kq_est", prm["kq_m"], prm["kq_k"], prm["kq_m"].numel(),
         20 + prm["k_norm_k"], est)
    outs = []
    for e in (None, est):
        q8 = torch.empty(B, nq, T, hd, dtype=torch.int8, device="cuda")
        tpos = torch.empty(B, nq, T, dtype=I64, device="cuda")
        kc, vc, table, width = paged(torch.zeros(B, nkv, cap, hd, dtype=torch.int8),
                                     torch.zeros(B, nkv, hd, cap, dtype=torch.int8), seed=T)
        call("detllm_qkv_epilogue", P, 1, B * T * P.shape[2], B, T, nq, nkv, xm, xk, pos,
             *common, q8, tpos, None, kc, vc, table, width, None, 0, e, None)
        outs.append((q8, tpos, kc, vc))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    assert outs[0][2].abs().sum().item() > 0


@pytest.mark.parametrize("B,T", [(4, 1), (1, 100)])
def test_qkv_epilogue_q_int64_min(B, T):
    """Q quantisation (model.py:317-323: QK smoothing, then quant_i8_pertoken)
    on heads holding a q of exactly INT64_MIN: QK smoothing scale 2^62 on
    channel 0 of every kv head, 1 elsewhere, so channel 0's q = r * 2^62
    wraps to 0, +-2^62 or INT64_MIN while the other channels stay below
    2^43. dyadic.py's head maximum skips the wrapped |INT64_MIN|, so such a
    head's quotients must come from the exact path. The q8 of both the
    one-token (B, T = 1) and the rows (R > 64) layouts against the oracle's
    composition of the same steps (oracle/model.py _qk_head_pipeline)."""
    from idempotent_llm_amd._lib import call
    from oracle import dyadic as ody, ops as oops
    print(f"[qkv epilogue q INT64_MIN B={B} T={T}]", flush=True)
    dims = art.MID
    prm = _layer_params(dims, 4)
    nq, nkv, hd = dims["n_q_heads"], dims["n_kv_heads"], 128
    rnd = torch.Generator().manual_seed(40 + T)
    P = torch.randint(-(1 << 19), 1 << 19, (1, B * T, (nq + 2 * nkv) * hd), generator=rnd,
                      dtype=torch.int32).cuda()
    xm = torch.randint(1 << 15, 1 << 16, (B * T,), generator=rnd, dtype=I64).cuda()
    xk = torch.randint(22, 30, (B * T,), generator=rnd, dtype=I64).cuda()
    pos = torch.randint(0, dims["max_pos"], (B * T,), generator=rnd, dtype=I64).cuda()
    qs = np.ones((nkv, hd), np.int64)
    qs[:, 0] = 1 << 62
    qs_m = torch.from_numpy(qs.reshape(-1)).cuda()
    common = (prm["q_m"], prm["q_k"], prm["k_m"], prm["k_k"], prm["v_m"], prm["v_k"],
              prm["q_norm_m"], prm["q_norm_k"], prm["k_norm_m"], prm["k_norm_k"], qs_m,
              prm["qs_k"], prm["kq_m"], prm["kq_k"], prm["ks_m"], prm["ks_k"], prm["vq_m"],
              prm["vq_k"], prm["cos"], prm["sin"], prm["cos"].shape[0])
    q8 = torch.empty(B, nq, T, hd, dtype=torch.int8, device="cuda")
    tpos = torch.empty(B, nq, T, dtype=I64, device="cuda")
    kc, vc, table, width = paged(torch.zeros(B, nkv, 256, hd, dtype=torch.int8),
                                 torch.zeros(B, nkv, hd, 256, dtype=torch.int8), seed=T)
    call("detllm_qkv_epilogue", P, 1, B * T * P.shape[2], B, T, nq, nkv, xm, xk, pos, *common,
         q8, tpos, None, kc, vc, table, width, None, 0, None, None)
    torch.cuda.synchronize()
    # the oracle's Q steps on the same inputs
    n = lambda t: t.cpu().numpy()
    Pq = n(P)[0][:, :nq * hd].astype(np.int64).reshape(B, T, nq, hd)
    y, _, _ = ody.requant_i32_common(Pq, n(xm).reshape(B, T, 1, 1), n(xk).reshape(B, T, 1, 1),
                                     n(prm["q_m"]).reshape(nq, hd), prm["q_k"], target_bits=16)
    yn, qkk = oops.di_rmsnorm_gamma(y, n(prm["q_norm_m"]), prm["q_norm_k"])
    yn = yn.transpose(0, 2, 1, 3)
    pb = np.broadcast_to(n(pos).reshape(B, 1, T), (B, nq, T))
    yr = oops.apply_int_rope(yn, n(prm["cos"]), n(prm["sin"]), pb)
    with np.errstate(over="ignore"):
        q = yr * np.repeat(qs, nq // nkv, axis=0)[None, :, None, :]
    one = np.ones((B, nq, T, 1), np.int64)
    want, _, _ = ody.quant_i8_pertoken(q, one, np.zeros_like(one) + qkk + prm["qs_k"])
    hit = (q == np.iinfo(np.int64).min).any(axis=-1)
    small = (np.abs(np.where(q == np.iinfo(np.int64).min, 0, q)).max(axis=-1) < (1 << 43))
    assert (hit & small).any()      # some heads take INT64_MIN with a maximum below 2^43
    np.testing.assert_array_equal(n(q8), want)


def _qkv_oracle(P, xm, xk, pos, prm, B, T, nq, nkv):
    """model.py:303-358 on the oracle: q8 and tpos of the Q heads, the K and
    V cache rows (k8, v8 [B, n_kv, T, 128]) of one Q/K/V product."""
    from oracle import dyadic as ody, ops as oops
    n = lambda t: t.cpu().numpy() if torch.is_tensor(t) else np.asarray(t)
    hd, g = 128, nq // nkv
    Pn = n(P)[0].astype(np.int64).reshape(B, T, nq + 2 * nkv, hd)
    xm4, xk4 = n(xm).reshape(B, T, 1, 1), n(xk).reshape(B, T, 1, 1)
    pos = n(pos).reshape(B, T)

    def head_pipeline(Ph, wm, wk, gm, gk, nh):
        y, _, _ = ody.requant_i32_common(Ph, xm4, xk4, n(wm).reshape(nh, hd), wk,
                                         target_bits=16)
        yn, kout = oops.di_rmsnorm_gamma(y, n(gm), gk)
        yn = yn.transpose(0, 2, 1, 3)
        pb = np.broadcast_to(pos[:, None, :], (B, nh, T))
        return oops.apply_int_rope(yn, n(prm["cos"]), n(prm["sin"]), pb), kout

    with np.errstate(over="ignore"):
        yq, qkk = head_pipeline(Pn[:, :, :nq], prm["q_m"], prm["q_k"], prm["q_norm_m"],
                                prm["q_norm_k"], nq)
        q = yq * np.repeat(n(prm["qs_m"]).reshape(nkv, hd), g, axis=0)[None, :, None, :]
        one = np.ones((B, nq, T, 1), np.int64)
        q8, qm, qk = ody.quant_i8_pertoken(q, one, np.zeros_like(one) + qkk + prm["qs_k"])
        ks_m = np.repeat(n(prm["ks_m"]), g).reshape(1, nq, 1, 1)
        ks_k = np.repeat(n(prm["ks_k"]), g).reshape(1, nq, 1, 1)
        sm, sk = ody.norm_scale(qm * ks_m, qk + ks_k)
        tpos = oops.di_exp_tpos(sm, sk)[..., 0]
        yk, _ = head_pipeline(Pn[:, :, nq:nq + nkv], prm["k_m"], prm["k_k"], prm["k_norm_m"],
                              prm["k_norm_k"], nkv)
        k8 = ody.requant_i8_static(yk, 1, 20 + prm["k_norm_k"], 1, 0,
                                   n(prm["kq_m"]).reshape(1, nkv, 1, hd),
                                   n(prm["kq_k"]).reshape(1, nkv, 1, hd))
        v8 = ody.requant_i8_static(Pn[:, :, nq + nkv:], xm4, xk4, n(prm["v_m"]).reshape(nkv, hd),
                                   prm["v_k"], n(prm["vq_m"]).reshape(1, 1, nkv, 1),
                                   n(prm["vq_k"]).reshape(1, 1, nkv, 1))
    return q8, tpos, k8, v8.transpose(0, 2, 1, 3), q


def _plant(prm, variant, nq, nkv):
    """Channel constants that send heads or lanes to the integer routines of
    the Q/K/V epilogue ("ranges"), or every Q head ("gamma"); "none" keeps the
    artifact's (the fp64 paths, with about a third of the Q heads above the
    2^43 maximum)."""
    prm = dict(prm)
    hd = 128
    cl = lambda k: prm[k].clone()
    if variant == "ranges":
        q_m, k_m, v_m, qs_m, kq_m, kq_k = (cl(k) for k in ("q_m", "k_m", "v_m", "qs_m", "kq_m",
                                                           "kq_k"))
        q_m[1 * hd + 5] = 1 << 21               # Q head 1: P w_m beyond the doubles
        k_m[0 * hd + 70] = -(1 << 21)           # K head 0
        v_m[1 * hd + 3] = 1 << 22               # V head 1: one lane per row
        qs_m[2 * hd + 0] = 1 << 15              # Q heads of kv head 2: smoothing too large
        qs_m[3 * hd:4 * hd] = (1 << 14) + 3     # Q heads of kv head 3: maxima near 2^50
        kq_k[4 * hd + 7] = 20 + prm["k_norm_k"] + 20   # K head 4 channel 7: n above 2^49
        kq_m[5 * hd + 9] = 1 << 50              # K head 5 channel 9: divisor above 2^49
        prm.update(q_m=q_m, k_m=k_m, v_m=v_m, qs_m=qs_m, kq_m=kq_m, kq_k=kq_k)
    elif variant == "gamma":
        g = cl("q_norm_m")
        g[9] = 1 << 12                          # every Q head: gamma beyond the doubles
        prm["q_norm_m"] = g
    return prm


@pytest.mark.parametrize("variant", ["none", "ranges", "gamma"])
@pytest.mark.parametrize("B,T", [(4, 1), (2, 40), (1, 100)])
def test_qkv_epilogue_every_path(variant, B, T):
    """The Q/K/V epilogue's exact fp64 paths and their integer fallbacks
    against the oracle (model.py:303-358: _qk_head_pipeline, QK smoothing,
    quant_i8_pertoken, the score scale's tpos, requant_i8_static of K and V),
    in the one-token layout (B, T = 1: one wave per head) and the rows layout
    (R > 64: four rows per wave), with the K divisor estimates derived per
    element and precomputed; zero product heads (the normalisation's zero
    case), rows with a row mantissa beyond 2^40 (V numerators that wrap) and
    the planted channels of _plant. The fused decode kernel writes the same
    cache bytes and attention output as the separate launches."""
    from idempotent_llm_amd._lib import call
    print(f"[qkv epilogue every path {variant} B={B} T={T}]", flush=True)
    dims = art.MID
    nq, nkv, hd = dims["n_q_heads"], dims["n_kv_heads"], 128
    prm = _plant(_layer_params(dims, 6), variant, nq, nkv)
    rnd = torch.Generator().manual_seed(B * 1000 + T)
    R = B * T
    P = torch.randint(-(1 << 19), 1 << 19, (1, R, (nq + 2 * nkv) * hd), generator=rnd,
                      dtype=torch.int32)
    P[0, 0, 9 * hd:10 * hd] = 0                 # Q head 9 of row 0: a zero head
    P[0, R - 1, (nq + 6) * hd:(nq + 7) * hd] = 0   # K head 6 of the last row
    P = P.cuda()
    xm = torch.randint(1 << 15, 1 << 16, (R,), generator=rnd, dtype=I64)
    xm[R // 2] = (1 << 40) + 7                  # V numerators of this row wrap
    xm = xm.cuda()
    xk = torch.randint(22, 30, (R,), generator=rnd, dtype=I64).cuda()
    pos = torch.randint(0, dims["max_pos"], (R,), generator=rnd, dtype=I64).cuda()
    want_q8, want_tpos, want_k, want_v, q = _qkv_oracle(P, xm, xk, pos, prm, B, T, nq, nkv)
    big = np.abs(q).max(axis=-1) >= (1 << 43)   # the Q maxima take both quotient forms
    if variant == "ranges" or R >= 64:
        assert big.any() and (~big).any()
    common = (prm["q_m"], prm["q_k"], prm["k_m"], prm["k_k"], prm["v_m"], prm["v_k"],
              prm["q_norm_m"], prm["q_norm_k"], prm["k_norm_m"], prm["k_norm_k"], prm["qs_m"],
              prm["qs_k"], prm["kq_m"], prm["kq_k"], prm["ks_m"], prm["ks_k"], prm["vq_m"],
              prm["vq_k"], prm["cos"], prm["sin"], prm["cos"].shape[0])
    est = torch.empty(prm["kq_m"].numel(), 4, dtype=I64, device="cuda")
    call("detllm_kq_est", prm["kq_m"], prm["kq_k"], prm["kq_m"].numel(),
         20 + prm["k_norm_k"], est)
    cap = 128
    for e in (None, est):
        q8 = torch.full((B, nq, T, hd), 99, dtype=torch.int8, device="cuda")
        tpos = torch.full((B, nq, T), -1, dtype=I64, device="cuda")
        kc, vc, table, width = paged(torch.zeros(B, nkv, cap, hd, dtype=torch.int8),
                                     torch.zeros(B, nkv, hd, cap, dtype=torch.int8), seed=T)
        call("detllm_qkv_epilogue", P, 1, R * P.shape[2], B, T, nq, nkv, xm, xk, pos, *common,
             q8, tpos, None, kc, vc, table, width, None, 0, e, None)
        torch.cuda.synchronize()
        k, v = unpaged(kc, vc, table, T)
        np.testing.assert_array_equal(q8.cpu().numpy(), want_q8)
        np.testing.assert_array_equal(tpos.cpu().numpy(), want_tpos)
        np.testing.assert_array_equal(k.cpu().numpy(), want_k)
        np.testing.assert_array_equal(v.cpu().numpy(), want_v)
    if T == 1:
        # the fused decode kernel (Q/K/V epilogue + attention) on the same
        # product, against the separate launches over a random cache
        slot, S = 50, 51
        k0 = torch.randint(-128, 128, (B, nkv, cap, hd), generator=rnd, dtype=torch.int8)
        v0 = torch.randint(-128, 128, (B, nkv, hd, cap), generator=rnd, dtype=torch.int8)
        valid = torch.ones(B, cap, dtype=torch.bool)
        k0, v0, table, width, valid = paged(k0, v0, valid, seed=3)
        vbytes = valid.view(torch.uint8)
        ka, va = k0.clone(), v0.clone()
        q8 = torch.empty(B, nq, 1, hd, dtype=torch.int8, device="cuda")
        tpos = torch.empty(B, nq, 1, dtype=I64, device="cuda")
        out_a = torch.empty(B, nq * hd, dtype=I64, device="cuda")
        call("detllm_qkv_epilogue", P, 1, R * P.shape[2], B, 1, nq, nkv, xm, xk, pos, *common,
             q8, tpos, None, ka, va, table, width, None, slot, None, None)
        call("detllm_attn_decode", q8, tpos, ka, va, table, width, vbytes, width * 128, B, S,
             nq, nkv, None, None, out_a, None)
        kb, vb = k0.clone(), v0.clone()
        out_b = torch.empty(B, nq * hd, dtype=I64, device="cuda")
        call("detllm_qkv_attn_decode", P, 1, R * P.shape[2], B, nq, nkv, xm, xk, pos, *common,
             kb, vb, table, width, None, slot, vbytes, width * 128, S, None, None, out_b, None)
        torch.cuda.synchronize()
        assert torch.equal(ka, kb) and torch.equal(va, vb) and torch.equal(out_a, out_b)
        k, v = unpaged(ka, va, table, S)
        np.testing.assert_array_equal(k[:, :, slot].cpu().numpy(), want_k[:, :, 0])
        np.testing.assert_array_equal(v[:, :, slot].cpu().numpy(), want_v[:, :, 0])
