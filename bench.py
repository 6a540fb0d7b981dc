"""Integer Qwen3-0.6B-shaped forward pass on one MI355X: decode tok/s at
batch 8 / 1 (config c3), int8 GEMM TOPS, and the other benchmark configs.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu] [--no-extras]

Headline (config c3 as configured): the full Qwen3-0.6B-shaped random-init
integer artifact (28 layers, hidden 1024, 16q/8kv x 128, FFN 3072, vocab
151936; seed 3); batch 8 = a 64-token seeded prompt (seed 30) plus 7 seeded
co-prompts (seed 31, 5-39 tokens) right-padded, as scripts/demo.py:113-124
builds its b8 config; one prefill then 511 greedy decode steps through the
graph-captured step with the pick inside the graph (GraphedDecode.step_greedy).
A "step" is one decode step of the whole batch. The K timed steps are the
window of the 511 decodes centred on their mean scanned-slot count (the
decodes scan 65..576 slots, mean 320.5), so a step's cost is the c3 mean;
the untimed steps before the window include the W warm-up steps and the
graph capture. ``c3_full`` times decodes 2..511 of the same run (all of c3
but the capturing first decode) and records the demo checkpoint hashes
(scripts/demo.py:58-75) of row 0 at batch 8 and of batch 1.

``roofline`` is the dominant decode kernel, the skinny int8 GEMM
``k_gemv_dec`` (112 launches per step): algorithmic bytes per launch (weights
+ activations + int32 outputs) over its average launch duration, timed with
HIP events around replays of a graph holding one batch-8 step's 112 launches
(model weights and K splits) on the stream that launches them; ``traffic`` is
the HBM bytes per launch from rocprofv3 FETCH_SIZE / WRITE_SIZE passes
(profiles/decode_traffic.json, with the kernel sources it was measured on).
``roofline_lm_head`` is the same for ``k_gemv_stream``; ``step_hbm`` is the
whole step: bytes a batch-8 c3 step must move over its measured time.
``cpu_baseline`` times the numpy restatement of the reference CPU path
(oracle/) on this host; ``cpu_configs`` gives its wall time per config.
"""

from __future__ import annotations

import argparse
import hashlib
import re
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
I8_PEAK_TOPS = 5000.0          # MI355X dense int8 MFMA, TOP/s
A100_B8_TOKS = 783.3           # reference's published A100 batch-8 decode tok/s (docs/RESULTS.md)
A100_B1_TOKS = 106.3
C3_PROMPT, C3_STEPS = 64, 512  # 64-token prompt; 512 greedy steps = 1 prefill pick + 511 decodes
PREFILL_LEN = 2048


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ------------------------------------------------------------------ c3 decode

def c3_inputs(B: int, vocab: int):
    """Config c3's prompts: the 64-token prompt (seed 30), and at batch 8 the
    7 seeded co-prompts (seed 31), right-padded."""
    import numpy as np
    from idempotent_llm_amd import artifact as art
    p0 = art.prompt_ids(30, C3_PROMPT, vocab)
    if B == 1:
        return p0[None], np.ones((1, len(p0)), dtype=bool)
    assert B == 8, "config c3 is batch 1 or 8"
    return art.right_pad([p0] + art.co_prompts(31, 7, vocab))


def _c3_start(model, B: int):
    """Prefill of the c3 batch, graph capture with the first decode.
    Returns (GraphedDecode, padded prompt length). The cache is planned for
    the whole run up front, as IntQwen3.generate plans it: the decodes then
    only map pages (no pool regrowth, no graph recapture)."""
    import torch
    from idempotent_llm_amd.graphed import GraphedDecode
    from idempotent_llm_amd.kvcache import KVCache
    ids, valid = c3_inputs(B, model.vocab)
    ids = torch.from_numpy(ids).cuda()
    valid = torch.from_numpy(valid).cuda()
    T = ids.shape[1]
    pos = torch.arange(T, device="cuda").expand(B, T)
    lens = valid.sum(dim=1)
    cache = KVCache().plan(model, B, T + C3_STEPS)
    first, _, _, cache = model._forward(ids, pos, cache, valid, (lens - 1).clamp(min=0))
    gd = GraphedDecode(model, cache, lens)
    gd.step_greedy(model.greedy_pick(first))      # decode 1 (captures the step graph)
    return gd, T


def c3_window(model, B: int, steps: int, warmup: int):
    """K = steps timed decodes of c3 centred on the mean scanned-slot count.
    Decode i (1..511) scans T + i slots. Returns a dict."""
    import torch
    gd, T = _c3_start(model, B)
    n_dec = C3_STEPS - 1
    mean_i = (1 + n_dec) / 2.0                     # mean decode index = mean slot count - T
    first = int(round(mean_i - (steps - 1) / 2.0))
    first = max(2 + warmup, min(first, n_dec - steps + 1))   # main() keeps this range non-empty
    for _ in range(2, first):                      # decodes 2 .. first-1: untimed (>= W)
        gd.step_greedy()
    torch.cuda.synchronize()
    toks = torch.empty(steps, B, dtype=torch.int64, device="cuda")
    t0 = time.perf_counter()
    for i in range(steps):
        toks[i] = gd.step_greedy()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    model.raise_if_device_error()
    return {"tok_s": B * steps / dt, "ms_per_step": 1e3 * dt / steps,
            "decodes": [first, first + steps - 1],
            "slots": [T + first, T + first + steps - 1], "untimed_decodes": first - 1}


def c3_full(model, B: int):
    """All of c3 but the capturing first decode: decodes 2..511 timed
    back to back (510 steps), the tokens recorded on the device."""
    import torch
    gd, T = _c3_start(model, B)
    n = C3_STEPS - 2
    toks = torch.empty(n, B, dtype=torch.int64, device="cuda")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(n):
        toks[i] = gd.step_greedy()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    model.raise_if_device_error()
    return {"tok_s": round(B * n / dt, 1), "ms_per_step": round(1e3 * dt / n, 4),
            "timed_decodes": [2, C3_STEPS - 1], "slots": [T + 2, T + C3_STEPS - 1]}


def c3_hashes(model):
    """Demo checkpoint hashes (token and logit chains of row 0) of c3 at
    batch 1 and batch 8 through the determinism harness; untimed."""
    from idempotent_llm_amd.demo import run_int8
    out = {}
    for B in (1, 8):
        tc, lc = run_int8(model, f"int8-rocm-b{B}", C3_STEPS)
        out[f"b{B}"] = {str(n): {"tokens": tc.at[n], "logits": lc.at[n]} for n in sorted(lc.at)}
    out["b8_row0_equals_b1"] = out["b1"] == out["b8"]
    return out


def c3_step_bytes(model, B: int, mean_slots: float) -> float:
    """Bytes one decode step must move (an algorithmic count): every weight
    matrix and LM head once, the per-channel scale vectors, and per row the
    embedding row, the new K/V rows, the int32 logits and the K/V of the
    scanned slots."""
    w = sum(L.wqkv.numel() + L.wo.numel() + L.wgu.numel() + L.wd.numel()
            for L in model.layers) + model.head_w.numel()
    scales = sum(t.numel() * t.element_size()
                 for L in model.layers for t in (L.pf_attn, L.pf_o, L.pf_mlp, L.down_m, L.as_m))
    scales += model.head_m.numel() * 8
    kv_slot = model.n_layers * 2 * model.n_kv * model.hd
    per_row = model.hidden + 16 + kv_slot + 4 * model.vocab + kv_slot * mean_slots
    return float(w + scales + B * per_row)


# ------------------------------------------------------------- roofline legs

def _graph_time_us(fn, reps: int, launches: int) -> float:
    """Average duration of one launch of ``fn``'s kernels: the launches are
    recorded into a HIP graph and the graph replayed ``reps`` times between
    two events on the capturing stream."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            fn()
        g.replay()
        s.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            g.replay()
        e1.record(s)
        e1.synchronize()
    torch.cuda.current_stream().wait_stream(s)
    return 1e3 * e0.elapsed_time(e1) / (reps * launches)


def decode_gemv_jobs(model, B: int):
    """The decode step's skinny GEMMs with the model's own weights and K
    splits on random int8 activations: layer jobs (q|k|v, o, gate|up, down
    per layer: k_gemv_dec) and the LM head (k_gemv_stream)."""
    import torch
    H, I_ = model.hidden, model.inter
    nqd = model.n_q * model.hd
    x_h = torch.randint(-127, 128, (B, H), dtype=torch.int8, device="cuda")
    x_a = torch.randint(-127, 128, (B, nqd), dtype=torch.int8, device="cuda")
    x_i = torch.randint(-127, 128, (B, I_), dtype=torch.int8, device="cuda")
    jobs = []
    for L in model.layers:
        for x, w in ((x_h, L.wqkv), (x_a, L.wo), (x_h, L.wgu), (x_i, L.wd)):
            N, K = w.shape
            ks = model._ksplit(N, K, B)
            jobs.append((x, w, torch.empty(ks, B, N, dtype=torch.int32, device="cuda"), ks))
    head = (x_h, model.head_w, torch.empty(1, B, model.vocab, dtype=torch.int32, device="cuda"),
            1)
    return jobs, head


def _job_bytes(jobs):
    return sum(w.numel() + x.numel() + 4 * x.shape[0] * w.shape[0] for x, w, _, _ in jobs)


def _code_text(src: str) -> str:
    """C++ source without comments and with whitespace collapsed: the part
    that decides the compiled kernels (string literals in these sources hold
    no comment markers)."""
    src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
    src = re.sub(r"//[^\n]*", " ", src)
    return " ".join(src.split())


def _csrc_sha(*names, root: str = ROOT) -> str:
    """Digest of the kernel sources' code (comments and layout excluded)."""
    h = hashlib.sha256()
    for n in names:
        with open(os.path.join(root, "idempotent_llm_amd", "csrc", n), encoding="utf-8") as f:
            h.update(_code_text(f.read()).encode())
    return h.hexdigest()[:16]


def _traffic(kernel: str):
    """HBM bytes per launch of `kernel` measured by rocprofv3 FETCH_SIZE and
    WRITE_SIZE passes over `bench.py --kernel-probe` (profiles/), or None.
    Marked stale when the kernel sources changed since the measurement."""
    path = os.path.join(ROOT, "profiles", "decode_traffic.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        rec = json.load(f)
    k = rec.get("kernels", {}).get(kernel)
    if k is None:
        return None, None
    stale = rec.get("csrc_sha") != _csrc_sha(*rec.get("csrc_files", []))
    src = {"file": "profiles/decode_traffic.json", "measured_at": rec.get("commit"),
           "stale": stale}
    return k["bytes_per_launch"], src


def gemv_rooflines(model, B: int):
    """k_gemv_dec (the layer GEMVs) and k_gemv_stream (LM head), each timed
    over a graph of one decode step's launches of that kernel."""
    from idempotent_llm_amd.backends import gemm_nt
    jobs, head = decode_gemv_jobs(model, B)

    def run(js):
        def f():
            for x, w, out, ks in js:
                gemm_nt(x, w, out=out, ksplit=ks)
        return f

    res = {}
    for name, js, reps in (("k_gemv_dec", jobs, 20), ("k_gemv_stream", [head], 50)):
        us = _graph_time_us(run(js), reps, len(js))
        per = _job_bytes(js) / len(js)
        achieved = per / (us * 1e-6) / 1e9
        traffic, src = _traffic(name)
        res[name] = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "traffic_source": src, "kernel": name, "batch": B,
                     "launches_per_step": len(js), "bytes_per_launch": int(per),
                     "avg_launch_us": round(us, 3),
                     "timing": f"HIP events around {reps} replays of a graph of one batch-{B} "
                               f"decode step's {len(js)} {name} launches"}
    return res["k_gemv_dec"], res["k_gemv_stream"]


def split_attention_case(model, B: int = 32, S: int = 4096, seed: int = 4):
    """The split-S decode attention at config c4's decode shape (B rows
    scanning S slots, the model's head counts) on a random paged cache with
    every slot valid. Returns (launch fn, algorithmic bytes per call, plan):
    the bytes are the K and V bytes scanned, the queries, DI-Exp constants and
    the int64 partial contexts written."""
    import torch
    from idempotent_llm_amd._lib import attn_split_plan, call
    from idempotent_llm_amd.kvcache import pages_from_contiguous
    nq, nkv, hd = model.n_q, model.n_kv, model.hd
    g = torch.Generator(device="cuda").manual_seed(seed)
    kc = torch.randint(-128, 128, (B, nkv, S, hd), device="cuda", dtype=torch.int8, generator=g)
    vc = torch.randint(-128, 128, (B, nkv, hd, S), device="cuda", dtype=torch.int8, generator=g)
    kp, vp, table = pages_from_contiguous(kc, vc, seed=seed)
    del kc, vc
    valid = torch.ones(B, S, dtype=torch.uint8, device="cuda")
    q8 = torch.randint(-128, 128, (B, nq, hd), device="cuda", dtype=torch.int8, generator=g)
    tpos = torch.randint(1, 1 << 22, (B, nq), device="cuda", dtype=torch.int64, generator=g)
    chunk, ns = attn_split_plan(B, S, nq, nkv)
    scores = torch.empty(B, nq, ns * chunk, dtype=torch.int32, device="cuda")
    cmax = torch.empty(B, nq, ns, dtype=torch.int32, device="cuda")
    out = torch.empty(ns, B, nq * hd, dtype=torch.int64, device="cuda")

    def run():
        call("detllm_attn_decode_split", q8, tpos, kp, vp, table, S // 128, valid, S, B, S, nq,
             nkv, None, chunk, scores, cmax, out, None)

    nbytes = 2 * B * nkv * S * hd + q8.numel() + 8 * tpos.numel() + 8 * out.numel()
    return run, nbytes, (chunk, ns)


def split_attention_roofline(model):
    """HBM roofline of the split-S decode attention (its two kernels) at the
    c4 shape, timed over graph replays of one call."""
    run, nbytes, (chunk, ns) = split_attention_case(model)
    us = _graph_time_us(run, 20, 1)
    achieved = nbytes / (us * 1e-6) / 1e9
    t1, src = _traffic("k_attn_split_scores")
    t2, _ = _traffic("k_attn_split_pv")
    traffic = t1 + t2 if t1 and t2 else None
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "traffic_source": src,
            "kernel": "k_attn_split_scores + k_attn_split_pv", "batch": 32, "slots": 4096,
            "chunk": chunk, "nsplit": ns, "bytes_per_call": int(nbytes),
            "avg_call_us": round(us, 3),
            "timing": "HIP events around 20 replays of a graph of one split-S attention call "
                      "(one layer of c4's decode at 4096 slots)"}


def kernel_probe(model, B: int, reps: int = 3):
    """Eager launches for counter passes (rocprofv3 --pmc): a plain device copy
    of known size (the calibration of FETCH_SIZE / WRITE_SIZE), the decode
    step's skinny GEMMs, then eager decode steps of the c3 batch at ~320
    slots (the row kernels and the fused attention)."""
    import torch
    from idempotent_llm_amd.backends import gemm_nt
    n = 256 << 20
    src = torch.empty(n, dtype=torch.int8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    jobs, head = decode_gemv_jobs(model, B)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        for x, w, out, ks in jobs + [head]:
            gemm_nt(x, w, out=out, ksplit=ks)
    torch.cuda.synchronize()
    ids, valid = c3_inputs(B, model.vocab)
    ids = torch.from_numpy(ids).cuda()
    valid = torch.from_numpy(valid).cuda()
    T = ids.shape[1]
    pos = torch.arange(T, device="cuda").expand(B, T)
    _, _, _, cache = model.forward(ids, pos, chunk_valid=valid)
    cur = torch.randint(100, 50000, (B, 1), device="cuda")
    one = torch.ones(B, 1, dtype=torch.bool, device="cuda")
    for i in range(256):                                   # eager decode up to ~320 slots
        if i == 256 - reps:
            torch.cuda.synchronize()
            log("kernel probe: eager decode steps at ~320 slots follow")
        model.forward(cur, torch.full((B, 1), T + i, device="cuda"), cache, one)
    torch.cuda.synchronize()
    # one-row decode steps (the fused-operand GEMVs)
    ids1, valid1 = c3_inputs(1, model.vocab)
    ids1 = torch.from_numpy(ids1).cuda()
    T1 = ids1.shape[1]
    _, _, _, cache1 = model.forward(ids1, torch.arange(T1, device="cuda")[None])
    for i in range(reps):
        model.forward(cur[:1], torch.full((1, 1), T1 + i, device="cuda"), cache1)
    torch.cuda.synchronize()
    del cache, cache1
    # the split-S attention at the c4 shape
    run, nbytes, plan = split_attention_case(model)
    for _ in range(reps):
        run()
    torch.cuda.synchronize()
    log(f"kernel probe: copy {n} B x {reps}, {len(jobs) + 1} GEMV launches x {reps} "
        f"({_job_bytes(jobs) / len(jobs):.0f} algorithmic B per k_gemv_dec launch), "
        f"256 eager decode steps at batch {B}, {reps} at batch 1, split-S attention x {reps} "
        f"(plan {plan}, {nbytes} algorithmic B per call)")


# ------------------------------------------------------------ other configs

def c0_bench():
    """Config c0: A int8 [64, 1024] x W int8 [1024, 3072] (seed 0) then
    requant_i8_static(P, 1, 0, m, 20, 1, 0) to int8, in one launch
    (detllm_igemv_requant_static: the int32 product stays in registers),
    timed over graph replays."""
    import torch
    from idempotent_llm_amd import artifact as art
    from idempotent_llm_amd._lib import call
    M, K, N = 64, 1024, 3072
    A = torch.from_numpy(art.rand_i8(0, "c0.A", (M, K))).cuda()
    Wt = torch.from_numpy(art.rand_i8(0, "c0.W", (K, N)).T.copy()).cuda()
    m = torch.from_numpy(art.uniform_int(0, "c0.m", (N,), 1 << 14, 1 << 15)).cuda()
    y8 = torch.empty(M, N, dtype=torch.int8, device="cuda")

    def run():
        for _ in range(10):
            call("detllm_igemv_requant_static", A, Wt, M, N, K, None, None, m, 20, 1, 0, y8)

    us = _graph_time_us(run, 20, 10)
    ops = 2.0 * M * N * K
    nbytes = M * K + K * N + 4 * N + M * N          # A, W, m as int32, y8 (3,420,160)
    return {"us": round(us, 2), "tops": round(ops / (us * 1e-6) / 1e12, 2),
            "frac_mfma_peak": round(ops / (us * 1e-6) / 1e12 / I8_PEAK_TOPS, 5),
            "hbm_gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
            "frac_hbm_peak": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "algorithmic_bytes": nbytes, "ksplit": 1,
            "kernels": "k_gemv_static (one launch: GEMV + requant_i8_static epilogue)"}


def prefill_bench(model, T: int):
    import torch
    from idempotent_llm_amd import artifact as art
    ids = torch.from_numpy(art.prompt_ids(30, T, model.vocab))[None].cuda()
    pos = torch.arange(T, device="cuda")[None]
    model.forward(ids, pos)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    model.forward(ids, pos)
    torch.cuda.synchronize()
    return T / (time.perf_counter() - t0)


def c4_inputs():
    from idempotent_llm_amd import artifact as art
    lens = art.uniform_int(4, "c4.lens", (32,), 16, 1025)
    prompts = [art.uniform_int(4, f"c4.prompt.{i}", (int(n),), 100, 50000)
               for i, n in enumerate(lens)]
    return prompts


def c4_bench(model, steps: int = 32, end_slots: int = 4096):
    """Config c4: 32 prompts of seeded lengths in [16, 1024], right-padded,
    prefill, then graphed decode until the cache holds `end_slots` slots;
    the last `steps` decodes (the 4096-slot regime) are timed."""
    import torch
    from idempotent_llm_amd import artifact as art
    from idempotent_llm_amd.graphed import GraphedDecode
    prompts = c4_inputs()
    ids, valid = art.right_pad(prompts)
    B, T = ids.shape
    ids = torch.from_numpy(ids).cuda()
    valid = torch.from_numpy(valid).cuda()
    pos = torch.arange(T, device="cuda").expand(B, T)
    vlens = valid.sum(dim=1)
    model._forward(ids, pos, None, valid, (vlens - 1).clamp(min=0))   # allocator warm-up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits, _, _, cache = model._forward(ids, pos, None, valid, (vlens - 1).clamp(min=0))
    torch.cuda.synchronize()
    t_pre = time.perf_counter() - t0
    gd = GraphedDecode(model, cache, vlens)
    gd.step_greedy(model.greedy_pick(logits))               # decode 1: slot T
    n_total = end_slots - T                                 # decodes until end_slots slots
    t_untimed = time.perf_counter()
    for _ in range(n_total - steps - 1):
        gd.step_greedy()
    torch.cuda.synchronize()
    t_untimed = time.perf_counter() - t_untimed
    t0 = time.perf_counter()
    for _ in range(steps):
        gd.step_greedy()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    model.raise_if_device_error()
    slots_end = T + n_total
    kv_slot = model.n_layers * 2 * model.n_kv * model.hd
    mean_slots = slots_end - (steps - 1) / 2.0
    step_bytes = c3_step_bytes(model, B, mean_slots)
    return {"batch": B, "prompt_tokens": int(sum(len(p) for p in prompts)), "padded_len": T,
            "prefill_s": round(t_pre, 4), "decode_tok_s": round(B * steps / dt, 1),
            "ms_per_step": round(1e3 * dt / steps, 4),
            "slots": [slots_end - steps + 1, slots_end],
            "kv_bytes_per_step": int(B * kv_slot * mean_slots),
            "step_hbm_gbs": round(step_bytes / (dt / steps) / 1e9, 1),
            "step_hbm_frac": round(step_bytes / (dt / steps) / 1e9 / HBM_PEAK_GBS, 4),
            "untimed_decodes_s": round(t_untimed, 2)}


def c1_c2_bench():
    """Config c1 (MLP block on 2048 tokens: norm-quant, gate|up GEMM, SwiGLU +
    quant, down GEMM, residual requant) and c2 (GQA attention prefill, 2048
    tokens, 16 q heads) device times with HIP events over graph replays."""
    import torch
    from idempotent_llm_amd import artifact as art
    from idempotent_llm_amd._lib import call
    from idempotent_llm_amd.backends import gemm_nt
    T, H, I = 2048, 1024, 3072
    dev = "cuda"
    h = torch.from_numpy(art.gauss_int(1, "c1.h", (T, H), 1 << 12).astype("int32")).to(dev)
    k_res = torch.full((T,), 24, dtype=torch.int64, device=dev)
    wgu = torch.randint(-127, 128, (2 * I, H), dtype=torch.int8, device=dev)
    wd = torch.randint(-127, 128, (H, I), dtype=torch.int8, device=dev)
    gm = torch.randint(1 << 14, 1 << 15, (I,), dtype=torch.int64, device=dev)
    dm = torch.randint(1 << 14, 1 << 15, (H,), dtype=torch.int64, device=dev)
    ones_h = torch.ones(H, dtype=torch.int64, device=dev)
    ones_i = torch.ones(I, dtype=torch.int64, device=dev)
    x8 = torch.empty(T, H, dtype=torch.int8, device=dev)
    y8 = torch.empty(T, I, dtype=torch.int8, device=dev)
    xm, xk, ym, yk = (torch.empty(T, dtype=torch.int64, device=dev) for _ in range(4))
    P1 = torch.empty(1, T, 2 * I, dtype=torch.int32, device=dev)
    P2 = torch.empty(1, T, H, dtype=torch.int32, device=dev)
    h_work = h.clone()

    def mlp():
        call("detllm_norm_quant", h, T, H, ones_h, 0, x8, xm, xk)
        gemm_nt(x8, wgu, out=P1)
        call("detllm_swiglu_quant", P1, 1, 0, T, I, xm, xk, gm, 20, gm, 20, ones_i, 0, y8, ym, yk,
             None, 0, 0, 0, 0)
        gemm_nt(y8, wd, out=P2)
        call("detllm_residual_normq", P2, 1, 0, T, H, ym, yk, dm, 20, 20, h_work, k_res, None, 0,
             None, None, None, None, 0, 0, 0, 0)

    us1 = _graph_time_us(mlp, 10, 1)
    ops1 = 2.0 * T * H * I * 3
    return ({"us": round(us1, 2), "gemm_tops": round(ops1 / (us1 * 1e-6) / 1e12, 1),
             "frac_mfma_peak": round(ops1 / (us1 * 1e-6) / 1e12 / I8_PEAK_TOPS, 4),
             "tokens_per_s": round(T / (us1 * 1e-6), 1)}, c2_bench())


def c2_bench():
    """Config c2: one GQA attention prefill launch (2048 queries, 16 q heads,
    8 kv heads, over a 2048-slot cache), device time with HIP events over
    graph replays."""
    import torch
    from idempotent_llm_amd._lib import call
    T = 2048
    dev = "cuda"
    from idempotent_llm_amd.kvcache import pages_from_contiguous
    q8 = torch.randint(-127, 128, (1, 16, T, 128), dtype=torch.int8, device=dev)
    tpos = torch.full((1, 16, T), 1 << 12, dtype=torch.int64, device=dev)
    kc = torch.randint(-127, 128, (1, 8, T, 128), dtype=torch.int8, device=dev)
    vc = torch.randint(-127, 128, (1, 8, 128, T), dtype=torch.int8, device=dev)
    kp, vp, table = pages_from_contiguous(kc, vc)
    valid = torch.ones(1, T, dtype=torch.uint8, device=dev)
    out = torch.empty(1, T, 16 * 128, dtype=torch.int64, device=dev)
    us2 = _graph_time_us(lambda: call("detllm_attn_prefill", q8, tpos, kp, vp, table,
                                      table.shape[1], valid, T, 1, T, 0, 16, 8, out), 10, 1)
    ops2 = 2.0 * 2 * 16 * (T * (T + 1) // 2) * 128
    return {"us": round(us2, 2), "tops": round(ops2 / (us2 * 1e-6) / 1e12, 1),
            "frac_mfma_peak": round(ops2 / (us2 * 1e-6) / 1e12 / I8_PEAK_TOPS, 4),
            "algorithmic_ops": int(ops2)}


def gemm_tops(T: int = PREFILL_LEN):
    """int8 GEMM TOP/s at the prefill shapes (T tokens): q|k|v, o, gate|up, down.
    Beside each, the same product through torch._int_mm (hipBLASLt on ROCm, the
    vendor library) on the same inputs, timed the same way, as a yardstick;
    `equal` records that both give the same int32 matrix."""
    import torch
    from idempotent_llm_amd.backends import gemm_nt
    dev = "cuda"
    shapes = {"qkv": (T, 4096, 1024), "o": (T, 1024, 2048), "gate_up": (T, 6144, 1024),
              "down": (T, 1024, 3072)}
    res = {}
    tot_ops = tot_us = 0.0
    for name, (M, N, K) in shapes.items():
        a = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev)
        w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev)
        out = torch.empty(1, M, N, dtype=torch.int32, device=dev)
        def run(a=a, w=w, out=out):
            for _ in range(20):
                gemm_nt(a, w, out=out)

        us = _graph_time_us(run, 10, 20)
        ops = 2.0 * M * N * K
        tops = ops / (us * 1e-6) / 1e12
        res[name] = {"M": M, "N": N, "K": K, "us": round(us, 2), "tops": round(tops, 1),
                     "frac_peak": round(tops / I8_PEAK_TOPS, 4)}
        wt = w.t()
        try:
            ref = torch._int_mm(a, wt)
            def run_vendor(a=a, wt=wt):
                for _ in range(20):
                    torch._int_mm(a, wt)

            vus = _graph_time_us(run_vendor, 10, 20)
            res[name]["vendor_int_mm"] = {"us": round(vus, 2),
                                          "tops": round(ops / (vus * 1e-6) / 1e12, 1),
                                          "equal": bool(torch.equal(out[0], ref))}
        except RuntimeError as e:   # no int8 GEMM in this torch build
            res[name]["vendor_int_mm"] = {"error": str(e)[:120]}
        tot_ops += ops
        tot_us += us
    tops = tot_ops / (tot_us * 1e-6) / 1e12
    res["all"] = {"tops": round(tops, 1), "frac_peak": round(tops / I8_PEAK_TOPS, 4)}
    return res


# ------------------------------------------------------------- CPU baseline

def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _cores() -> int:
    cores = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit():
        cores = min(cores, int(omp))
    return cores


def cpu_baseline(art_dir: str, steps: int = 3):
    """The numpy restatement of the reference CPU path (oracle/) on this host:
    the headline figure (c3 batch-1 decode tok/s: 64-token prompt prefill,
    then `steps` decode steps) and a wall time per config on a bounded sample
    of each."""
    import numpy as np
    from idempotent_llm_amd import artifact as art
    from oracle import dyadic as ody
    from oracle import gemm as ogemm
    from oracle import ops as oops
    from oracle.model import IntQwen3Oracle
    cfg = {}
    # c0: the whole config
    A = art.rand_i8(0, "c0.A", (64, 1024))
    W = art.rand_i8(0, "c0.W", (1024, 3072))
    m = art.uniform_int(0, "c0.m", (3072,), 1 << 14, 1 << 15)
    t0 = time.perf_counter()
    ody.requant_i8_static(ogemm.int_gemm(A, W), 1, 0, m, 20, 1, 0)
    cfg["c0"] = {"s": round(time.perf_counter() - t0, 4), "sample": "whole config"}
    # c1: the whole MLP block on 2048 tokens
    T, H, I = 2048, 1024, 3072
    h = art.gauss_int(1, "c1.h", (T, H), 1 << 12).astype(np.int32)
    Wg, Wu, Wd = (art.rand_i8(1, f"c1.{n}", s) for n, s in
                  (("gate", (H, I)), ("up", (H, I)), ("down", (I, H))))
    gm = art.uniform_int(1, "c1.gate_m", (I,), 1 << 14, 1 << 15)
    dm = art.uniform_int(1, "c1.down_m", (H,), 1 << 14, 1 << 15)
    t0 = time.perf_counter()
    y = oops.di_rmsnorm(h).astype(np.int64)
    x8, xm, xk = ody.quant_i8_pertoken(y, np.ones((T, 1), np.int64), np.full((T, 1), 20))
    g_, ogm, ogk = ody.requant_i32_common(ogemm.int_gemm(x8, Wg), xm, xk, gm, 20, 14)
    u_, oum, ouk = ody.requant_i32_common(ogemm.int_gemm(x8, Wu), xm, xk, gm, 20, 14)
    ys, ym, yk = oops.di_swiglu(g_, ogm, ogk, u_, oum, ouk)
    y8, y8m, y8k = ody.quant_i8_pertoken(ys, ym, yk)
    d, ddm, ddk = ody.requant_i32_common(ogemm.int_gemm(y8, Wd), y8m, y8k, dm, 20, 20)
    ody.residual_add(h, np.full((T, 1), 24), d, ddm, ddk)
    cfg["c1"] = {"s": round(time.perf_counter() - t0, 3), "sample": "whole config (2048 tokens)"}
    # c2: attention prefill, 512 of the 2048 causal query rows' work (first 512 tokens)
    Tq = 512
    q8 = np.clip(art.gauss_int(2, "c2.q", (16, Tq, 128), 32), -127, 127).astype(np.int8)
    k8 = np.clip(art.gauss_int(2, "c2.k", (8, Tq, 128), 32), -127, 127).astype(np.int8)
    v8 = np.clip(art.gauss_int(2, "c2.v", (8, Tq, 128), 32), -127, 127).astype(np.int8)
    causal = np.arange(Tq)[None, :] <= np.arange(Tq)[:, None]
    sm = np.full((Tq, 1), 46341, np.int64)
    sk = np.full((Tq, 1), 26, np.int64)
    t0 = time.perf_counter()
    for hq in range(16):
        sc = ogemm.int_gemm(q8[hq], np.ascontiguousarray(k8[hq // 2].T))
        p = oops.di_softmax(sc, sm, sk, causal)
        ogemm.int_gemm_u16i8(p, v8[hq // 2])
    cfg["c2"] = {"s": round(time.perf_counter() - t0, 3),
                 "sample": f"first {Tq} of 2048 tokens (scores, softmax, P.V; 1/16 of the "
                           "causal pairs)"}
    # c3: batch-1 decode of the full model
    o = IntQwen3Oracle(art_dir)
    ids, _ = c3_inputs(1, o.vocab)
    pos = np.arange(C3_PROMPT, dtype=np.int64)[None]
    t0 = time.perf_counter()
    logits, _, _, cache = o.forward(ids, pos)
    t_pre = time.perf_counter() - t0
    cur = o.greedy_pick(logits[:, -1])
    t0 = time.perf_counter()
    for i in range(steps):
        lg, _, _, cache = o.forward(cur[:, None], np.array([[C3_PROMPT + i]]), cache)
        cur = o.greedy_pick(lg[:, 0])
    dt = time.perf_counter() - t0
    cfg["c3"] = {"s_per_decode_step": round(dt / steps, 3), "prefill_s": round(t_pre, 3),
                 "sample": f"batch 1, 64-token prefill then {steps} decode steps"}
    # c4: a labelled prefix (batch 32, prompts cut to 16 tokens, 1 decode step)
    prompts = [p[:16] for p in c4_inputs()]
    ids4 = np.stack(prompts)
    t0 = time.perf_counter()
    lg4, _, _, c4c = o.forward(ids4, np.broadcast_to(np.arange(16), ids4.shape))
    cur4 = o.greedy_pick(lg4[:, -1])
    o.forward(cur4[:, None], np.full((32, 1), 16), c4c, np.ones((32, 1), dtype=bool))
    cfg["c4"] = {"s": round(time.perf_counter() - t0, 3),
                 "sample": "prefix: batch 32, prompts cut to 16 tokens, prefill + 1 decode step"}
    head = {"value": round(steps / dt, 4), "unit": "tok/s", "cores": _cores(),
            "cpu_model": _cpu_model(), "kind": "port",
            "sample": f"c3 batch 1: {steps} decode steps after the 64-token prefill (prefill "
                      f"untimed), full 28-layer model, numpy oracle"}
    return head, cfg


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extras", action="store_true",
                    help="c3 decode only (no GEMM/roofline/config legs)")
    ap.add_argument("--kernel-probe", action="store_true",
                    help="only launch a known-size copy, the decode GEMVs and eager decode steps "
                         "(for rocprofv3 --pmc counter passes), then exit")
    ap.add_argument("--gemm-probe", action="store_true",
                    help="only time the prefill-shape int8 GEMMs (no model), print them, exit")
    ap.add_argument("--attn-probe", action="store_true",
                    help="only time the c2 attention prefill (no model), print it, exit")
    ap.add_argument("--prefill-probe", action="store_true",
                    help="only time 2048-token prefills of the model, print them, exit")
    ap.add_argument("--roofline-probe", action="store_true",
                    help="only time the decode GEMV graphs of the roofline legs, print, exit")
    ap.add_argument("--split-probe", action="store_true",
                    help="only time the split-S decode attention at the c4 shape, print, exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}): this build "
              "measures the integer forward pass on a single MI355X", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.steps > C3_STEPS - 2 - args.warmup:
        print(f"--steps must be in [1, {C3_STEPS - 2 - args.warmup}] (c3 has {C3_STEPS - 1} "
              "decodes; the first captures the graph)", file=sys.stderr)
        sys.exit(2)

    import torch
    from idempotent_llm_amd import artifact as art
    from idempotent_llm_amd.model import IntQwen3
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.gemm_probe:
        print(json.dumps({"2048": gemm_tops(), "c4": gemm_tops(32 * 1021)}), flush=True)
        return
    if args.attn_probe:
        print(json.dumps({"c2_attention_prefill_2048": c2_bench()}), flush=True)
        return

    with tempfile.TemporaryDirectory(prefix="detllm_bench_") as d:
        t0 = time.perf_counter()
        art.make_artifact(d, art.QWEN3_0_6B, seed=3)
        log(f"artifact generated in {time.perf_counter() - t0:.1f}s")
        model = IntQwen3(d, backend="rocm")
        log("model loaded")
        if args.prefill_probe:
            tps = [round(prefill_bench(model, PREFILL_LEN), 1) for _ in range(3)]
            print(json.dumps({"prefill_tok_s_2048": tps}), flush=True)
            return
        if args.kernel_probe:
            kernel_probe(model, 8)
            return
        if args.roofline_probe:
            r, rs = gemv_rooflines(model, 8)
            print(json.dumps({"roofline": r, "roofline_lm_head": rs}), flush=True)
            return
        if args.split_probe:
            print(json.dumps({"roofline_attn_split": split_attention_roofline(model)}),
                  flush=True)
            return
        w8 = c3_window(model, 8, args.steps, args.warmup)
        log(f"c3 b8: {w8['tok_s']:.1f} tok/s ({w8['ms_per_step']:.3f} ms/step, slots "
            f"{w8['slots']})")
        w1 = c3_window(model, 1, args.steps, args.warmup)
        log(f"c3 b1: {w1['tok_s']:.1f} tok/s ({w1['ms_per_step']:.3f} ms/step)")
        mean_slots = sum(w8["slots"]) / 2.0
        step_bytes = c3_step_bytes(model, 8, mean_slots)
        step_gbs = step_bytes / (w8["ms_per_step"] * 1e-3) / 1e9
        extras = {}
        roof = roof_head = None
        if not args.no_extras:
            extras["c3_full"] = {"b8": c3_full(model, 8), "b1": c3_full(model, 1)}
            log(f"c3 full: {extras['c3_full']}")
            extras["c3_hashes"] = c3_hashes(model)
            log(f"c3 hashes: b8 row 0 == b1: {extras['c3_hashes']['b8_row0_equals_b1']}")
            roof, roof_head = gemv_rooflines(model, 8)
            log(f"roofline: {roof}")
            log(f"roofline LM head: {roof_head}")
            extras["c0_gemm_requant"] = c0_bench()
            log(f"c0: {extras['c0_gemm_requant']}")
            extras["prefill_tok_s_2048"] = round(prefill_bench(model, PREFILL_LEN), 1)
            log(f"prefill 2048: {extras['prefill_tok_s_2048']} tok/s")
            extras["int8_gemm_prefill"] = gemm_tops()
            log(f"gemm: {extras['int8_gemm_prefill']['all']}")
            # the same four products at c4's prefill size (32 rows padded to
            # 1,021 tokens: M = 32,672), where the 256x256 tiles run
            extras["int8_gemm_prefill_c4"] = gemm_tops(32 * 1021)
            log(f"gemm c4: {extras['int8_gemm_prefill_c4']['all']}")
            c1, c2 = c1_c2_bench()
            extras["c1_mlp_block_2048"] = c1
            extras["c2_attention_prefill_2048"] = c2
            log(f"c1: {c1} c2: {c2}")
            extras["c4_batch32"] = c4_bench(model)
            log(f"c4: {extras['c4_batch32']}")
            extras["roofline_attn_split"] = split_attention_roofline(model)
            log(f"split-S attention roofline: {extras['roofline_attn_split']}")
        del model
        torch.cuda.empty_cache()
        cpu = cpu_cfg = None
        if not args.no_cpu:
            cpu, cpu_cfg = cpu_baseline(d)
            log(f"cpu baseline: {cpu} {cpu_cfg}")

    line = {
        "metric": "decode tok/s at batch 1/8 + int8 GEMM TOPS (% peak); bit-exact vs CPU",
        "value": round(w8["tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(w8["ms_per_step"], 4),
        "higher_is_better": True, "scaling": "weak",
        "vs_baseline": round(w8["tok_s"] / A100_B8_TOKS, 3),
        "dtype": "int8", "data": "synthetic (seeded random-init integer artifact and prompts)",
        "config": {"workload": "c3: Qwen3-0.6B-shaped integer decode, batch 8 (64-token prompt + "
                               "7 co-prompts, right-padded), 511 graphed greedy decodes; the "
                               f"{args.steps} timed decodes centred on the mean slot count",
                   "global_batch": 8, "seq_len": C3_PROMPT, "decode_steps": C3_STEPS - 1,
                   "timed_decodes": w8["decodes"], "timed_slots": w8["slots"],
                   "parallelism": "none (1 GPU)",
                   "vs_baseline_ref": "A100 batch-8 int8 final 783.3 tok/s (docs/RESULTS.md)"},
        "batch1": {"value": round(w1["tok_s"], 2), "unit": "tok/s",
                   "ms_per_step": round(w1["ms_per_step"], 4),
                   "vs_a100_b1": round(w1["tok_s"] / A100_B1_TOKS, 3)},
        "step_hbm": {"bytes_per_step": int(step_bytes), "achieved": round(step_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(step_gbs / HBM_PEAK_GBS, 4), "batch": 8,
                     "mean_slots": mean_slots},
        "roofline": roof,
        "roofline_lm_head": roof_head,
        "cpu_baseline": cpu,
        "cpu_configs": cpu_cfg,
        **extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
