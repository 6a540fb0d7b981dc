"""Decode throughput of the integer Qwen3-0.6B-shaped forward pass on one MI355X.

Usage: python bench.py [--gpus 1] [--steps 64] [--warmup 10] [--no-cpu]

Workload (the configuration the headline metric is quoted on): the full
Qwen3-0.6B-shaped random-init integer artifact (28 layers, hidden 1024,
16q/8kv x 128, FFN 3072, vocab 151936; seed 3), seeded random prompts of 128
ids in [100, 50000), greedy decode through the graph-captured step, timed as
the reference's scripts/bench.py:31-43 does: 10 warm-up steps, then K steps,
tok/s = B * K / seconds. A "step" is one decode step of the whole batch
(graph replay of 28 layers + LM head, then the on-device greedy pick).

``value`` is batch-8 decode tok/s; batch 1, prefill (2048 tokens) and the
int8 GEMM TOPS at the prefill shapes are reported beside it. ``roofline``
describes the kernel that dominates the decode step (the skinny int8 GEMM
``k_gemv_nt``): algorithmic bytes per launch (weights + activations + int32
outputs) over its average launch duration, timed with HIP events on the
stream it runs on. ``cpu_baseline`` times the numpy CPU restatement of the
reference path (``oracle/``) on this host for a few decode steps.
"""

from __future__ import annotations

import argparse
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
A100_B8_TOKS = 783.3           # reference's published A100 batch-8 decode tok/s
PROMPT_LEN = 128
PREFILL_LEN = 2048


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _prompts(B: int, T: int, vocab: int):
    import numpy as np
    from idempotent_llm_amd import artifact as art
    rows = [art.prompt_ids(30 + b, T, vocab) for b in range(B)]
    return np.stack(rows)


def decode_bench(model, B: int, steps: int, warmup: int):
    """Reference methodology (scripts/bench.py:31-43) on the rocm backend.
    Returns (tok/s, ms/step, tokens [B, steps])."""
    import torch
    from idempotent_llm_amd.graphed import GraphedDecode
    ids = torch.from_numpy(_prompts(B, PROMPT_LEN, model.vocab)).cuda()
    pos = torch.arange(PROMPT_LEN, device="cuda").expand(B, PROMPT_LEN)
    lens = torch.full((B,), PROMPT_LEN, dtype=torch.int64, device="cuda")
    logits, _, _, cache = model.forward(ids, pos)
    gd = GraphedDecode(model, cache, lens)
    # the greedy pick runs inside the captured step (GraphedDecode.step_greedy:
    # the same tokens and logits as greedy_pick(step(cur)))
    gd.step_greedy(model.greedy_pick(logits[:, -1]))
    for _ in range(warmup - 1):
        gd.step_greedy()
    torch.cuda.synchronize()
    toks = torch.empty(steps, B, dtype=torch.int64, device="cuda")  # rows: contiguous copies
    t0 = time.perf_counter()
    for i in range(steps):
        toks[i] = gd.step_greedy()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return B * steps / dt, 1e3 * dt / steps, toks.t().cpu()


def prefill_bench(model, T: int):
    import torch
    ids = torch.from_numpy(_prompts(1, T, model.vocab)).cuda()
    pos = torch.arange(T, device="cuda")[None]
    model.forward(ids, pos)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    model.forward(ids, pos)
    torch.cuda.synchronize()
    return T / (time.perf_counter() - t0)


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
    """The decode step's skinny GEMMs (q|k|v, o, gate|up, down per layer and
    the LM head) with the model's own weights and K splits, on random int8
    activations: [(x, w, out, ksplit)], and their algorithmic bytes."""
    import torch
    dev = "cuda"
    H, I_ = model.hidden, model.inter
    nqd = model.n_q * model.hd
    x_h = torch.randint(-127, 128, (B, H), dtype=torch.int8, device=dev)
    x_a = torch.randint(-127, 128, (B, nqd), dtype=torch.int8, device=dev)
    x_i = torch.randint(-127, 128, (B, I_), dtype=torch.int8, device=dev)
    jobs = []
    for L in model.layers:
        for x, w in ((x_h, L.wqkv), (x_a, L.wo), (x_h, L.wgu), (x_i, L.wd)):
            N, K = w.shape
            ks = model._ksplit(N, K)
            jobs.append((x, w, torch.empty(ks, B, N, dtype=torch.int32, device=dev), ks))
    N, K = model.head_w.shape
    jobs.append((x_h, model.head_w, torch.empty(1, B, N, dtype=torch.int32, device=dev), 1))
    nbytes = sum(w.numel() + x.numel() + 4 * B * w.shape[0] for x, w, _, _ in jobs)
    return jobs, nbytes


def _traffic():
    """HBM bytes per skinny-GEMM launch measured by rocprofv3 FETCH_SIZE and
    WRITE_SIZE passes over `bench.py --kernel-probe` (profiles/), or None."""
    path = os.path.join(ROOT, "profiles", "gemv_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        rec = json.load(f)
    return rec.get("bytes_per_launch")


def gemv_roofline(model, B: int):
    """Algorithmic bytes per launch / average launch duration of the decode
    step's skinny GEMMs, timed over a graph of the step's launches."""
    from idempotent_llm_amd.backends import gemm_nt
    jobs, nbytes = decode_gemv_jobs(model, B)

    def run():
        for x, w, out, ks in jobs:
            gemm_nt(x, w, out=out, ksplit=ks)

    us = _graph_time_us(run, 20, len(jobs))
    per_launch = nbytes / len(jobs)
    achieved = per_launch / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": _traffic(),
            "kernel": "k_gemv_nt<1,4,2> (LM head: k_gemv_stream)", "batch": B,
            "launches_per_step": len(jobs),
            "bytes_per_launch": int(per_launch), "avg_launch_us": round(us, 3)}


def kernel_probe(model, B: int, reps: int = 3):
    """Eager launches for counter passes (rocprofv3 --pmc): a plain device copy
    of known size (the calibration of FETCH_SIZE / WRITE_SIZE), then the decode
    step's skinny GEMMs."""
    import torch
    from idempotent_llm_amd.backends import gemm_nt
    n = 256 << 20
    src = torch.empty(n, dtype=torch.int8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    jobs, nbytes = decode_gemv_jobs(model, B)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        for x, w, out, ks in jobs:
            gemm_nt(x, w, out=out, ksplit=ks)
    torch.cuda.synchronize()
    log(f"kernel probe: copy {n} B x {reps}, {len(jobs)} GEMV launches x {reps} "
        f"({nbytes / len(jobs):.0f} algorithmic B per launch)")


def c4_decode_bench(model, steps: int = 128, warmup: int = 10):
    """Config c4's batch: 32 prompts of seeded lengths in [16, 1024],
    right-padded, prefill, then graphed decode; tok/s = 32 * steps / s."""
    import torch
    from idempotent_llm_amd import artifact as art
    from idempotent_llm_amd.graphed import GraphedDecode
    lens = art.uniform_int(4, "c4.lens", (32,), 16, 1025)
    prompts = [art.uniform_int(4, f"c4.prompt.{i}", (int(n),), 100, 50000)
               for i, n in enumerate(lens)]
    ids, valid = art.right_pad(prompts)
    B, T = ids.shape
    ids = torch.from_numpy(ids).cuda()
    valid = torch.from_numpy(valid).cuda()
    pos = torch.arange(T, device="cuda").expand(B, T)
    vlens = valid.sum(dim=1)
    # one untimed prefill first (as prefill_bench does): the first one also
    # pays the allocator's growth for the batch-32 caches and activations
    model._forward(ids, pos, None, valid, (vlens - 1).clamp(min=0))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits, _, _, cache = model._forward(ids, pos, None, valid, (vlens - 1).clamp(min=0))
    torch.cuda.synchronize()
    t_pre = time.perf_counter() - t0
    gd = GraphedDecode(model, cache, vlens)
    gd.step_greedy(model.greedy_pick(logits))
    for _ in range(warmup - 1):
        gd.step_greedy()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        gd.step_greedy()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return {"batch": B, "prompt_tokens": int(lens.sum()), "padded_len": T,
            "prefill_s": round(t_pre, 4), "decode_tok_s": round(B * steps / dt, 1),
            "ms_per_step": round(1e3 * dt / steps, 4),
            "slots": [T + warmup, T + warmup + steps]}


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
        call("detllm_swiglu_quant", P1, 1, 0, T, I, xm, xk, gm, 20, gm, 20, ones_i, 0, y8, ym, yk)
        gemm_nt(y8, wd, out=P2)
        call("detllm_residual_normq", P2, 1, 0, T, H, ym, yk, dm, 20, 20, h_work, k_res, None, 0,
             None, None, None)

    us1 = _graph_time_us(mlp, 10, 1)
    ops1 = 2.0 * T * H * I * 3
    return ({"us": round(us1, 2), "gemm_tops": round(ops1 / (us1 * 1e-6) / 1e12, 1),
             "tokens_per_s": round(T / (us1 * 1e-6), 1)}, c2_bench())


def c2_bench():
    """Config c2: one GQA attention prefill launch (2048 queries, 16 q heads,
    8 kv heads, over a 2048-slot cache), device time with HIP events over
    graph replays."""
    import torch
    from idempotent_llm_amd._lib import call
    T = 2048
    dev = "cuda"
    q8 = torch.randint(-127, 128, (1, 16, T, 128), dtype=torch.int8, device=dev)
    tpos = torch.full((1, 16, T), 1 << 12, dtype=torch.int64, device=dev)
    kc = torch.randint(-127, 128, (1, 8, T, 128), dtype=torch.int8, device=dev)
    vc = torch.randint(-127, 128, (1, 8, 128, T), dtype=torch.int8, device=dev)
    valid = torch.ones(1, T, dtype=torch.uint8, device=dev)
    out = torch.empty(1, T, 16 * 128, dtype=torch.int64, device=dev)
    us2 = _graph_time_us(lambda: call("detllm_attn_prefill", q8, tpos, kc, vc, valid, T, 1, T,
                                      0, 16, 8, T, out), 10, 1)
    ops2 = 2.0 * 2 * 16 * (T * (T + 1) // 2) * 128
    return {"us": round(us2, 2), "tops": round(ops2 / (us2 * 1e-6) / 1e12, 1),
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


def cpu_baseline(art_dir: str, steps: int = 3):
    """Decode tok/s of the numpy CPU restatement (oracle/) at batch 1: prefill
    of the 128-token prompt (untimed), then ``steps`` timed decode steps."""
    import numpy as np
    from oracle.model import IntQwen3Oracle
    o = IntQwen3Oracle(art_dir)
    ids = _prompts(1, PROMPT_LEN, o.vocab)
    pos = np.arange(PROMPT_LEN, dtype=np.int64)[None]
    logits, _, _, cache = o.forward(ids, pos)
    cur = o.greedy_pick(logits[:, -1])
    t0 = time.perf_counter()
    for i in range(steps):
        lg, _, _, cache = o.forward(cur[:, None], np.array([[PROMPT_LEN + i]]), cache)
        cur = o.greedy_pick(lg[:, 0])
    dt = time.perf_counter() - t0
    cores = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit():
        cores = min(cores, int(omp))
    return {"value": round(steps / dt, 4), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"batch 1, {steps} decode steps after a {PROMPT_LEN}-token prefill "
                      f"(prefill untimed), full 28-layer model, numpy oracle"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extras", action="store_true",
                    help="decode only (no prefill/GEMM/roofline legs)")
    ap.add_argument("--kernel-probe", action="store_true",
                    help="only launch a known-size copy and the decode GEMVs eagerly "
                         "(for rocprofv3 --pmc counter passes), then exit")
    ap.add_argument("--gemm-probe", action="store_true",
                    help="only time the prefill-shape int8 GEMMs (no model), print them, exit")
    ap.add_argument("--attn-probe", action="store_true",
                    help="only time the c2 attention prefill (no model), print it, exit")
    ap.add_argument("--prefill-probe", action="store_true",
                    help="only time 2048-token prefills of the model, print them, exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}): the integer "
              "forward pass here is built and measured on a single MI355X", file=sys.stderr)
        sys.exit(2)

    import torch
    from idempotent_llm_amd import artifact as art
    from idempotent_llm_amd.model import IntQwen3
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.gemm_probe:
        print(json.dumps(gemm_tops()), flush=True)
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
        B = args.batch
        if args.kernel_probe:
            kernel_probe(model, B)
            return
        tps, ms, toks = decode_bench(model, B, args.steps, args.warmup)
        log(f"decode b{B}: {tps:.1f} tok/s ({ms:.3f} ms/step)")
        tps1, ms1, toks1 = decode_bench(model, 1, args.steps, args.warmup)
        log(f"decode b1: {tps1:.1f} tok/s ({ms1:.3f} ms/step)")
        invariant = bool(torch.equal(toks[0], toks1[0]))
        extras = {}
        roof = None
        if not args.no_extras:
            extras["prefill_tok_s_2048"] = round(prefill_bench(model, PREFILL_LEN), 1)
            log(f"prefill 2048: {extras['prefill_tok_s_2048']} tok/s")
            extras["int8_gemm_prefill"] = gemm_tops()
            log(f"gemm: {extras['int8_gemm_prefill']['all']}")
            roof = gemv_roofline(model, B)
            log(f"roofline: {roof}")
            extras["c4_batch32"] = c4_decode_bench(model)
            log(f"c4: {extras['c4_batch32']}")
            c1, c2 = c1_c2_bench()
            extras["c1_mlp_block_2048"] = c1
            extras["c2_attention_prefill_2048"] = c2
            log(f"c1: {c1} c2: {c2}")
        del model
        torch.cuda.empty_cache()
        cpu = None
        if not args.no_cpu:
            cpu = cpu_baseline(d)
            log(f"cpu baseline: {cpu}")

    line = {
        "metric": "decode tok/s at batch 1/8 + int8 GEMM TOPS (% peak); bit-exact vs CPU",
        "value": round(tps, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": round(tps / A100_B8_TOKS, 3) if B == 8 else None,
        "dtype": "int8", "data": "synthetic (seeded random-init integer artifact and prompts)",
        "config": {"workload": f"c3: Qwen3-0.6B-shaped integer decode, batch {B}, "
                               f"{PROMPT_LEN}-token prompt, hipGraph step + greedy pick",
                   "global_batch": B, "seq_len": PROMPT_LEN, "parallelism": "none (1 GPU)",
                   "vs_baseline_ref": "A100 batch-8 int8 final 783.3 tok/s"},
        "batch1": {"value": round(tps1, 2), "unit": "tok/s", "ms_per_step": round(ms1, 4)},
        "batch_invariant_row0": invariant,
        "roofline": roof,
        "cpu_baseline": cpu,
        **extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
