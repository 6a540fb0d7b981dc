"""Determinism harness on the rocm backend (scripts/demo.py:101-164, 248-330).

One prompt, several execution configurations, one chain hash. The configs
mirror the reference's int8 ones with the backend renamed:

  int8-rocm-b1     batch 1, graph-captured decode
  int8-rocm-b8     the prompt plus 7 seeded co-prompts, right-padded; row 0
                   is hashed (``all_rows=True`` hashes every row)
  int8-rocm-split  prefill of the first half of the prompt, the rest token by
                   token, then graph-captured decode

Hashes follow scripts/demo.py:58-75 (``hashchain.HashChain``): the logits
row of every step as little-endian int32 bytes, the tokens as 8 little-endian
bytes, checkpoints at 64/128/256/512 steps. Steps run back to back on the
device: the greedy pick is captured in the step graph
(``GraphedDecode.step_greedy``), each step's logits row and token are copied
into device staging buffers, and the host reads them once, after the last
step, to hash them. ``detllm_logits_digest`` gives a 64-bit on-device digest
per row for comparisons that need no host copy.

There is no tokenizer offline: the prompt is 64 seeded ids in [100, 50000)
(``artifact.prompt_ids(30, 64, vocab)``) unless one is passed in.

    python -m idempotent_llm_amd.demo --artifact DIR [--config int8-rocm-b8] [--steps 512]
"""

from __future__ import annotations

import argparse
import time

import numpy as np
import torch

from . import artifact as art
from ._lib import call
from .hashchain import CHECKPOINTS, HashChain

PROMPT_TOKENS = 64
CONFIGS = ("int8-rocm-b1", "int8-rocm-b8", "int8-rocm-split")
I64 = torch.int64


def logits_digest(rows: torch.Tensor) -> torch.Tensor:
    """64-bit digest of each int32 row [R, V] on the device (uint64 values
    carried in an int64 tensor): the wrapping sum over i of
    splitmix64_mix((i << 32) | (uint32) x_i). Equal rows give equal digests;
    the sum is order-independent, so the reduction tree cannot change it."""
    r = rows.contiguous()
    R, V = r.shape
    out = torch.empty(R, dtype=I64, device=r.device)
    call("detllm_logits_digest", r, R, V, out)
    return out


def _chains(tokens: np.ndarray, rows: np.ndarray):
    tc, lc = HashChain(), HashChain()
    for t, r in zip(tokens, rows):
        tc.update_token(int(t))
        lc.update_logits(r)
    for c in (tc, lc):      # the final step is always a checkpoint (demo.py:254-256)
        c.at.setdefault(len(c.steps), c.h.hex()[:16])
    return tc, lc


def run_int8(model, config: str, steps: int, prompt: np.ndarray | None = None,
             co_prompts: list | None = None, all_rows: bool = False):
    """scripts/demo.py:101-164 on the rocm runtime. Returns (token_chain,
    logit_chain) of row 0, or lists of them per row with ``all_rows``."""
    if config not in CONFIGS:
        raise ValueError(f"unknown config {config!r}; expected one of {CONFIGS}")
    dev = model.device
    V = model.vocab
    if prompt is None:
        prompt = art.prompt_ids(30, PROMPT_TOKENS, V)
    prompt = np.asarray(prompt, dtype=np.int64)
    from .graphed import GraphedDecode
    if config.endswith("b8"):
        if co_prompts is None:
            co_prompts = art.co_prompts(31, 7, V)
        ids, valid = art.right_pad([prompt] + list(co_prompts))
        ids_g, valid_g = torch.from_numpy(ids).to(dev), torch.from_numpy(valid).to(dev)
        B, T = ids.shape
        pos = torch.arange(T, device=dev).expand(B, T)
        lens = valid_g.sum(dim=1)
        first, _, _, cache = model._forward(ids_g, pos, None, valid_g, (lens - 1).clamp(min=0))
    else:
        B = 1
        T = len(prompt)
        ids_g = torch.from_numpy(prompt).to(dev)[None]
        if config.endswith("split"):
            half = T // 2
            pos = torch.arange(half, device=dev)[None]
            lg, _, _, cache = model.forward(ids_g[:, :half], pos)
            first = lg[:, -1]
            for t in range(half, T):
                lg, _, _, cache = model.forward(ids_g[:, t:t + 1],
                                                torch.full((1, 1), t, device=dev), cache)
                first = lg[:, 0]
        else:
            pos = torch.arange(T, device=dev)[None]
            first, _, _, cache = model._forward(ids_g, pos, None, None,
                                                torch.full((1,), T - 1, device=dev))
        lens = torch.full((1,), T, dtype=I64, device=dev)
    keep = B if all_rows else 1
    stage_l = torch.empty(steps, keep, V, dtype=torch.int32, device=dev)
    stage_t = torch.empty(steps, keep, dtype=I64, device=dev)
    cur = model.greedy_pick(first)
    stage_l[0].copy_(first[:keep])
    stage_t[0].copy_(cur[:keep])
    if steps > 1:
        gd = GraphedDecode(model, cache, lens)
        nxt = gd.step_greedy(cur)
        for i in range(1, steps):
            stage_l[i].copy_(gd.out_pick[:keep, 0])
            stage_t[i].copy_(nxt[:keep])
            if i + 1 < steps:
                nxt = gd.step_greedy()
    model.raise_if_device_error()
    toks = stage_t.cpu().numpy()
    rows = stage_l.cpu().numpy()
    chains = [_chains(toks[:, r], rows[:, r]) for r in range(keep)]
    if all_rows:
        return [c[0] for c in chains], [c[1] for c in chains]
    return chains[0]


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--artifact", required=True, help="artifact directory (reference schema)")
    ap.add_argument("--config", choices=CONFIGS, help="run one configuration")
    ap.add_argument("--steps", type=int, default=512)
    a = ap.parse_args(argv)
    from .model import IntQwen3
    m = IntQwen3(a.artifact, backend="rocm")
    print(f"artifact sha256: {art.artifact_digest(a.artifact)[:16]}")
    print(f"hardware: GPU={torch.cuda.get_device_name(0)} | torch {torch.__version__}\n")
    for cfg in ([a.config] if a.config else CONFIGS):
        t0 = time.perf_counter()
        tc, lc = run_int8(m, cfg, a.steps)
        dt = time.perf_counter() - t0
        print(f"{cfg}  ({a.steps} tokens, {dt:.1f}s)")
        for n in sorted(lc.at):
            print(f"  @{n:<4} tokens {tc.at[n]}   logits {lc.at[n]}")


if __name__ == "__main__":
    main()
