"""Write the config-c4 prefix fixture from the CPU oracle.

Config c4 is the full Qwen3-0.6B-shaped model (random-init artifact, seed 3)
on 32 prompts of seeded lengths in [16, 1024] (seed 4, ids in [100, 50000)),
right-padded into one batch (scripts/demo.py:113-124 builds its batches the
same way), prefilled, then decoded greedily. The full run (decode until the
cache holds 4096 slots) would take the CPU oracle days; this fixture covers
its prefix: the prefill and the first STEPS - 1 decodes of every row.

The oracle computes each row on its own (batch 1, the prompt at its own
length, no padding), in parallel worker processes: the reference's batching
contract (model.py:8-17, tests/test_determinism.py:71-93) makes a row's
logits independent of the batch around it, so these are the rows the padded
batch of 32 must produce, and the GPU test, which runs the padded batch,
checks parity and batch invariance at once.

The oracle (``oracle.model.IntQwen3Oracle``) is the line-by-line numpy
restatement of the reference's CPU path, pinned by the reference-written
model goldens. Decoding follows generate() (model.py:492-531): the first
token is the greedy pick of each row's logits at its last valid position,
decode step s feeds it at position len + s - 1.

Written: ``c4_prefix.json`` with the prompt lengths, the padded length and,
per row, the greedy tokens and the demo chain hashes (scripts/demo.py:58-75
byte format) of the logits rows and of the tokens at every step.

    python tests/golden/make_c4_fixture.py [--steps 8] [--workers 4] [--out tests/golden/c4_prefix.json]
"""

from __future__ import annotations

import argparse
import json
import multiprocessing as mp
import os
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from idempotent_llm_amd import artifact as art  # noqa: E402
from idempotent_llm_amd.hashchain import HashChain  # noqa: E402
from oracle.model import IntQwen3Oracle  # noqa: E402

ARTIFACT_SEED, INPUT_SEED, BATCH = 3, 4, 32


def c4_prompts():
    lens = art.uniform_int(INPUT_SEED, "c4.lens", (BATCH,), 16, 1025)
    return [art.uniform_int(INPUT_SEED, f"c4.prompt.{i}", (int(n),), 100, 50000)
            for i, n in enumerate(lens)]


def _row(args):
    d, b, prompt, steps = args
    o = IntQwen3Oracle(d)
    t0 = time.time()
    L = len(prompt)
    toks, rows = o.generate(prompt[None], steps)
    lc, tc = HashChain(), HashChain()
    for s in range(steps):
        tc.update_token(int(toks[0, s]))
        lc.update_logits(rows[s][0])
    print(f"row {b} (len {L}) {time.time() - t0:.1f}s", flush=True)
    return b, {"tokens": [int(t) for t in toks[0]], "logit_chain": lc.steps,
               "token_chain": tc.steps}


def run(steps: int, out: str, workers: int):
    prompts = c4_prompts()
    ids, _ = art.right_pad(prompts)
    res = {"config": "c4", "steps": steps, "artifact_seed": ARTIFACT_SEED,
           "input_seed": INPUT_SEED, "lens": [len(p) for p in prompts],
           "padded_len": int(ids.shape[1]), "rows_computed": "each row alone (batch 1)"}
    with tempfile.TemporaryDirectory() as d:
        t0 = time.time()
        art.make_artifact(d, art.QWEN3_0_6B, seed=ARTIFACT_SEED)
        res["artifact_sha256"] = art.artifact_digest(d)
        print(f"artifact {time.time() - t0:.1f}s", flush=True)
        order = sorted(range(BATCH), key=lambda b: -len(prompts[b]))   # longest first
        jobs = [(d, b, prompts[b], steps) for b in order]
        rows = {}
        with mp.get_context("spawn").Pool(workers) as pool:
            for b, rec in pool.imap_unordered(_row, jobs):
                rows[b] = rec
    res["rows"] = [rows[b] for b in range(BATCH)]
    with open(out, "w") as f:
        json.dump(res, f)
    print(f"wrote {out}")


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=8)
    ap.add_argument("--out", default=os.path.join(HERE, "c4_prefix.json"))
    ap.add_argument("--workers", type=int, default=4)
    a = ap.parse_args()
    run(a.steps, a.out, a.workers)
