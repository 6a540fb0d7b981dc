"""Write the config-c3 chain-hash fixture from the CPU oracle.

Config c3 is the full Qwen3-0.6B-shaped model (random-init artifact, seed 3)
decoding 512 greedy steps (one prefill + 511 decodes) from a 64-token prompt
(seed 30), at batch 1, at batch 8 (the prompt plus 7 seeded co-prompts,
right-padded, as scripts/demo.py:113-124 builds its b8 config) and in the
"split" form (prefill the first 32 tokens, feed tokens 32..63 one at a time,
then generate; scripts/demo.py:125-155).

The oracle (``oracle.model.IntQwen3Oracle``) is the line-by-line numpy
restatement of the reference's CPU path, pinned by the reference-written
model goldens; this script only runs it at full size, which takes minutes,
so the GPU tests can compare every step of every row with it.

Written: ``c3_chains.json`` with, per config and row, the greedy tokens, the
demo chain hashes (scripts/demo.py:58-75 byte format) of the logits rows and
of the tokens at every step, and the artifact digest.

    python tests/golden/make_c3_fixture.py [--steps 512] [--out tests/golden/c3_chains.json]
"""

from __future__ import annotations

import argparse
import json
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

PROMPT_SEED, PROMPT_LEN, CO_SEED, ARTIFACT_SEED = 30, 64, 31, 3


def _chains(tokens, rows):
    lc, tc = HashChain(), HashChain()
    for t, r in zip(tokens, rows):
        tc.update_token(int(t))
        lc.update_logits(r)
    return {"tokens": [int(t) for t in tokens], "logit_chain": lc.steps,
            "token_chain": tc.steps}


def run(steps: int, out: str):
    V = art.QWEN3_0_6B["vocab"]
    res = {"config": "c3", "steps": steps, "artifact_seed": ARTIFACT_SEED,
           "prompt_seed": PROMPT_SEED, "prompt_len": PROMPT_LEN, "co_prompt_seed": CO_SEED}
    with tempfile.TemporaryDirectory() as d:
        t0 = time.time()
        art.make_artifact(d, art.QWEN3_0_6B, seed=ARTIFACT_SEED)
        res["artifact_sha256"] = art.artifact_digest(d)
        print(f"artifact {time.time() - t0:.1f}s", flush=True)
        o = IntQwen3Oracle(d)
        p0 = art.prompt_ids(PROMPT_SEED, PROMPT_LEN, V)

        t0 = time.time()
        toks, lg = o.generate(p0[None], steps)
        res["b1"] = _chains(toks[0], [r[0] for r in lg])
        print(f"b1 {time.time() - t0:.1f}s", flush=True)

        t0 = time.time()
        ids, valid = art.right_pad([p0] + art.co_prompts(CO_SEED, 7, V))
        res["b8_ids_shape"] = list(ids.shape)
        res["b8_lens"] = [int(x) for x in valid.sum(axis=1)]
        toks, lg = o.generate(ids, steps, chunk_valid=valid)
        res["b8"] = [_chains(toks[r], [x[r] for x in lg]) for r in range(ids.shape[0])]
        print(f"b8 {time.time() - t0:.1f}s", flush=True)

        # split: prefill half, then the rest token by token, then greedy steps
        t0 = time.time()
        half = PROMPT_LEN // 2
        pos = np.arange(half, dtype=np.int64)[None]
        logits, _, _, cache = o.forward(p0[None, :half], pos)
        last = logits[:, -1]
        for t in range(half, PROMPT_LEN):
            lgt, _, _, cache = o.forward(p0[None, t:t + 1], np.array([[t]], np.int64), cache)
            last = lgt[:, 0]
        rows = [last[0]]
        cur = o.greedy_pick(last)
        tk = [int(cur[0])]
        for step in range(1, steps):
            lgt, _, _, cache = o.forward(cur[:, None], np.array([[PROMPT_LEN + step - 1]]),
                                         cache, np.ones((1, 1), dtype=bool))
            rows.append(lgt[0, 0])
            cur = o.greedy_pick(lgt[:, 0])
            tk.append(int(cur[0]))
        res["split"] = _chains(tk, rows)
        print(f"split {time.time() - t0:.1f}s", flush=True)
    with open(out, "w") as f:
        json.dump(res, f)
    print(f"wrote {out}")


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--out", default=os.path.join(HERE, "c3_chains.json"))
    a = ap.parse_args()
    run(a.steps, a.out)
