"""Write the artifact the reference's offline quantiser makes of a small
random Qwen3 float model, for the bit-level parity test of
idempotent_llm_amd.prepare.prepare (tests/test_prepare.py).

Run in the build container only (the reference is not present on GPU boxes):

    python tests/golden/make_prepare_artifact.py [--ref /root/reference/src]

The reference's prepare() (src/detllm/prepare.py:228-434) fetches its float
model and tokenizer from the Hub and its calibration text from a dataset
(:239-240, :172-174). Here, inside this script only, those three loaders are
replaced by local objects: the model loader returns the seeded small Qwen3 of
tests/floatmodel.py, the tokenizer returns fixed calibration token ids (the
rows of ``calib_ids`` below, concatenated, so the reference's chunking
``ids[s * calib_len:(s + 1) * calib_len]`` yields exactly those rows) and the
dataset is a one-line stand-in the tokenizer ignores. Everything else is the
reference's code as written, run on the CPU with one thread.

Writes ``prepare_artifact.json``: per variant the build options, the
config.json the reference wrote, and per tensor its dtype, shape and the
SHA-256 of its bytes, plus the full values of every int64 tensor (the scale
mantissas and shifts) so a mismatch names the tensor and the channels.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import types

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
CALIB_SEED, CALIB_SHAPE = 5, (4, 64)
# name: (prepare() options, small_float_model() options)
VARIANTS = {
    "default": ({}, {}),
    "no_smoothing_qk_alpha_0p5": ({"smooth_acts": False, "smooth_o": False, "qk_alpha": 0.5},
                                  {}),
    "outlier_channels": ({}, {"outliers": True}),
}


def calib_ids() -> np.ndarray:
    return np.random.default_rng(CALIB_SEED).integers(0, 1000, CALIB_SHAPE, dtype=np.int64)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference/src")
    args = ap.parse_args()
    import torch
    import transformers
    import datasets
    sys.path.insert(0, args.ref)
    sys.path.insert(0, os.path.dirname(HERE))
    from detllm import prepare as ref_prepare
    from artifact_record import describe
    from floatmodel import small_float_model

    torch.set_num_threads(1)
    ids = calib_ids()

    class Tok:
        def __call__(self, text, return_tensors=None):
            return types.SimpleNamespace(input_ids=torch.from_numpy(ids.reshape(1, -1)))

    model_box = {}
    saved = (transformers.AutoTokenizer.from_pretrained,
             transformers.AutoModelForCausalLM.from_pretrained, datasets.load_dataset)
    transformers.AutoTokenizer.from_pretrained = staticmethod(lambda *a, **k: Tok())
    transformers.AutoModelForCausalLM.from_pretrained = staticmethod(
        lambda *a, **k: model_box["m"])
    datasets.load_dataset = lambda *a, **k: {"text": ["(calibration ids are fixed)"]}
    out = {"float_model": "tests/floatmodel.py small_float_model(seed=0, **model_options)",
           "calib_ids": f"numpy default_rng({CALIB_SEED}).integers(0, 1000, {CALIB_SHAPE})",
           "model_id": "test-small-qwen3", "variants": {}}
    try:
        for name, (opts, model_opts) in VARIANTS.items():
            model_box["m"] = small_float_model(seed=0, **model_opts)
            with tempfile.TemporaryDirectory() as d:
                ref_prepare.prepare(d, calib_samples=CALIB_SHAPE[0], calib_len=CALIB_SHAPE[1],
                                    device="cpu", model_id="test-small-qwen3", **opts)
                rec = describe(d)
            rec["options"], rec["model_options"] = opts, model_opts
            out["variants"][name] = rec
            print(name, len(rec["tensors"]), "tensors")
    finally:
        (transformers.AutoTokenizer.from_pretrained,
         transformers.AutoModelForCausalLM.from_pretrained, datasets.load_dataset) = saved
    with open(os.path.join(HERE, "prepare_artifact.json"), "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print("wrote", os.path.join(HERE, "prepare_artifact.json"))


if __name__ == "__main__":
    main()
