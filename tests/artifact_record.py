"""A comparable record of an integer artifact directory: per tensor its
dtype, shape and the SHA-256 of its bytes (plus the values of int64
tensors), and the config.json contents."""

import hashlib
import json
import os

import numpy as np


def describe(out_dir: str) -> dict:
    from safetensors.numpy import load_file
    t = load_file(os.path.join(out_dir, "model.safetensors"))
    tensors = {}
    for name in sorted(t):
        a = np.ascontiguousarray(t[name])
        rec = {"dtype": str(a.dtype), "shape": list(a.shape),
               "sha256": hashlib.sha256(a.tobytes()).hexdigest()}
        if a.dtype == np.int64:
            rec["values"] = a.reshape(-1).tolist()
        tensors[name] = rec
    with open(os.path.join(out_dir, "config.json")) as f:
        config = json.load(f)
    return {"config": config, "tensors": tensors}


def differences(got: dict, want: dict) -> list:
    """Names of the tensors / config keys that differ (empty when equal)."""
    out = []
    for name in sorted(set(got["tensors"]) | set(want["tensors"])):
        g, w = got["tensors"].get(name), want["tensors"].get(name)
        if g != w:
            out.append(name)
    for key in sorted(set(got["config"]) | set(want["config"])):
        if got["config"].get(key) != want["config"].get(key):
            out.append("config." + key)
    return out
