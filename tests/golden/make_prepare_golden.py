"""Write golden vectors of the reference's offline fitting helpers
(src/detllm/prepare.py:43-115: fit_dyadic_float, quant_weight_per_channel,
quant_embedding_per_row, fit_dyadic_float_vec, fit_gamma_dyadic) on seeded
float inputs, for idempotent_llm_amd.prepare's parity tests.

Run in the build container only (the reference is not present on GPU boxes):

    python tests/golden/make_prepare_golden.py [--ref /root/reference/src]

Writes ``prepare_helpers.npz`` (inputs and outputs). Only these pure
functions are taken from the reference: its prepare() itself needs a Hub
checkpoint, tokenizer and dataset.
"""

from __future__ import annotations

import argparse
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def vectors(P):
    import torch
    g = torch.Generator().manual_seed(7)
    out = {}
    # scalar fits over many magnitudes, including exact powers of two and
    # values whose mantissa rounds up to 2^bits
    s = torch.cat([torch.exp(torch.empty(2000, dtype=torch.float64).uniform_(-30, 30, generator=g)),
                   torch.tensor([1.0, 0.5, 2.0 ** -20, 3.0, (2 ** 16 - 0.25) / 2 ** 20,
                                 (2 ** 16 - 0.5) / 2 ** 16, 1.999999999])])
    fit = np.array([P.fit_dyadic_float(float(v)) for v in s], dtype=np.int64)
    out["fit_s"] = s.numpy()
    out["fit_m"], out["fit_k"] = fit[:, 0], fit[:, 1]
    fit14 = np.array([P.fit_dyadic_float(float(v), 14) for v in s[:500]], dtype=np.int64)
    out["fit14_m"], out["fit14_k"] = fit14[:, 0], fit14[:, 1]
    m, k = P.fit_dyadic_float_vec(s)
    out["vec_m"], out["vec_k"] = m.numpy(), k.numpy()
    # weights: channels of very different magnitude, one all-zero channel
    W = torch.randn(48, 120, generator=g, dtype=torch.float64)
    W = W * torch.exp(torch.empty(48, 1, dtype=torch.float64).uniform_(-6, 3, generator=g))
    W[5] = 0.0
    out["w"] = W.numpy()
    for bits in (8, 16):
        q, m, k = P.quant_weight_per_channel(W.float(), weight_bits=bits)
        out[f"w{bits}_q"], out[f"w{bits}_m"], out[f"w{bits}_k"] = q.numpy(), m.numpy(), np.int64(k)
    E = torch.randn(120, 64, generator=g) * torch.exp(torch.empty(120, 1).uniform_(-5, 2, generator=g))
    out["e"] = E.numpy()
    e8, em, ek = P.quant_embedding_per_row(E)
    out["e8"], out["em"], out["ek"] = e8.numpy(), em.numpy(), ek.numpy()
    gam = torch.randn(128, generator=g) * 0.7 + 0.3
    out["gamma"] = gam.numpy()
    gm, gk = P.fit_gamma_dyadic(gam)
    out["gamma_m"], out["gamma_k"] = gm.numpy(), np.int64(gk)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference/src")
    args = ap.parse_args()
    sys.path.insert(0, args.ref)
    import importlib
    P = importlib.import_module("detllm.prepare")
    np.savez_compressed(os.path.join(HERE, "prepare_helpers.npz"), **vectors(P))
    print("written", os.path.join(HERE, "prepare_helpers.npz"))


if __name__ == "__main__":
    main()
