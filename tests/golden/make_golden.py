"""Write golden vectors from the reference's CPU ("reference") integer path.

Run in the build container only (the reference is not present on GPU boxes):

    python tests/golden/make_golden.py [--ref /root/reference/src]

What it writes (all small; inputs are stored with the outputs):
  * ``dyadic.npz``  — scaled_round_div, fit_dyadic_ratio, norm_scale,
    quant_i8_pertoken, requant_i32_common, requant_i8_rowcol,
    requant_i8_static, residual_renorm / _from_delta / _add
    (reference src/detllm/dyadic.py:45-206);
  * ``ops.npz``     — di_exp, di_softmax (masks, clip, p_out 15 and 8),
    di_rmsnorm(_gamma), di_swiglu, apply_int_rope and the int16 RoPE tables
    (src/detllm/ops/*.py);
  * ``model_<name>.json`` — for seeded random-init artifacts in the reference
    schema (built by ``idempotent_llm_amd.artifact``): the artifact sha256,
    prefill logits digests, greedy tokens, the demo chain hashes
    (scripts/demo.py:58-75) for batch-1, a right-padded batch and a split
    prefill, and greedy_pick on crafted tie rows (src/detllm/model.py:105-531).

Only functions that no closed form or brute-force check pins are taken from
the reference here; integer primitives and GEMMs are pinned in the tests by
Python ints, ``math.isqrt`` and naive loops instead.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))


def _np(t):
    import torch
    if isinstance(t, torch.Tensor):
        return t.detach().cpu().numpy()
    return np.asarray(t)


def _i64(g, shape, lo, hi):
    import torch
    return torch.randint(lo, hi, shape, generator=g, dtype=torch.int64)


def dyadic_vectors(dy):
    import torch
    I64 = torch.int64
    out = {}
    g = torch.Generator().manual_seed(100)
    # scaled_round_div: both signs of e, signed numerators
    num = _i64(g, (4000,), -(1 << 40), 1 << 40)
    den = _i64(g, (4000,), 1, 1 << 20)
    e = _i64(g, (4000,), -20, 21)
    out["srd_num"], out["srd_den"], out["srd_e"] = _np(num), _np(den), _np(e)
    out["srd_out"] = _np(dy.scaled_round_div(num, den, e))
    # fit_dyadic_ratio: tensor den and scalar 127, incl. powers of two
    num = torch.cat([_i64(g, (4000,), 1, 1 << 40),
                     torch.tensor([1, 2, 3, 127, 254, 1 << 15, (1 << 16) - 1, 1 << 30,
                                   (1 << 46) + 12345, (1 << 52) - 1], dtype=I64)])
    den = torch.cat([_i64(g, (4000,), 1, 1 << 20), torch.full((10,), 127, dtype=I64)])
    m, e = dy.fit_dyadic_ratio(num, den)
    out["fit_num"], out["fit_den"], out["fit_m"], out["fit_e"] = map(_np, (num, den, m, e))
    m, e = dy.fit_dyadic_ratio(num, 127)
    out["fit127_m"], out["fit127_e"] = _np(m), _np(e)
    # norm_scale: growing and shrinking mantissas, rounding-overflow cases
    m = torch.cat([_i64(g, (4000,), 1, 1 << 40),
                   torch.tensor([0, 1, 2, (1 << 15) - 1, 1 << 15, (1 << 16) - 1, 1 << 16,
                                 (1 << 17) - 1, (1 << 17) - 2, (1 << 33) - 1, (1 << 62) - 1],
                                dtype=I64)])
    k = _i64(g, m.shape, 0, 60)
    m2, k2 = dy.norm_scale(m, k)
    out["ns_m"], out["ns_k"], out["ns_m2"], out["ns_k2"] = map(_np, (m, k, m2, k2))
    # quant_i8_pertoken: int32 rows, int64 rows, zero rows
    x = torch.randint(-(1 << 24), 1 << 24, (48, 1024), generator=g, dtype=torch.int32)
    x[5] = 0
    x[7, :] = 3
    xm = _i64(g, (48, 1), 1 << 15, 1 << 16)
    xk = _i64(g, (48, 1), 20, 40)
    q8, qm, qk = dy.quant_i8_pertoken(x, xm, xk)
    out.update(q_x=_np(x), q_m=_np(xm), q_k=_np(xk), q_x8=_np(q8), q_mo=_np(qm), q_ko=_np(qk))
    x = _i64(g, (32, 128), -(1 << 46), 1 << 46)
    xm = _i64(g, (32, 1), 1, 1 << 34)
    xk = _i64(g, (32, 1), 0, 70)
    q8, qm, qk = dy.quant_i8_pertoken(x, xm, xk)
    out.update(q64_x=_np(x), q64_m=_np(xm), q64_k=_np(xk), q64_x8=_np(q8), q64_mo=_np(qm),
               q64_ko=_np(qk))
    # requant_i32_common for each target width used by the model
    P = torch.randint(-(1 << 25), 1 << 25, (40, 512), generator=g, dtype=torch.int32)
    P[3] = 0
    rm = _i64(g, (40, 1), 1 << 15, 1 << 16)
    rk = _i64(g, (40, 1), 10, 40)
    cm = _i64(g, (512,), 1 << 14, 1 << 16)
    out.update(rq_P=_np(P), rq_rm=_np(rm), rq_rk=_np(rk), rq_cm=_np(cm))
    for tb in (12, 14, 16, 20):
        y, m, k = dy.requant_i32_common(P, rm, rk, cm, 24, target_bits=tb)
        out[f"rq{tb}_y"], out[f"rq{tb}_m"], out[f"rq{tb}_k"] = _np(y), _np(m), _np(k)
    # requant_i8_rowcol: int32 P and int64 P large enough to force the pre-shift
    y8, m, k = dy.requant_i8_rowcol(P, rm, rk, cm, 24)
    out.update(rc_y8=_np(y8), rc_m=_np(m), rc_k=_np(k))
    P64 = _i64(g, (24, 2048), -(1 << 40), 1 << 40)
    P64[2] = 0
    cm64 = _i64(g, (2048,), 1 << 14, 1 << 20)
    rm64 = _i64(g, (24, 1), 1, 4)
    rk64 = _i64(g, (24, 1), 0, 20)
    y8, m, k = dy.requant_i8_rowcol(P64, rm64, rk64, cm64, 30)
    out.update(rc64_P=_np(P64), rc64_cm=_np(cm64), rc64_rm=_np(rm64), rc64_rk=_np(rk64),
               rc64_y8=_np(y8), rc64_m=_np(m), rc64_k=_np(k))
    # requant_i8_static: per-(row) and per-(head, channel) target scales,
    # both shift signs
    Ps = torch.randint(-(1 << 24), 1 << 24, (6, 9, 4, 128), generator=g, dtype=torch.int32)
    srm = _i64(g, (6, 9, 1, 1), 1 << 15, 1 << 16)
    srk = _i64(g, (6, 9, 1, 1), 5, 30)
    scm = _i64(g, (4, 128), 1 << 14, 1 << 16)
    ssm = _i64(g, (1, 1, 4, 1), 1 << 15, 1 << 16)
    ssk = _i64(g, (1, 1, 4, 1), 20, 60)
    y8 = dy.requant_i8_static(Ps, srm, srk, scm, 24, ssm, ssk)
    out.update(rs_P=_np(Ps), rs_rm=_np(srm), rs_rk=_np(srk), rs_cm=_np(scm), rs_sm=_np(ssm),
               rs_sk=_np(ssk), rs_y8=_np(y8))
    kk = _i64(g, (2, 4, 7, 128), -(1 << 36), 1 << 36)
    kq_m = _i64(g, (1, 4, 1, 128), 1 << 15, 1 << 16)
    kq_k = _i64(g, (1, 4, 1, 128), 15, 40)
    one = torch.ones(1, dtype=I64)
    krow = torch.tensor(31, dtype=I64)
    y8 = dy.requant_i8_static(kk, one, krow, one, 0, kq_m, kq_k)
    out.update(rsk_x=_np(kk), rsk_m=_np(kq_m), rsk_k=_np(kq_k), rsk_y8=_np(y8))
    y8 = dy.requant_i8_static(P, one, torch.zeros(1, dtype=I64), cm, 20, 1, 0)  # config-0 form
    out["rs0_y8"] = _np(y8)
    # residual stream
    h64 = torch.cat([_i64(g, (16, 256), -(1 << 40), 1 << 40),
                     _i64(g, (16, 256), -(1 << 10), 1 << 10),
                     torch.zeros(2, 256, dtype=I64)])
    kr = _i64(g, (34, 1), -10, 40)
    h, k2 = dy.residual_renorm(h64, kr)
    out.update(rr_h64=_np(h64), rr_k=_np(kr), rr_h=_np(h), rr_k2=_np(k2))
    d = torch.randint(-(1 << 20), 1 << 20, (20, 1024), generator=g, dtype=torch.int32)
    dm = _i64(g, (20, 1), 1 << 15, 1 << 16)
    dk = _i64(g, (20, 1), 20, 50)
    h, k2 = dy.residual_from_delta(d, dm, dk)
    out.update(rf_d=_np(d), rf_dm=_np(dm), rf_dk=_np(dk), rf_h=_np(h), rf_k=_np(k2))
    d2 = torch.randint(-(1 << 20), 1 << 20, (20, 1024), generator=g, dtype=torch.int32)
    dm2 = _i64(g, (20, 1), 1 << 15, 1 << 16)
    dk2 = _i64(g, (20, 1), 20, 50)
    h3, k3 = dy.residual_add(h, k2, d2, dm2, dk2)
    out.update(ra_d=_np(d2), ra_dm=_np(dm2), ra_dk=_np(dk2), ra_h=_np(h3), ra_k=_np(k3))
    return out


def ops_vectors(ops_mod, rope_mod, rms_mod):
    import torch
    I64 = torch.int64
    out = {}
    g = torch.Generator().manual_seed(200)
    # di_exp over a range of per-row scales
    rows = 32
    m = _i64(g, (rows, 1), 1 << 15, 1 << 16)
    k = _i64(g, (rows, 1), 10, 40)
    x = -_i64(g, (rows, 700), 0, 1 << 22)
    x[:, 0] = 0
    res, tpos = ops_mod.di_exp(x, m, k)
    out.update(exp_x=_np(x), exp_m=_np(m), exp_k=_np(k), exp_res=_np(res), exp_tpos=_np(tpos))
    # di_softmax with causal/padding masks, an all-masked row, clip, 8-bit
    sc = torch.randint(-(1 << 21), 1 << 21, (3, 4, 5, 200), generator=g, dtype=torch.int32)
    sm = _i64(g, (3, 4, 5, 1), 1 << 15, 1 << 16)
    sk = _i64(g, (3, 4, 5, 1), 20, 34)
    valid = torch.rand(3, 4, 5, 200, generator=g) < 0.7
    valid[0, 0, 0] = False
    valid[1, 2, 3] = False
    valid[2, 1, :, 100:] = False
    p15 = ops_mod.di_softmax(sc, sm, sk, valid)
    p8 = ops_mod.di_softmax(sc, sm, sk, valid, p_out_bits=8)
    pc = ops_mod.di_softmax(sc, sm, sk, valid, clip_c=15)
    out.update(sm_x=_np(sc), sm_m=_np(sm), sm_k=_np(sk), sm_valid=_np(valid),
               sm_p15=_np(p15), sm_p8=_np(p8), sm_pc15=_np(pc))
    # di_rmsnorm: hidden and head widths, zero / tiny / huge rows
    for n in (1024, 128, 3072):
        xr = torch.randint(-(1 << 29), 1 << 29, (24, n), generator=g, dtype=torch.int32)
        xr[1] = 0
        xr[2] = torch.randint(-3, 4, (n,), generator=g, dtype=torch.int32)
        xr[3, :] = 0
        xr[3, 5] = -(1 << 30)
        y = rms_mod.di_rmsnorm(xr)
        out[f"rms{n}_x"], out[f"rms{n}_y"] = _np(xr), _np(y)
    x64 = _i64(g, (16, 128), -(1 << 40), 1 << 40)
    out["rms64_x"], out["rms64_y"] = _np(x64), _np(rms_mod.di_rmsnorm(x64))
    xg = torch.randint(-(1 << 16), 1 << 16, (2, 5, 4, 128), generator=g, dtype=torch.int32)
    gm = _i64(g, (128,), -(1 << 13), 1 << 13)
    yg, kout = rms_mod.di_rmsnorm_gamma(xg, gm, 13)
    out.update(rmsg_x=_np(xg), rmsg_gm=_np(gm), rmsg_y=_np(yg), rmsg_k=np.int64(kout))
    # di_swiglu
    gate = torch.randint(-(1 << 14), (1 << 14) + 1, (24, 3072), generator=g, dtype=torch.int32)
    up = torch.randint(-(1 << 14), (1 << 14) + 1, (24, 3072), generator=g, dtype=torch.int32)
    gate[0, :8] = torch.tensor([0, 1, -1, 1 << 14, -(1 << 14), 5, -5, 0], dtype=torch.int32)
    gm = _i64(g, (24, 1), 1 << 15, 1 << 16)
    gk = _i64(g, (24, 1), 18, 34)
    um = _i64(g, (24, 1), 1 << 15, 1 << 16)
    uk = _i64(g, (24, 1), 18, 34)
    y, ym, yk = ops_mod.di_swiglu(gate, gm, gk, up, um, uk)
    out.update(sw_g=_np(gate), sw_u=_np(up), sw_gm=_np(gm), sw_gk=_np(gk), sw_um=_np(um),
               sw_uk=_np(uk), sw_y=_np(y), sw_ym=_np(ym), sw_yk=_np(yk))
    # RoPE: tables (offline float) and the integer rotation
    cos_t, sin_t = rope_mod.build_rope_tables(128, 4096, 1e6)
    out["rope_cos_digest"] = np.frombuffer(hashlib.sha256(_np(cos_t).tobytes()).digest(),
                                           dtype=np.uint8)
    out["rope_sin_digest"] = np.frombuffer(hashlib.sha256(_np(sin_t).tobytes()).digest(),
                                           dtype=np.uint8)
    xr = _i64(g, (2, 4, 6, 128), -(1 << 36), 1 << 36)
    pos = _i64(g, (2, 4, 6), 0, 4096)
    yr = rope_mod.apply_int_rope(xr, cos_t, sin_t, pos)
    out.update(rope_x=_np(xr), rope_pos=_np(pos), rope_y=_np(yr))
    return out


def _chain_hashes(rows):
    """scripts/demo.py:58-75 — h_i = sha256(h_{i-1} || int32-LE logits row)."""
    h = hashlib.sha256(b"detllm-demo-v1").digest()
    steps = []
    for r in rows:
        h = hashlib.sha256(h + np.ascontiguousarray(_np(r), dtype="<i4").tobytes()).digest()
        steps.append(h.hex()[:16])
    return steps


def _tok_chain(toks):
    h = hashlib.sha256(b"detllm-demo-v1").digest()
    steps = []
    for t in toks:
        h = hashlib.sha256(h + int(t).to_bytes(8, "little")).digest()
        steps.append(h.hex()[:16])
    return steps


def model_vectors(name, dims, seed, prompt_len, new_tokens, co_count):
    import torch
    from detllm.model import IntQwen3

    from idempotent_llm_amd import artifact as art
    rec = {"dims": dims, "seed": seed}
    with tempfile.TemporaryDirectory() as tmp:
        art.make_artifact(tmp, dims, seed)
        rec["artifact_sha256"] = art.artifact_digest(tmp)
        model = IntQwen3(tmp, backend="reference")
        V = dims["vocab"]
        ids = torch.from_numpy(art.prompt_ids(seed * 10, prompt_len, V))
        pos = torch.arange(prompt_len).unsqueeze(0)
        # prefill logits (and the guard: no float on the numerical path)
        logits, xm, xk, _ = model.forward(ids.unsqueeze(0), pos, guard=True)
        rec["prompt"] = ids.tolist()
        rec["prefill_chain"] = _chain_hashes(logits[0])
        rec["prefill_last_row"] = logits[0, -1].tolist()
        rec["prefill_xm"] = xm[0, :, 0].tolist()
        rec["prefill_xk"] = xk[0, :, 0].tolist()
        # batch-1 greedy generation
        toks, steps = model.generate(ids.unsqueeze(0), new_tokens)
        rec["b1_tokens"] = toks[0].tolist()
        rec["b1_logit_chain"] = _chain_hashes([s[0] for s in steps])
        rec["b1_token_chain"] = _tok_chain(toks[0])
        # right-padded batch with seeded co-prompts (scripts/demo.py:113-124)
        seqs = [ids.numpy()] + art.co_prompts(seed * 10 + 1, co_count, V)
        bids, valid = art.right_pad(seqs)
        toks_b, steps_b = model.generate(torch.from_numpy(bids), new_tokens,
                                         chunk_valid=torch.from_numpy(valid))
        rec["batch_ids"] = bids.tolist()
        rec["batch_valid"] = valid.astype(int).tolist()
        rec["batch_tokens"] = toks_b.tolist()
        rec["batch_row_chains"] = [_chain_hashes([s[b] for s in steps_b])
                                   for b in range(len(seqs))]
        # split prefill: first half at once, rest token by token, then decode
        half = prompt_len // 2
        lg, _, _, cache = model.forward(ids[:half].unsqueeze(0), pos[:, :half])
        rows = []
        for t in range(half, prompt_len):
            lg, _, _, cache = model.forward(ids[t:t + 1].unsqueeze(0),
                                            torch.tensor([[t]]), cache)
            rows.append(lg[0, 0])
        rec["split_tail_chain"] = _chain_hashes(rows)
        # greedy_pick with crafted ties (lowest id wins)
        base = logits[0, -1].clone()
        picks = []
        tie_rows = []
        for r in range(4):
            row = base.clone()
            j = int(model.greedy_pick(row.unsqueeze(0))[0])
            hm = model.head_m
            # make another id tie exactly: same scaled value needs equal
            # logit*head_m; use an id with an identical head_m mantissa if any
            same = (hm == hm[j]).nonzero().flatten().tolist()
            others = [s for s in same if s != j]
            if others:
                o = others[r % len(others)]
                row[o] = row[j]
            tie_rows.append(row.tolist())
            picks.append(int(model.greedy_pick(row.unsqueeze(0))[0]))
        rec["tie_rows"] = tie_rows
        rec["tie_picks"] = picks
    with open(os.path.join(HERE, f"model_{name}.json"), "w") as f:
        json.dump(rec, f)
    return rec


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference/src")
    ap.add_argument("--only", default="all")
    args = ap.parse_args()
    sys.path.insert(0, args.ref)
    sys.path.insert(0, ROOT)
    import torch
    torch.set_num_threads(8)
    from detllm import dyadic as dy
    from detllm import ops as ops_mod
    import importlib
    rms_mod = importlib.import_module("detllm.ops.di_rmsnorm")
    rope_mod = importlib.import_module("detllm.ops.rope")

    from idempotent_llm_amd import artifact as art
    if args.only in ("all", "dyadic"):
        np.savez_compressed(os.path.join(HERE, "dyadic.npz"), **dyadic_vectors(dy))
    if args.only in ("all", "ops"):
        np.savez_compressed(os.path.join(HERE, "ops.npz"),
                            **ops_vectors(ops_mod, rope_mod, rms_mod))
    if args.only in ("all", "tiny"):
        model_vectors("tiny", art.TINY, seed=11, prompt_len=24, new_tokens=20, co_count=3)
    if args.only in ("all", "mid"):
        model_vectors("mid", art.MID, seed=12, prompt_len=40, new_tokens=12, co_count=3)
    print("golden vectors written to", HERE)


if __name__ == "__main__":
    main()
