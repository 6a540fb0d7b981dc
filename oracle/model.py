"""CPU restatement of ``IntQwen3`` (``src/detllm/model.py:105-531``).

Runs the reference backend's dataflow on numpy int64 arrays: artifact load
(:106-183), ``_norm_quant`` (:187-198), ``_qk_head_pipeline`` (:200-216),
``_forward`` (:233-286), ``_layer`` (:288-428), ``_lm_head`` (:430-432),
``greedy_pick`` (:482-490) and ``generate`` (:492-531). The KV cache is the
reference's contiguous int8 ``[B, n_kv, S, hd]`` per layer with a ``valid``
slot mask; the reference's static-capacity / graphed variants compute the same
bits by construction (graphed.py:12-20), so only the dynamic form is restated.

Pinned: tests/golden/model_tiny.json and model_mid.json — logits, tokens and demo chain hashes
written by running the reference's own ``IntQwen3(backend="reference")`` on a
seeded random-init artifact (tests/golden/make_golden.py).
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass, field

import numpy as np

from . import dyadic as dy
from . import ops
from .gemm import exact_matmul_f32, int_gemm, matmul_i64
from .intmath import I32, I64, as64, shl

LAYER_LINEARS = ("q", "k", "v", "o", "gate", "up", "down")


@dataclass
class OracleKV:
    """model.py:67-102 — per-layer int8 K/V, ``valid`` [B, S], ``length``."""
    k8: list = field(default_factory=list)
    v8: list = field(default_factory=list)
    valid: np.ndarray | None = None
    length: int = 0


class IntQwen3Oracle:
    def __init__(self, artifact_dir: str):
        from safetensors.numpy import load_file
        with open(os.path.join(artifact_dir, "config.json")) as f:
            self.cfg = json.load(f)
        t = load_file(os.path.join(artifact_dir, "model.safetensors"))
        for name, v in t.items():   # model.py:117-119
            assert v.dtype in (np.int8, np.int16, np.int32, np.int64), (name, v.dtype)
        c = self.cfg
        self.n_layers = c["n_layers"]; self.hidden = c["hidden"]
        self.n_q = c["n_q_heads"]; self.n_kv = c["n_kv_heads"]; self.hd = c["head_dim"]
        self.vocab = c["vocab"]
        self.group = self.n_q // self.n_kv
        self.t = t
        self.embed_e8 = t["embed.e8"]; self.embed_m = t["embed.m"]; self.embed_k = t["embed.k"]
        self.head_w8t = t["head.w8t"]; self.head_m = t["head.m"]; self.head_k = c["head"]["k"]
        self.rope_cos = t["rope.cos"]; self.rope_sin = t["rope.sin"]
        self.layers = []
        for i in range(self.n_layers):
            p = f"layers.{i}."
            Lc = c["layers"][i]
            L = {}
            for nm in LAYER_LINEARS:
                L[nm + "_w8t"] = t[p + nm + ".w8t"]
                L[nm + "_m"] = t[p + nm + ".m"]
                L[nm + "_k"] = int(Lc[nm]["k"])
            L["q_norm_m"] = t[p + "q_norm.m"]; L["q_norm_k"] = int(Lc["q_norm_k"])
            L["k_norm_m"] = t[p + "k_norm.m"]; L["k_norm_k"] = int(Lc["k_norm_k"])
            for nm in ("qs", "as", "ms", "ds", "os"):
                L[nm + "_m"] = t[p + nm + "_m"]; L[nm + "_k"] = int(Lc[nm + "_k"])
            for nm in ("kq_m", "kq_k", "ks_m", "ks_k", "vq_m", "vq_k"):
                L[nm] = t[p + nm]
            # model.py:165-176: merged attention-output column scale
            vk_shared = int(L["vq_k"].max())
            aligned = shl(as64(L["vq_m"]), vk_shared - as64(L["vq_k"]))
            per_q_head = np.repeat(aligned, self.group)
            L["attn_out_col_m"] = np.repeat(per_q_head, self.hd)
            L["attn_out_col_k"] = vk_shared + (ops.P_OUT_BITS - 1)
            L["k_rowk"] = ops.OUT_FRAC_BITS + L["k_norm_k"]
            self.layers.append(L)
        self._w32: dict = {}

    # -- exact GEMM against a cached float32 copy of a weight matrix -------
    def _gemm_w(self, x8: np.ndarray, key: str, w8t: np.ndarray) -> np.ndarray:
        w32 = self._w32.get(key)
        if w32 is None:
            w32 = w8t.astype(np.float32)
            self._w32[key] = w32
        return exact_matmul_f32(x8, w32).astype(I32)

    # -- helpers (model.py:187-216) ----------------------------------------
    def _norm_quant(self, h, k_res, sm_m=None, sm_k=0):
        y = ops.di_rmsnorm(h)
        kq = np.full_like(as64(k_res), ops.OUT_FRAC_BITS)
        if sm_m is not None:
            y = as64(y) * as64(sm_m)
            kq = kq + sm_k
        one = np.ones_like(as64(k_res))
        return dy.quant_i8_pertoken(y, one, kq)

    def _qk_head_pipeline(self, P, row_m, row_k, w_m, w_k, gamma_m, gamma_k,
                          n_heads, positions):
        B, T, _ = P.shape
        Ph = P.reshape(B, T, n_heads, self.hd)
        cm = w_m.reshape(n_heads, self.hd)
        y, _m, _k = dy.requant_i32_common(Ph, row_m[..., None], row_k[..., None],
                                          cm, w_k, target_bits=16)
        yn, k_out = ops.di_rmsnorm_gamma(y, gamma_m, gamma_k)
        yn = yn.transpose(0, 2, 1, 3)
        pos = np.broadcast_to(positions[:, None, :], (B, n_heads, T))
        yr = ops.apply_int_rope(yn, self.rope_cos, self.rope_sin, pos)
        return yr, k_out

    # -- forward (model.py:220-286) -----------------------------------------
    def forward(self, ids, positions, cache: OracleKV | None = None, chunk_valid=None,
                head_rows=None):
        """model.py:220-286. head_rows (int [B], optional): the LM head only at
        position head_rows[b] of each row, logits [B, vocab] (the final norm,
        quantisation and head GEMM act row by row, so this is the same rows
        the full [B, T, vocab] logits hold; generate() keeps only those)."""
        ids = np.asarray(ids, dtype=I64)
        positions = np.asarray(positions, dtype=I64)
        B, T = ids.shape
        if chunk_valid is None:
            chunk_valid = np.ones((B, T), dtype=bool)
        chunk_valid = np.asarray(chunk_valid, dtype=bool)
        if cache is None:
            cache = OracleKV()
        S_past = cache.length
        e8 = self.embed_e8[ids]
        em = self.embed_m[ids][..., None]
        ek = self.embed_k[ids][..., None]
        h, k_res = dy.residual_from_delta(e8.astype(I32), em, ek)
        valid_all = chunk_valid if cache.valid is None else np.concatenate(
            [cache.valid, chunk_valid], axis=1)
        cache.valid = valid_all
        S = valid_all.shape[1]
        slot = np.arange(S)
        causal = slot[None, :] <= (S_past + np.arange(T))[:, None]
        mask = valid_all[:, None, None, :] & causal[None, None, :, :]
        for li, L in enumerate(self.layers):
            h, k_res = self._layer(li, L, h, k_res, mask, positions, cache, S_past, S)
        cache.length = S
        if head_rows is not None:
            sel = (np.arange(B), np.asarray(head_rows, dtype=I64))
            h, k_res = h[sel][:, None], k_res[sel][:, None]
        x8, xm, xk = self._norm_quant(h, k_res)
        logits = self._gemm_w(x8, "head", self.head_w8t)
        if head_rows is not None:
            return logits[:, 0], xm[:, 0], xk[:, 0], cache
        return logits, xm, xk, cache

    def _layer(self, li, L, h, k_res, mask, positions, cache, S_past, S):
        """model.py:288-428 (dynamic cache mode)."""
        B, T = h.shape[0], h.shape[1]
        g, hd, n_q, n_kv = self.group, self.hd, self.n_q, self.n_kv
        p = f"{li}."
        x8, xm, xk = self._norm_quant(h, k_res, L["as_m"], L["as_k"])
        Pq = self._gemm_w(x8, p + "q", L["q_w8t"])
        Pk = self._gemm_w(x8, p + "k", L["k_w8t"])
        Pv = self._gemm_w(x8, p + "v", L["v_w8t"])
        q, qkk = self._qk_head_pipeline(Pq, xm, xk, L["q_m"], L["q_k"], L["q_norm_m"],
                                        L["q_norm_k"], n_q, positions)
        kk, _ = self._qk_head_pipeline(Pk, xm, xk, L["k_m"], L["k_k"], L["k_norm_m"],
                                       L["k_norm_k"], n_kv, positions)
        qs = np.repeat(L["qs_m"].reshape(n_kv, hd), g, axis=0)
        q = q * qs[None, :, None, :]
        qkk = qkk + L["qs_k"]
        one = np.ones((B, n_q, T, 1), dtype=I64)
        q8, qm, qk = dy.quant_i8_pertoken(q, one, np.zeros_like(one) + qkk)
        k8 = dy.requant_i8_static(kk, 1, L["k_rowk"], 1, 0,
                                  L["kq_m"].reshape(1, n_kv, 1, hd),
                                  L["kq_k"].reshape(1, n_kv, 1, hd))
        Pvh = Pv.reshape(B, T, n_kv, hd)
        v8 = dy.requant_i8_static(Pvh, xm[..., None], xk[..., None],
                                  L["v_m"].reshape(n_kv, hd), L["v_k"],
                                  L["vq_m"].reshape(1, 1, n_kv, 1),
                                  L["vq_k"].reshape(1, 1, n_kv, 1))
        v8 = v8.transpose(0, 2, 1, 3)
        if len(cache.k8) <= li:
            cache.k8.append(k8)
            cache.v8.append(v8)
        else:
            cache.k8[li] = np.concatenate([cache.k8[li], k8], axis=2)
            cache.v8[li] = np.concatenate([cache.v8[li], v8], axis=2)
        K8, V8 = cache.k8[li], cache.v8[li]
        assert K8.shape[2] == S
        # score scale per (b, q-head, t): model.py:469-474 / :372-374
        ks_m = np.repeat(L["ks_m"], g).reshape(1, n_q, 1, 1)
        ks_k = np.repeat(L["ks_k"], g).reshape(1, n_q, 1, 1)
        sm, sk = dy.norm_scale(qm * ks_m, qk + ks_k)
        # exact integer attention: every query row is independent, so the
        # reference's query chunking (model.py:383-402) does not change bits
        K8r = np.repeat(K8, g, axis=1)
        V8r = np.repeat(V8, g, axis=1)
        attn = np.empty((B, n_q, T, hd), dtype=I64)
        CH = max(1, min(T, (1 << 24) // max(1, B * n_q * S)))
        for q0 in range(0, T, CH):
            q1 = min(T, q0 + CH)
            scores = int_gemm(q8[:, :, q0:q1], np.ascontiguousarray(K8r.transpose(0, 1, 3, 2)))
            probs = ops.di_softmax(scores, sm[:, :, q0:q1], sk[:, :, q0:q1],
                                   np.broadcast_to(mask[:, :, q0:q1], (B, n_q, q1 - q0, S)))
            attn[:, :, q0:q1] = matmul_i64(probs, V8r)
        attn = attn.transpose(0, 2, 1, 3).reshape(B, T, n_q * hd)
        rk0 = np.zeros((B, T, 1), dtype=I64) + L["os_k"]
        a8, am, ak = dy.requant_i8_rowcol(attn * as64(L["os_m"]), np.ones_like(rk0), rk0,
                                          L["attn_out_col_m"], L["attn_out_col_k"])
        Po = self._gemm_w(a8, p + "o", L["o_w8t"])
        d, dm, dk = dy.requant_i32_common(Po, am, ak, L["o_m"], L["o_k"], target_bits=20)
        h, k_res = dy.residual_add(h, k_res, d, dm, dk)
        # MLP (model.py:414-427)
        x8, xm, xk = self._norm_quant(h, k_res, L["ms_m"], L["ms_k"])
        Pg = self._gemm_w(x8, p + "gate", L["gate_w8t"])
        Pu = self._gemm_w(x8, p + "up", L["up_w8t"])
        gate, gm, gk = dy.requant_i32_common(Pg, xm, xk, L["gate_m"], L["gate_k"], target_bits=14)
        up, um, uk = dy.requant_i32_common(Pu, xm, xk, L["up_m"], L["up_k"], target_bits=14)
        y, ym, yk = ops.di_swiglu(gate, gm, gk, up, um, uk)
        y8, y8m, y8k = dy.quant_i8_pertoken(y * as64(L["ds_m"]), ym, yk + L["ds_k"])
        Pd = self._gemm_w(y8, p + "down", L["down_w8t"])
        d, dm, dk = dy.requant_i32_common(Pd, y8m, y8k, L["down_m"], L["down_k"], target_bits=20)
        return dy.residual_add(h, k_res, d, dm, dk)

    # -- decoding (model.py:482-531) ----------------------------------------
    def greedy_pick(self, logits_row):
        """int64 argmax of logits*head_m with the lowest-id tie-break."""
        scaled = as64(logits_row) * as64(self.head_m)
        mx = scaled.max(axis=-1, keepdims=True)
        idx = np.broadcast_to(np.arange(self.vocab, dtype=I64), scaled.shape)
        cand = np.where(scaled == mx, idx, self.vocab)
        return cand.min(axis=-1)

    def generate(self, ids, max_new: int, chunk_valid=None):
        ids = np.asarray(ids, dtype=I64)
        B, T0 = ids.shape
        if chunk_valid is None:
            chunk_valid = np.ones((B, T0), dtype=bool)
        positions = np.broadcast_to(np.arange(T0, dtype=I64), (B, T0))
        logits, _, _, cache = self.forward(ids, positions, None, chunk_valid)
        lens = np.asarray(chunk_valid, dtype=bool).sum(axis=1).astype(I64)
        last = np.maximum(lens - 1, 0)
        step_logits = [logits[np.arange(B), last]]
        cur = self.greedy_pick(step_logits[0])
        out = [cur]
        for step in range(1, max_new):
            pos = (lens + step - 1)[:, None]
            lg, _, _, cache = self.forward(cur[:, None], pos, cache, np.ones((B, 1), dtype=bool))
            step_logits.append(lg[:, 0])
            cur = self.greedy_pick(lg[:, 0])
            out.append(cur)
        return np.stack(out, axis=1), step_logits
