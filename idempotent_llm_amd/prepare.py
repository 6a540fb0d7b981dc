"""Offline float quantiser: a Qwen3 float checkpoint -> the integer artifact
the runtime loads (the contract of the reference's src/detllm/prepare.py:
same schema, same fitting rules, so its artifacts and these are
interchangeable).

This is the one place where floats are allowed: weights are fitted in
float64, calibration runs the float model. Nothing here is on the integer
path; the runtime reads only the artifact (int tensors + a config of integer
scalars).

Offline by construction: the float model is a local Hugging Face checkpoint
directory (or a model object) and the calibration tokens are given by the
caller (``calib_ids``: int64 [n_samples, calib_len], for instance a
tokenised local text file); the reference fetches both from the Hub and a
dataset (prepare.py:239-240, :144-146).

Steps (prepare.py:228-434):
  1. architecture checks (Qwen3, tied embeddings, QK-Norm, int32 headroom);
  2. calibration: per-channel maxima of the post-QK-norm, post-RoPE K and Q
     (Q aggregated over each GQA group), per-head V maxima, and the maxima of
     the activations entering q|k|v, gate|up (RMSNorm output with gamma
     removed), down and o;
  3. fitting: per-output-channel int8 weights with one shift per tensor,
     per-row embedding scales, gamma mantissas, analytic activation smoothing
     (alpha = 0.5) folded into the consumer weights, QK smoothing
     (alpha = qk_alpha) with static per-channel K and per-head V int8 scales;
  4. write model.safetensors + config.json.
"""

from __future__ import annotations

import argparse
import json
import math
import os

import numpy as np
import torch

from .artifact import rope_tables

ROPE_FRAC_BITS = 14
F64 = torch.float64
I64 = torch.int64


# ---------------------------------------------------------------------------
# dyadic fits (prepare.py:43-115)
# ---------------------------------------------------------------------------

def fit_dyadic_float(s: float, bits: int = 16) -> tuple[int, int]:
    """(m, k) with m / 2^k ~ s and 2^(bits-1) <= m < 2^bits (prepare.py:43-52):
    k from the exponent of s, m rounded; a mantissa rounded up to 2^bits is
    halved (rounding half up) with k one lower."""
    assert s > 0
    k = bits - 1 - math.floor(math.log2(s))
    m = round(s * 2.0 ** k)
    if m >= 1 << bits:
        m, k = (m + 1) // 2, k - 1
    assert 1 << (bits - 1) <= m < 1 << bits, (s, m, k)
    return m, k


def fit_dyadic_float_vec(s: torch.Tensor, bits: int = 16):
    """Element-wise fit_dyadic_float for s > 0 (prepare.py:90-99): a mantissa
    that rounds up to 2^bits is refitted at k - 1. Returns int64 (m, k)."""
    s = s.to(F64)
    k = (bits - 1) - torch.floor(torch.log2(s)).to(I64)
    m = torch.round(s * torch.pow(2.0, k.to(F64))).to(I64)
    up = m >= (1 << bits)
    k = torch.where(up, k - 1, k)
    m = torch.where(up, torch.round(s * torch.pow(2.0, k.to(F64))).to(I64), m)
    return m.clamp(min=1), k


def quant_weight_per_channel(W: torch.Tensor, bits: int = 16, weight_bits: int = 8):
    """W float [out, in] -> (w int8 [out, in], m int64 [out], k int)
    (prepare.py:55-73): symmetric per output channel, scale s_c =
    max|W[c]| / lim; the mantissas m_c = round(s_c 2^k) share one k chosen
    from the largest scale (refitted one lower if it rounds to 2^bits).
    weight_bits 16 gives int16 weights (a diagnostic width)."""
    W = W.to(F64)
    lim = (1 << (weight_bits - 1)) - 1
    s = W.abs().amax(dim=1).clamp(min=1e-12) / lim
    q = torch.round(W / s[:, None]).clamp(-lim, lim)
    q = q.to(torch.int8 if weight_bits == 8 else torch.int16)
    k = bits - 1 - math.floor(math.log2(float(s.max())))
    m = torch.round(s * 2.0 ** k).to(I64)
    if int(m.max()) >= 1 << bits:
        k -= 1
        m = torch.round(s * 2.0 ** k).to(I64)
    return q, m.clamp(min=1), k


def quant_embedding_per_row(E: torch.Tensor):
    """E float [V, H] -> (e8 int8, m int64 [V], k int64 [V]) (prepare.py:76-87):
    one scale per row, each with its own shift (a row is one token)."""
    E = E.to(F64)
    s = E.abs().amax(dim=1).clamp(min=1e-12) / 127.0
    e8 = torch.round(E / s[:, None]).clamp(-127, 127).to(torch.int8)
    m, k = fit_dyadic_float_vec(s, 16)
    return e8, m, k


def fit_gamma_dyadic(gamma: torch.Tensor, bits: int = 14):
    """Signed per-channel gamma -> (m int64, k int) with one shift sized so that
    max |m| lies in [2^(bits-1), 2^bits) (prepare.py:102-115)."""
    g = gamma.to(F64)
    amax = float(g.abs().max())
    assert amax > 0
    k = bits - 1 - math.floor(math.log2(amax))
    m = torch.round(g * 2.0 ** k).to(I64)
    if int(m.abs().max()) >= 1 << bits:
        k -= 1
        m = torch.round(g * 2.0 ** k).to(I64)
    return m, k


def _smooth_dyadic(f: torch.Tensor, top_bits: int = 13):
    """A positive factor vector as a shared-shift dyadic (m, k) with the
    largest mantissa at top_bits bits; returns (m, k, the exact values m/2^k)
    (the inverse-smoothing and QK factors of prepare.py:298-301, :389-392)."""
    k = top_bits - math.floor(math.log2(float(f.max())))
    m = torch.round(f * 2.0 ** k).to(I64).clamp(min=1)
    return m, k, m.to(F64) * 2.0 ** -k


# ---------------------------------------------------------------------------
# calibration (prepare.py:120-226)
# ---------------------------------------------------------------------------

class _Capture:
    """Forward hooks on one Qwen3 decoder layer's modules: the QK-norm
    outputs, v_proj output, both RMSNorm outputs, and the inputs of o_proj
    and down_proj."""

    def __init__(self, layer):
        self.t = {}
        a, mlp = layer.self_attn, layer.mlp
        out = lambda key: (lambda mod, inp, o: self.t.__setitem__(key, o.detach()))
        inp = lambda key: (lambda mod, i: self.t.__setitem__(key, i[0].detach()))
        self.handles = [a.q_norm.register_forward_hook(out("q")),
                        a.k_norm.register_forward_hook(out("k")),
                        a.v_proj.register_forward_hook(out("v")),
                        layer.input_layernorm.register_forward_hook(out("attn_in")),
                        layer.post_attention_layernorm.register_forward_hook(out("mlp_in")),
                        a.o_proj.register_forward_pre_hook(inp("o_in")),
                        mlp.down_proj.register_forward_pre_hook(inp("down_in"))]

    def remove(self):
        for h in self.handles:
            h.remove()


def _heads_first_time(x: torch.Tensor, n_heads: int) -> torch.Tensor:
    """[B, T, heads, hd] whatever the module emitted ([B, heads, T, hd] or
    [B, T, heads, hd])."""
    if x.shape[1] == n_heads and x.shape[2] != n_heads:
        x = x.transpose(1, 2)
    return x


def _rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Float RoPE on [B, T, heads, hd] (HF tiling: rotate_half pairs j, j + hd/2)."""
    hd = x.shape[-1]
    rot = torch.cat([-x[..., hd // 2:], x[..., :hd // 2]], dim=-1)
    T = x.shape[1]
    return x * cos[None, :T, None, :] + rot * sin[None, :T, None, :]


def _rope_theta(cfg) -> float:
    if getattr(cfg, "rope_theta", None) is not None:
        return float(cfg.rope_theta)
    return float(cfg.rope_parameters["rope_theta"])


@torch.no_grad()
def calibration_maxima(model, calib_ids: torch.Tensor, device) -> dict:
    """Run the float model over the calibration rows; per layer the maxima the
    fits need (prepare.py:120-226): k [n_kv, hd] and q (grouped) [n_kv, hd]
    after QK-norm and RoPE, v [n_kv], and the input maxima attn_in / mlp_in
    (RMSNorm output divided by its gamma), o_in, down_in per channel."""
    cfg = model.config
    L = cfg.num_hidden_layers
    n_q, n_kv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    T = calib_ids.shape[1]
    j = torch.arange(hd // 2, dtype=F64)
    inv = _rope_theta(cfg) ** (-2.0 * j / hd)
    ang = torch.outer(torch.arange(T, dtype=F64), inv)
    ang = torch.cat([ang, ang], dim=-1)
    cos, sin = torch.cos(ang).float(), torch.sin(ang).float()
    acc = {"k": torch.zeros(L, n_kv, hd), "q": torch.zeros(L, n_kv, hd),
           "v": torch.zeros(L, n_kv), "attn_in": torch.zeros(L, cfg.hidden_size),
           "mlp_in": torch.zeros(L, cfg.hidden_size),
           "o_in": torch.zeros(L, n_q * hd), "down_in": torch.zeros(L, cfg.intermediate_size)}
    caps = [_Capture(layer) for layer in model.model.layers]
    try:
        for row in calib_ids:
            model(row[None].to(device))
            for i, (cap, layer) in enumerate(zip(caps, model.model.layers)):
                t = {k: v.float().cpu() for k, v in cap.t.items()}
                k = _rotate(_heads_first_time(t["k"], n_kv), cos, sin)
                acc["k"][i] = torch.maximum(acc["k"][i], k.abs().amax(dim=(0, 1)))
                q = _rotate(_heads_first_time(t["q"], n_q), cos, sin).abs().amax(dim=(0, 1))
                q = q.view(n_kv, n_q // n_kv, hd).amax(dim=1)
                acc["q"][i] = torch.maximum(acc["q"][i], q)
                v = t["v"].reshape(*t["v"].shape[:2], n_kv, hd)
                acc["v"][i] = torch.maximum(acc["v"][i], v.abs().amax(dim=(0, 1, 3)))
                for key, g in (("attn_in", layer.input_layernorm.weight),
                               ("mlp_in", layer.post_attention_layernorm.weight)):
                    g = g.detach().float().cpu()
                    # the runtime quantises x / rms without gamma (gamma folds
                    # into the consumer weights)
                    x = t[key] / (torch.where(g >= 0, 1.0, -1.0) * g.abs().clamp(min=1e-4))
                    acc[key][i] = torch.maximum(acc[key][i], x.abs().amax(dim=(0, 1)))
                for key in ("o_in", "down_in"):
                    acc[key][i] = torch.maximum(acc[key][i], t[key].abs().amax(dim=(0, 1)))
    finally:
        for cap in caps:
            cap.remove()
    return acc


# smoothing factors (activation and QK) are clamped to [1/SMOOTH_CLAMP,
# SMOOTH_CLAMP] (prepare.py:297, :387)
SMOOTH_CLAMP = 64.0


def _relative(s: torch.Tensor) -> torch.Tensor:
    """Activation smoothing keeps only the relative scale of its factors:
    they are divided by their median (prepare.py:296)."""
    return s / s.median()


def _act_smoothing(act_max: torch.Tensor, weights: list, alpha: float = 0.5):
    """Analytic SmoothQuant factors for one linear-input site (prepare.py:
    285-302): s_c = amax_c^alpha / wmax_c^(1-alpha), normalised by the median,
    clamped to [1/64, 64]. The runtime multiplies the activation by the dyadic
    1/s (inv_m / 2^inv_k); the weights take the exactly matching s. Returns
    (inv_m int64, inv_k int, s used [C] float64)."""
    wmax = torch.stack([w.to(F64).abs().amax(dim=0) for w in weights]).amax(dim=0)
    s = act_max.to(F64).clamp(min=1e-5).pow(alpha) / wmax.clamp(min=1e-5).pow(1 - alpha)
    s = _relative(s).clamp(1 / SMOOTH_CLAMP, SMOOTH_CLAMP)
    inv_m, inv_k, inv = _smooth_dyadic(1.0 / s)
    return inv_m, inv_k, 1.0 / inv


# ---------------------------------------------------------------------------
# the artifact (prepare.py:228-434)
# ---------------------------------------------------------------------------

def _check_architecture(cfg):
    assert cfg.model_type == "qwen3", cfg.model_type
    assert cfg.tie_word_embeddings, "expected tied embeddings (the LM head is the embedding)"
    for K in (cfg.hidden_size, cfg.intermediate_size, cfg.num_attention_heads * cfg.head_dim,
              cfg.num_key_value_heads * cfg.head_dim):
        assert K * 127 * 127 < 2 ** 31, K      # int32 GEMM accumulators
    assert cfg.max_position_embeddings * 128 * 127 < 2 ** 31  # probabilities x V


@torch.no_grad()
def prepare(out_dir: str, model, calib_ids, kv_margin: float = 1.05, device=None,
            smooth_o: bool = True, smooth_acts: bool = True, weight_bits: int = 8,
            qk_alpha: float = 0.3, model_id: str | None = None) -> str:
    """Quantise a Qwen3 float model into an integer artifact in out_dir.

    model: a transformers Qwen3ForCausalLM or a local checkpoint directory;
    calib_ids: int64 [n_samples, calib_len] calibration tokens (array or
    tensor). The options are the reference's (prepare.py:228-233)."""
    from safetensors.torch import save_file
    if isinstance(model, str):
        from transformers import AutoModelForCausalLM
        model_id = model_id or model
        model = AutoModelForCausalLM.from_pretrained(model, dtype=torch.float32)
    model = model.float().eval()
    device = device or ("cuda" if torch.cuda.is_available() else "cpu")
    cfg = model.config
    _check_architecture(cfg)
    calib_ids = torch.as_tensor(np.asarray(calib_ids), dtype=I64)
    assert calib_ids.ndim == 2 and calib_ids.numel() > 0, "calib_ids: [n_samples, calib_len]"
    L, H = cfg.num_hidden_layers, cfg.hidden_size
    n_q, n_kv, hd, inter = (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
                            cfg.intermediate_size)
    model.to(device)
    mx = calibration_maxima(model, calib_ids, device)
    model.cpu()

    tensors: dict = {}
    conf: dict = {
        "model_id": model_id or "local-float-model",
        "n_layers": L, "hidden": H, "n_q_heads": n_q, "n_kv_heads": n_kv, "head_dim": hd,
        "intermediate": inter, "vocab": cfg.vocab_size,
        "max_pos": int(cfg.max_position_embeddings), "rope_frac_bits": ROPE_FRAC_BITS,
        "eos_token_id": int(cfg.eos_token_id if cfg.eos_token_id is not None
                            else cfg.vocab_size - 1),
        # build parameters (documentation; the runtime ignores them)
        "calib_samples": int(calib_ids.shape[0]), "calib_len": int(calib_ids.shape[1]),
        "kv_margin": kv_margin, "qk_alpha": qk_alpha, "smooth_o": smooth_o,
        "smooth_acts": smooth_acts, "weight_bits": weight_bits, "layers": [],
    }

    def linear(name, W, col_scale=None):
        """Store W [out, in] (times per-input-column factors) as w8t [in, out]."""
        W = W.detach().to(F64)
        if col_scale is not None:
            W = W * col_scale.to(F64)[None, :]
        q, m, k = quant_weight_per_channel(W, weight_bits=weight_bits)
        tensors[name + ".w8t"] = q.t().contiguous()
        tensors[name + ".m"] = m
        return {"k": k, "min_m": int(m.min())}

    emb = model.model.embed_tokens.weight.detach()
    tensors["embed.e8"], tensors["embed.m"], tensors["embed.k"] = quant_embedding_per_row(emb)
    # LM head: the tied embedding with the final RMSNorm's gamma folded in
    conf["head"] = linear("head", emb, model.model.norm.weight.detach())
    cos_t, sin_t = rope_tables(hd, int(cfg.max_position_embeddings), _rope_theta(cfg))
    tensors["rope.cos"] = torch.from_numpy(cos_t)
    tensors["rope.sin"] = torch.from_numpy(sin_t)

    def ident(n):
        return torch.ones(n, dtype=I64), 0, torch.ones(n, dtype=F64)

    sqrt_hd = math.sqrt(hd)
    for i, layer in enumerate(model.model.layers):
        p, Lc = f"layers.{i}.", {}
        a, mlp = layer.self_attn, layer.mlp
        g_attn = layer.input_layernorm.weight.detach().to(F64)
        g_mlp = layer.post_attention_layernorm.weight.detach().to(F64)
        Wq, Wk, Wv = (w.weight.detach().to(F64) * g_attn[None, :]
                      for w in (a.q_proj, a.k_proj, a.v_proj))
        Wg, Wu = (w.weight.detach().to(F64) * g_mlp[None, :] for w in (mlp.gate_proj, mlp.up_proj))
        Wd, Wo = mlp.down_proj.weight.detach().to(F64), a.o_proj.weight.detach().to(F64)
        # activation smoothing: runtime multiplies by 1/s, weights by s
        sites = (("as", mx["attn_in"][i], [Wq, Wk, Wv], smooth_acts, H),
                 ("ms", mx["mlp_in"][i], [Wg, Wu], smooth_acts, H),
                 ("ds", mx["down_in"][i], [Wd], smooth_acts, inter),
                 ("os", mx["o_in"][i], [Wo], smooth_o, n_q * hd))
        s_used = {}
        for nm, amax, ws, on, n in sites:
            m_, k_, s_ = _act_smoothing(amax, ws) if on else ident(n)
            tensors[p + nm + "_m"] = m_
            Lc[nm + "_k"] = k_
            s_used[nm] = s_
        Lc["q"] = linear(p + "q", Wq, s_used["as"])
        Lc["k"] = linear(p + "k", Wk, s_used["as"])
        Lc["v"] = linear(p + "v", Wv, s_used["as"])
        Lc["o"] = linear(p + "o", Wo, s_used["os"])
        Lc["gate"] = linear(p + "gate", Wg, s_used["ms"])
        Lc["up"] = linear(p + "up", Wu, s_used["ms"])
        Lc["down"] = linear(p + "down", Wd, s_used["ds"])
        tensors[p + "q_norm.m"], Lc["q_norm_k"] = fit_gamma_dyadic(a.q_norm.weight.detach())
        tensors[p + "k_norm.m"], Lc["k_norm_k"] = fit_gamma_dyadic(a.k_norm.weight.detach())
        # QK smoothing (prepare.py:375-394): c_d = maxK^a / maxQ^(1-a) cancels
        # in q . k; Q takes the dyadic c at runtime, K's static per-channel
        # scale is c_d sK_h with one base scale per kv head
        kc = mx["k"][i].to(F64).clamp(min=1e-6)
        qc = mx["q"][i].to(F64).clamp(min=1e-6)
        c = (kc.pow(qk_alpha) / qc.pow(1 - qk_alpha)).clamp(1 / SMOOTH_CLAMP, SMOOTH_CLAMP)
        qs_m, qs_k, c_used = _smooth_dyadic(c)
        tensors[p + "qs_m"] = qs_m
        Lc["qs_k"] = qs_k
        s_kh = (kc / c_used).amax(dim=1) * kv_margin / 127.0        # [n_kv]
        tensors[p + "kq_m"], tensors[p + "kq_k"] = fit_dyadic_float_vec(c_used * s_kh[:, None])
        fits = [(fit_dyadic_float(float(s_kh[h]) / sqrt_hd),
                 fit_dyadic_float(float(mx["v"][i, h]) * kv_margin / 127.0)) for h in range(n_kv)]
        tensors[p + "ks_m"] = torch.tensor([f[0][0] for f in fits], dtype=I64)
        tensors[p + "ks_k"] = torch.tensor([f[0][1] for f in fits], dtype=I64)
        tensors[p + "vq_m"] = torch.tensor([f[1][0] for f in fits], dtype=I64)
        tensors[p + "vq_k"] = torch.tensor([f[1][1] for f in fits], dtype=I64)
        conf["layers"].append(Lc)

    for name, t in tensors.items():
        assert not t.is_floating_point(), f"float tensor in the artifact: {name}"
    os.makedirs(out_dir, exist_ok=True)
    save_file({k: v.contiguous() for k, v in tensors.items()},
              os.path.join(out_dir, "model.safetensors"))
    with open(os.path.join(out_dir, "config.json"), "w") as f:
        json.dump(conf, f, indent=1)
    return out_dir


def main():
    ap = argparse.ArgumentParser(description="quantise a local Qwen3 float checkpoint")
    ap.add_argument("--model-dir", required=True, help="local Hugging Face checkpoint directory")
    ap.add_argument("--calib-ids", required=True,
                    help=".npy of int64 calibration tokens [n_samples, calib_len]")
    ap.add_argument("--out", required=True)
    ap.add_argument("--device", default=None)
    ap.add_argument("--kv-margin", type=float, default=1.05)
    ap.add_argument("--no-smooth-o", action="store_true")
    ap.add_argument("--no-smooth-acts", action="store_true")
    ap.add_argument("--weight-bits", type=int, default=8)
    ap.add_argument("--qk-alpha", type=float, default=0.3)
    args = ap.parse_args()
    prepare(args.out, args.model_dir, np.load(args.calib_ids), kv_margin=args.kv_margin,
            device=args.device, smooth_o=not args.no_smooth_o,
            smooth_acts=not args.no_smooth_acts, weight_bits=args.weight_bits,
            qk_alpha=args.qk_alpha)
    print(f"artifact written to {args.out}")


if __name__ == "__main__":
    main()
