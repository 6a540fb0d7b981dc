"""IntQwen3 on the "rocm" backend: the reference runtime API
(``src/detllm/model.py:105-531``) driving fused gfx950 HIP kernels.

Public surface (same names, argument meaning and return values as the
reference): ``IntQwen3(artifact_dir, backend)``, ``.forward(ids, positions,
cache=None, chunk_valid=None, guard=False) -> (logits, row_m, row_k, cache)``,
``.generate(ids, max_new, guard=False, chunk_valid=None, stop_at_eos=False,
use_graph=False) -> (tokens, step_logits)``, ``.greedy_pick(logits_row)``,
``KVCache``, ``LayerWeights``. Batching/masking model as in model.py:8-17:
right padding, a validity flag per cache slot, explicit positions, K/V
quantised once when produced.

One layer is 9 launches, each fusing everything between two GEMMs
(model.py:288-428):

  x8 --GEMM[q|k|v]--> qkv_epilogue (per-head requant, QK-norm, RoPE,
      smoothing, Q int8 + DI-Exp constant, K/V int8 into the cache)
     --> attention (prefill: MFMA 3-pass; decode: per (row, kv-head))
     --> merge_rowcol (attention-output requant to int8)
     --GEMM[o]--> residual_normq (requant, residual add, RMSNorm, MLP quant)
     --GEMM[gate|up]--> swiglu_quant
     --GEMM[down]--> residual_normq (... next layer's attention quant)

Memory layout in HBM (all integer; built once at load by integer
permutation of the artifact's tensors): weights as [out, in] int8 with
q|k|v and gate|up concatenated along out; per-channel mantissas int64; the
KV cache paged (kvcache.py: per-layer page pools of 128 slots, a page table
per row) plus a [B, slots] validity mask.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass

import torch

from . import dyadic as dy
from . import ops
from ._lib import attn_split_plan, call, gemv_plan, pro_fits, raise_for_error_word
from .backends import canonical_backend, gemm_nt, int_gemm, int_gemm_u16i8
from .guard import NoFloatMode
from .kvcache import PAGE, KVCache  # noqa: F401  (KVCache is part of this module's API)

I64 = torch.int64
P_OUT_BITS = 15
OUT_FRAC_BITS = 20
GREEDY_CHUNK = 2048
# slots the decode attention scans at most (int32 MFMA accumulators of P.V:
# 128 * 128 * S < 2^31)
DEC_MAX_SLOTS = 131071
# decode rows scanning at least this many slots use the split-S attention
SPLIT_MIN_SLOTS = 2048
# decode batches up to this many rows have the attention write the merge's
# row statistics: one row takes the o-GEMV that quantises its own K range of
# the merged row (detllm_igemv_merge_ext: c3 b1 1.136 -> 1.126 ms per step),
# more rows the merge launch cut into 256-column pieces (detllm_merge_ext)
MERGE_EXT_ROWS = 8


@dataclass
class LayerWeights:
    """Per-layer device tensors in kernel layout (model.py:41-64 contents)."""
    idx: int
    wqkv: torch.Tensor   # [(n_q + 2 n_kv) * hd, H] int8
    wo: torch.Tensor     # [H, n_q * hd]
    wgu: torch.Tensor    # [2 I, H]
    wd: torch.Tensor     # [H, I]
    q_m: torch.Tensor; q_k: int
    k_m: torch.Tensor; k_k: int
    v_m: torch.Tensor; v_k: int
    o_m: torch.Tensor; o_k: int
    gate_m: torch.Tensor; gate_k: int
    up_m: torch.Tensor; up_k: int
    down_m: torch.Tensor; down_k: int
    q_norm_m: torch.Tensor; q_norm_k: int
    k_norm_m: torch.Tensor; k_norm_k: int
    qs_m: torch.Tensor; qs_k: int
    as_m: torch.Tensor; as_k: int
    ms_m: torch.Tensor; ms_k: int
    ds_m: torch.Tensor; ds_k: int
    os_m: torch.Tensor; os_k: int
    kq_m: torch.Tensor; kq_k: torch.Tensor
    ks_m: torch.Tensor; ks_k: torch.Tensor
    vq_m: torch.Tensor; vq_k: torch.Tensor
    attn_out_col_m: torch.Tensor
    attn_out_col_k: int
    osc_m: torch.Tensor | None = None     # os_m * attn_out_col_m (fused o-GEMM)
    # the per-column scale vectors each row kernel reads, packed contiguously
    # so the skinny GEMM before it can prefetch them as one range
    pf_attn: torch.Tensor | None = None   # Q/K/V epilogue + attention-output merge
    pf_o: torch.Tensor | None = None      # residual after o
    pf_mlp: torch.Tensor | None = None    # SwiGLU
    # per-channel divisors of the static K requantisation, [n_kv * 128, 4]
    # int64 (detllm_kq_est): layer constants computed once at load
    kq_est: torch.Tensor | None = None

    # the reference's field names (model.py:41-64) as views of the kernel
    # layout, for code written against the reference class (seam overrides)
    @property
    def q_w8t(self) -> torch.Tensor:
        return self.wqkv[:self.q_m.numel()].t()

    @property
    def k_w8t(self) -> torch.Tensor:
        nq = self.q_m.numel()
        return self.wqkv[nq:nq + self.k_m.numel()].t()

    @property
    def v_w8t(self) -> torch.Tensor:
        return self.wqkv[self.q_m.numel() + self.k_m.numel():].t()

    @property
    def o_w8t(self) -> torch.Tensor:
        return self.wo.t()

    @property
    def gate_w8t(self) -> torch.Tensor:
        return self.wgu[:self.gate_m.numel()].t()

    @property
    def up_w8t(self) -> torch.Tensor:
        return self.wgu[self.gate_m.numel():].t()

    @property
    def down_w8t(self) -> torch.Tensor:
        return self.wd.t()

    @property
    def k_rowk(self) -> int:
        return OUT_FRAC_BITS + self.k_norm_k


def _pack(L: LayerWeights, names) -> torch.Tensor:
    """Move the named int64 tensors of L into one buffer (views keep their
    shapes and values); returns the buffer."""
    ts = [getattr(L, n) for n in names]
    buf = torch.cat([t.reshape(-1) for t in ts])
    off = 0
    for n, t in zip(names, ts):
        setattr(L, n, buf[off:off + t.numel()].view(t.shape))
        off += t.numel()
    return buf


class IntQwen3:
    # decode steps of at most this many rows run the fused-operand GEMVs
    # (the skinny GEMM's operand row kernel inside it, one launch fewer per
    # row kernel); more rows run the separate row kernels
    fused_decode_rows = 1
    # K split of the one-row down GEMV with the SwiGLU row fused in
    # (detllm_igemv_swiglu); 0 runs the SwiGLU row kernel and the GEMV apart
    fused_swiglu_ksplit = 3

    def __init__(self, artifact_dir: str, backend: str = "rocm"):
        from safetensors.torch import load_file
        self.backend = canonical_backend(backend)
        if self.backend != "rocm":
            raise ValueError(f"backend {backend!r} is served by detllm itself; this package "
                             "implements the 'rocm' backend")
        if not torch.cuda.is_available():
            raise RuntimeError("the rocm backend needs a gfx950 GPU (torch.cuda unavailable)")
        self.device = torch.device("cuda")
        with open(os.path.join(artifact_dir, "config.json")) as f:
            self.cfg = json.load(f)
        tensors = load_file(os.path.join(artifact_dir, "model.safetensors"))
        for name, t in tensors.items():   # model.py:117-119
            assert t.dtype in (torch.int8, torch.int16, torch.int32, torch.int64), \
                f"float tensor in artifact: {name} {t.dtype}"
        c = self.cfg
        self.n_layers = c["n_layers"]; self.hidden = c["hidden"]
        self.n_q = c["n_q_heads"]; self.n_kv = c["n_kv_heads"]; self.hd = c["head_dim"]
        self.vocab = c["vocab"]; self.inter = c["intermediate"]
        assert self.hd == 128, "the rocm kernels are specialised to head_dim 128"
        assert self.n_q % self.n_kv == 0 and self.n_q // self.n_kv in (1, 2, 4, 8)
        assert self.hidden % 16 == 0 and self.inter % 16 == 0
        assert self.hidden <= 4096 and self.inter <= 4096 and self.n_q * self.hd <= 4096, \
            "the fused row kernels hold a row of at most 4096 columns in one block"
        assert self.hd * 127 * 127 < 2 ** 31 and self.inter * 127 * 127 < 2 ** 31
        dev = self.device
        g = lambda n: tensors[n].to(dev)
        gt = lambda n: tensors[n].t().contiguous().to(dev)   # [in, out] -> [out, in]
        self.embed_e8 = g("embed.e8"); self.embed_m = g("embed.m"); self.embed_k = g("embed.k")
        self.head_w = gt("head.w8t")                       # [V, H]
        self.head_m = g("head.m"); self.head_k = c["head"]["k"]
        self.rope_cos = g("rope.cos").contiguous(); self.rope_sin = g("rope.sin").contiguous()
        self.max_pos = self.rope_cos.shape[0]
        group = self.n_q // self.n_kv
        self.layers: list[LayerWeights] = []
        for i in range(self.n_layers):
            p = f"layers.{i}."
            Lc = c["layers"][i]
            wqkv = torch.cat([tensors[p + "q.w8t"], tensors[p + "k.w8t"], tensors[p + "v.w8t"]],
                             dim=1).t().contiguous().to(dev)
            wgu = torch.cat([tensors[p + "gate.w8t"], tensors[p + "up.w8t"]],
                            dim=1).t().contiguous().to(dev)
            vq_m = tensors[p + "vq_m"].to(I64); vq_k = tensors[p + "vq_k"].to(I64)
            # model.py:165-176: merged attention-output column scale
            vk_shared = int(vq_k.max())
            aligned = torch.bitwise_left_shift(vq_m, vk_shared - vq_k)
            col_m = aligned.repeat_interleave(group).repeat_interleave(self.hd)
            self.layers.append(LayerWeights(
                idx=i, wqkv=wqkv, wo=gt(p + "o.w8t"), wgu=wgu, wd=gt(p + "down.w8t"),
                q_m=g(p + "q.m"), q_k=int(Lc["q"]["k"]), k_m=g(p + "k.m"), k_k=int(Lc["k"]["k"]),
                v_m=g(p + "v.m"), v_k=int(Lc["v"]["k"]), o_m=g(p + "o.m"), o_k=int(Lc["o"]["k"]),
                gate_m=g(p + "gate.m"), gate_k=int(Lc["gate"]["k"]),
                up_m=g(p + "up.m"), up_k=int(Lc["up"]["k"]),
                down_m=g(p + "down.m"), down_k=int(Lc["down"]["k"]),
                q_norm_m=g(p + "q_norm.m"), q_norm_k=int(Lc["q_norm_k"]),
                k_norm_m=g(p + "k_norm.m"), k_norm_k=int(Lc["k_norm_k"]),
                qs_m=g(p + "qs_m").reshape(-1).contiguous(), qs_k=int(Lc["qs_k"]),
                as_m=g(p + "as_m"), as_k=int(Lc["as_k"]), ms_m=g(p + "ms_m"), ms_k=int(Lc["ms_k"]),
                ds_m=g(p + "ds_m"), ds_k=int(Lc["ds_k"]), os_m=g(p + "os_m"), os_k=int(Lc["os_k"]),
                kq_m=g(p + "kq_m").reshape(-1).contiguous(),
                kq_k=g(p + "kq_k").reshape(-1).contiguous(),
                ks_m=g(p + "ks_m"), ks_k=g(p + "ks_k"), vq_m=vq_m.to(dev), vq_k=vq_k.to(dev),
                attn_out_col_m=col_m.to(dev), attn_out_col_k=vk_shared + (P_OUT_BITS - 1)))
        del tensors
        for L in self.layers:
            # the attention-output merge's per-column factor os_m * col_m
            # (int64, wrapping as the kernel's own product does) for the
            # fused o-GEMM
            L.osc_m = L.os_m * L.attn_out_col_m
            L.pf_attn = _pack(L, ["q_m", "k_m", "v_m", "q_norm_m", "k_norm_m", "qs_m", "kq_m",
                                  "kq_k", "ks_m", "ks_k", "vq_m", "vq_k", "os_m",
                                  "attn_out_col_m", "osc_m"])
            L.pf_o = _pack(L, ["o_m", "ms_m"])
            L.pf_mlp = _pack(L, ["gate_m", "up_m", "ds_m"])
            L.kq_est = torch.empty(L.kq_m.numel(), 4, dtype=I64, device=dev)
            call("detllm_kq_est", L.kq_m, L.kq_k, L.kq_m.numel(), 20 + L.k_norm_k, L.kq_est)
        self._greedy_scratch = {}
        self._plans: dict = {}
        self._split_plans: dict = {}
        # decode rows run the fused-operand GEMVs where their shapes allow
        L0 = self.layers[0]
        nqkv, nqh = L0.wqkv.shape[0], self.n_q * self.hd
        self._fused_decode = {
            M: (self.hidden <= 1024 and nqh <= 2048
                and pro_fits(self.hidden, self._ksplit(nqkv, self.hidden, M))
                and pro_fits(nqh, self._ksplit(self.hidden, nqh, M))
                and pro_fits(self.hidden, self._ksplit(2 * self.inter, self.hidden, M)))
            for M in (1, 2)}
        # device error word of the index checks the reference does on the
        # host (IndexError from embed_e8[ids] / cos_t[positions]); the
        # kernels OR bits into it, raise_if_device_error() reads it
        self._err = torch.zeros(1, dtype=torch.int32, device=dev)
        # reference attributes (model.py:177-183) that seam overrides read
        self._one1 = torch.ones(1, dtype=I64, device=dev)
        self._layer_compiled = None

    def raise_if_device_error(self):
        """Synchronise on the error word and raise IndexError (as the
        reference's embed_e8[ids] / cos_t[positions] do) when a kernel saw a
        token id or position outside its table since the last check."""
        word = int(self._err.item())
        if word:
            self._err.zero_()
            raise_for_error_word(word, vocab=self.vocab, max_pos=self.max_pos)

    def _check_host_indices(self, ids: torch.Tensor, positions: torch.Tensor):
        """Host tensors are checked before the copy, so a bad index raises
        where the reference's indexing raises."""
        for t, n, what in ((ids, self.vocab, "token id"), (positions, self.max_pos, "position")):
            if t.device.type == "cpu" and t.numel():
                lo, hi = int(t.min()), int(t.max())
                if lo < -n or hi >= n:
                    bad = lo if lo < -n else hi
                    raise IndexError(f"{what} {bad} is out of bounds for dimension 0 "
                                     f"with size {n}")

    # reference-layout view of the LM head (model.py:136)
    @property
    def head_w8t(self) -> torch.Tensor:
        return self.head_w.t()

    # -- GEMM dispatch ---------------------------------------------------------
    def _ksplit(self, N: int, K: int, M: int = 1) -> int:
        key = (N, K, M > 1)  # the plan differs between one row and several
        ks = self._plans.get(key)
        if ks is None:
            ks = gemv_plan(M, N, K)
            self._plans[key] = ks
        return ks

    def _next_gemm(self, w, R: int):
        """Trailing arguments of a decode row kernel that name the skinny GEMM
        launched right after it (x . w^T over R rows, _gemm's K split): the
        row launch pulls w into the L2 caches meanwhile (a hint; results do
        not depend on it)."""
        if w is None or R > 64:
            return (None, 0, 0, 0)
        N, K = w.shape
        return (w, N, K, self._ksplit(N, K, R))

    def _gemm(self, x: torch.Tensor, w: torch.Tensor, prefetch=(), split: bool = True):
        """x . w^T as int32 partials [ks, R, N] (ks = 1 unless split and the
        skinny GEMM's plan splits K). prefetch: up to four device tensors the
        next kernels read; the skinny GEMM pulls them into the memory-side
        cache while it streams w (a hint, results unchanged)."""
        R, K = x.shape
        N = w.shape[0]
        if R > 64:
            return gemm_nt(x, w), 1, R * N
        ks = self._ksplit(N, K, R) if split else 1
        P = torch.empty(ks, R, N, dtype=torch.int32, device=self.device)
        pf = []
        for t in prefetch[:4]:
            pf += [t, t.numel() * t.element_size()]
        pf += [None, 0] * (4 - len(prefetch[:4]))
        call("detllm_igemv_nt_pf", x, w, P, R, N, K, ks, R * N, *pf)
        return P, ks, R * N

    # -- forward (model.py:220-286) ------------------------------------------------
    def forward(self, ids: torch.Tensor, positions: torch.Tensor, cache: KVCache | None = None,
                chunk_valid: torch.Tensor | None = None, guard: bool = False):
        """ids, positions: int64 [B, T]; chunk_valid: bool [B, T] (True = real).

        Returns (logits int32 [B, T, vocab], logit_row_m, logit_row_k, cache)."""
        if guard:
            with NoFloatMode():
                return self._forward(ids, positions, cache, chunk_valid)
        return self._forward(ids, positions, cache, chunk_valid)

    def _forward(self, ids, positions, cache, chunk_valid, head_rows=None):
        dev = self.device
        self._check_host_indices(ids, positions)
        ids = ids.to(device=dev, dtype=I64)
        positions = positions.to(device=dev, dtype=I64)
        B, T = ids.shape
        if cache is None:
            cache = KVCache()
        cache.check_rows(B)
        static = cache.static_cap > 0
        S_past = cache.length
        if static:
            # the step's slot flag is set before the replay (graphed.py)
            assert T == 1, "graphed (static-capacity) mode decodes one token per row"
            S = min(cache.static_cap, DEC_MAX_SLOTS)
        else:
            S = S_past + T
            cache.reserve(self, B, S)
            if chunk_valid is None:
                cache.valid_buf[:, S_past:S] = True
            else:
                cache.valid_buf[:, S_past:S] = chunk_valid.to(dev)
        H, R = self.hidden, B * T
        # one decode row: the GEMVs run their operand's row kernel themselves
        # (at 2+ rows the fused prologue gives each row one wave, whose chain
        # over 16+ columns per lane outlasts the separate launches: c3 b8
        # 2.38 vs 1.53 ms per step, b1 1.30 vs 1.64 the other way round)
        fused = (T == 1 and R <= self.fused_decode_rows
                 and self._fused_decode[1 if R == 1 else 2])
        # the fused decode stack double-buffers the residual (h = buffer 0)
        hb = torch.empty(2 if fused else 1, R, H, dtype=torch.int32, device=dev)
        kb = torch.empty(2 if fused else 1, R, dtype=I64, device=dev)
        h, k_res = hb[0], kb[0]
        x8 = torch.empty(R, H, dtype=torch.int8, device=dev)
        xm = torch.empty(R, dtype=I64, device=dev)
        xk = torch.empty(R, dtype=I64, device=dev)
        L0 = self.layers[0]
        call("detllm_embed_normq", ids.contiguous().view(-1), R, H, self.vocab, self.embed_e8,
             self.embed_m, self.embed_k, h, k_res, L0.as_m, L0.as_k, x8, xm, xk, self._err)
        pos = positions.contiguous().view(-1)
        if fused:
            self._layers_fused(B, hb, kb, x8, xm, xk, pos, cache, S_past, S, static)
        else:
            for li, L in enumerate(self.layers):
                nxt = self.layers[li + 1] if li + 1 < self.n_layers else None
                self._layer(L, nxt, B, T, h, k_res, x8, xm, xk, pos, cache, S_past, S, static)
        if not static:
            cache.length = S
        if head_rows is not None:
            sel = (torch.arange(B, device=dev), head_rows)
            logits = self._lm_head(x8.view(B, T, H)[sel].contiguous(), xm.view(B, T)[sel],
                                   xk.view(B, T)[sel])
            return logits, xm.view(B, T, 1), xk.view(B, T, 1), cache
        logits = self._lm_head(x8.view(B, T, H), xm.view(B, T, 1), xk.view(B, T, 1))
        return logits, xm.view(B, T, 1), xk.view(B, T, 1), cache

    # -- seams (model.py:430-432, :469-478): override points for diagnostics --------
    def _lm_head(self, x8: torch.Tensor, xm: torch.Tensor, xk: torch.Tensor) -> torch.Tensor:
        """Seam: the LM head GEMM, x8 [..., H] int8 -> int32 [..., vocab]
        (xm/xk unused on the integer path, model.py:430-432)."""
        lead = x8.shape[:-1]
        x2 = x8.reshape(-1, self.hidden).contiguous()
        logits = self._gemm(x2, self.head_w, (self.head_m,), split=False)[0][0]
        return logits.view(*lead, self.vocab)

    def _attn_scores(self, q8, qm, qk, K8r, L, group, aux=None):
        """Seam (model.py:469-474): int8 Q.K^T with the per-row dyadic score
        scale. Called by prefill only when a subclass overrides a seam; the
        default prefill runs the fused attention kernel, same bits."""
        scores = int_gemm(q8, K8r.transpose(-1, -2).contiguous(), self.backend)
        ks_m = L.ks_m.repeat_interleave(group).view(1, self.n_q, 1, 1)
        ks_k = L.ks_k.repeat_interleave(group).view(1, self.n_q, 1, 1)
        return (scores,) + dy.norm_scale(qm * ks_m, qk + ks_k)

    def _attn_context(self, probs, V8r, L, aux=None):
        """Seam (model.py:476-478): 15-bit probabilities x int8 V, exact
        hi/lo split (backends.py:152-164)."""
        return int_gemm_u16i8(probs, V8r, self.backend)

    def _norm_quant(self, h: torch.Tensor, k_res: torch.Tensor,
                    sm_m: torch.Tensor | None = None, sm_k: int = 0):
        """model.py:187-198 on the op kernels: RMSNorm (scale (1, 20)), the
        optional smoothing multiply, per-token int8 quantisation. The layer
        kernels fuse the same integers; this form serves code written
        against the reference class."""
        y = ops.di_rmsnorm(h)
        kq = torch.full_like(k_res, OUT_FRAC_BITS)
        if sm_m is not None:
            y = y.to(I64) * sm_m
            kq = kq + sm_k
        return dy.quant_i8_pertoken(y, torch.ones_like(k_res), kq)

    def enable_layer_compile(self):
        """model.py:452-467 compiles the per-layer function with inductor;
        every layer here is already a fixed sequence of hand-fused kernels,
        so there is nothing to compile (kept for the same API)."""

    def enable_layer_cudagraphs(self):
        """model.py:434-450; see enable_layer_compile. The whole decode step
        is one HIP graph (GraphedDecode)."""

    def _seams_overridden(self) -> bool:
        cls = type(self)
        return (cls._attn_scores is not IntQwen3._attn_scores
                or cls._attn_context is not IntQwen3._attn_context)

    def _qk_head_pipeline(self, P, row_m, row_k, w_m, w_k, gamma_m, gamma_k, n_heads,
                          positions):
        """model.py:200-216 on the op kernels: per-(token, head)
        requant_i32_common(16), di_rmsnorm_gamma, permute, RoPE. P [B, T,
        n_heads * hd] int32 -> (int64 [B, n_heads, T, hd], k). The fused
        epilogue computes the same integers; this form feeds the seams'
        diagnostics."""
        B, T, _ = P.shape
        Ph = P.view(B, T, n_heads, self.hd)
        cm = w_m.view(n_heads, self.hd)
        y, _, _ = dy.requant_i32_common(Ph, row_m.unsqueeze(-1), row_k.unsqueeze(-1), cm, w_k,
                                        target_bits=16)
        yn, k_out = ops.di_rmsnorm_gamma(y, gamma_m, gamma_k)
        yn = yn.permute(0, 2, 1, 3)
        pos = positions.view(B, 1, T).expand(B, n_heads, T)
        return ops.apply_int_rope(yn, self.rope_cos, self.rope_sin, pos), k_out

    def _layer(self, L: LayerWeights, nxt, B, T, h, k_res, x8, xm, xk, pos, cache: KVCache,
               S_past, S, static):
        P, ns, st = self._gemm(x8, L.wqkv, (L.pf_attn,))
        attn = self._attend(L, B, T, P, ns, st, xm, xk, pos, cache, S_past, S, static)
        self._after_attention(L, nxt, B, T, attn, h, k_res, x8, xm, xk)

    def _split_plan(self, B: int, S: int):
        """(chunk, nsplit) of the split-S decode attention, or None when the
        one-block-per-(row, kv head) kernel is used (fewer slots than
        SPLIT_MIN_SLOTS, or one chunk)."""
        if S < SPLIT_MIN_SLOTS:
            return None
        key = (B, S)
        plan = self._split_plans.get(key)
        if plan is None:
            plan = attn_split_plan(B, S, self.n_q, self.n_kv)
            self._split_plans[key] = plan
        return plan if plan[1] > 1 else None

    def _attend(self, L: LayerWeights, B, T, P, ns, st, xm, xk, pos, cache: KVCache, S_past, S,
                static):
        """Q/K/V epilogue (cache write) and attention of one layer from the
        QKV partials P. Returns (attn, nsplit, split_stride, ext): int64
        context partials [nsplit][B * T][n_q * hd] whose sum is the context,
        and the merge statistics [B][n_kv][2] of a decode step's context
        (detllm_qkv_attn_decode_ext), else None."""
        dev = self.device
        R, nq, nkv, hd = B * T, self.n_q, self.n_kv, self.hd
        li = L.idx
        valid = cache.valid_buf.view(torch.uint8)
        plan = self._split_plan(B, S) if T == 1 else None
        if plan is not None:
            # long rows: Q/K/V epilogue, then the split-S attention
            chunk, nsp = plan
            q8 = torch.empty(B, nq, 1, hd, dtype=torch.int8, device=dev)
            tpos = torch.empty(B, nq, 1, dtype=I64, device=dev)
            call("detllm_qkv_epilogue", P, ns, st, B, 1, nq, nkv, xm, xk, pos,
                 L.q_m, L.q_k, L.k_m, L.k_k, L.v_m, L.v_k, L.q_norm_m, L.q_norm_k,
                 L.k_norm_m, L.k_norm_k, L.qs_m, L.qs_k, L.kq_m, L.kq_k, L.ks_m, L.ks_k,
                 L.vq_m, L.vq_k, self.rope_cos, self.rope_sin, self.max_pos, q8, tpos, None,
                 *cache.layer_args(li), cache.len_idx if static else None,
                 0 if static else S_past, L.kq_est, self._err)
            scores = torch.empty(B, nq, nsp * chunk, dtype=torch.int32, device=dev)
            cmax = torch.empty(B, nq, nsp, dtype=torch.int32, device=dev)
            attn = torch.empty(nsp, R, nq * hd, dtype=I64, device=dev)
            call("detllm_attn_decode_split", q8, tpos, *cache.layer_args(li), valid, cache.cap,
                 B, S, nq, nkv, cache.nslots if static else None, chunk, scores, cmax, attn,
                 self._err)
            return attn, nsp, R * nq * hd, None
        attn = torch.empty(R, nq * hd, dtype=I64, device=dev)
        if T == 1 and nq // nkv <= 2:
            # decode: Q/K/V epilogue and attention in one launch
            scratch = self._decode_scratch(B, S)
            args = (P, ns, st, B, nq, nkv, xm, xk, pos,
                    L.q_m, L.q_k, L.k_m, L.k_k, L.v_m, L.v_k, L.q_norm_m, L.q_norm_k,
                    L.k_norm_m, L.k_norm_k, L.qs_m, L.qs_k, L.kq_m, L.kq_k, L.ks_m, L.ks_k,
                    L.vq_m, L.vq_k, self.rope_cos, self.rope_sin, self.max_pos,
                    *cache.layer_args(li), cache.len_idx if static else None,
                    0 if static else S_past, valid, cache.cap, S,
                    cache.nslots if static else None, scratch, attn, self._err)
            if B <= MERGE_EXT_ROWS and nq * hd <= 2048 and nkv <= 8:
                # with the merge's row statistics, for the o-GEMV that
                # quantises its own K range of the operand
                ext = torch.empty(B, nkv, 2, dtype=I64, device=dev)
                call("detllm_qkv_attn_decode_ext", *args, L.osc_m, ext)
                return attn, 1, 0, ext
            call("detllm_qkv_attn_decode", *args)
        elif T > 1 and self._seams_overridden():
            self._attention_seams(L, B, T, P, ns, st, xm, xk, pos, cache, S_past, S, attn)
        else:
            self._attention(L, B, T, P, ns, st, xm, xk, pos, cache, S_past, S, static, attn)
        return attn, 1, 0, None

    def _partials(self, R: int, N: int, K: int):
        ks = self._ksplit(N, K, R)
        return torch.empty(ks, R, N, dtype=torch.int32, device=self.device), ks, R * N

    def _layers_fused(self, B, hb, kb, x8, xm, xk, pos, cache, S_past, S, static):
        """The decoder stack for a decode row (T == 1, B == 1) with each
        skinny GEMM's operand row kernel fused into it (detllm_igemv_merge,
        detllm_igemv_resnormq, detllm_igemv_swiglu): per layer
        QKV-GEMM(+residual_normq of the previous layer's down product) ->
        attention -> o-GEMM(+merge) -> gate|up-GEMM(+residual_normq of the o
        product) -> down-GEMM(+SwiGLU);
        the same integers as _layer's sequence. The residual alternates
        between two buffers (a fused launch reads one while its lead block
        writes the other): hb [2, B, H], kb [2, B] with the embedding's
        residual in buffer 0."""
        dev = self.device
        R, H, nq, hd, I_ = B, self.hidden, self.n_q, self.hd, self.inter
        cur = 0
        am = torch.empty(R, dtype=I64, device=dev)
        ak = torch.empty(R, dtype=I64, device=dev)
        y8 = torch.empty(R, I_, dtype=torch.int8, device=dev)
        ym = torch.empty(R, dtype=I64, device=dev)
        yk = torch.empty(R, dtype=I64, device=dev)
        L0 = self.layers[0]
        P, ns, st = self._gemm(x8, L0.wqkv, (L0.pf_attn,))
        for li, L in enumerate(self.layers):
            nxt = self.layers[li + 1] if li + 1 < self.n_layers else None
            attn = self._attend(L, B, 1, P, ns, st, xm, xk, pos, cache, S_past, S, static)
            Po, nso, sto = self._partials(R, H, nq * hd)
            if attn[3] is not None:
                call("detllm_igemv_merge_ext", L.wo, Po, R, H, nq * hd, nso, sto, attn[0],
                     L.osc_m, L.os_k, L.attn_out_col_k, attn[3], self.n_kv, am, ak, 0,
                     L.pf_o, L.pf_o.numel() * 8, None, 0)
            else:
                call("detllm_igemv_merge", L.wo, Po, R, H, nq * hd, nso, sto, *attn[:3],
                     L.osc_m, L.os_k, None, L.attn_out_col_k, am, ak, L.pf_o,
                     L.pf_o.numel() * 8, None, 0)
            Pg, nsg, stg = self._partials(R, 2 * I_, H)
            call("detllm_igemv_resnormq", L.wgu, Pg, R, 2 * I_, H, nsg, stg, Po, nso, sto, am, ak,
                 L.o_m, L.o_k, 20, hb[cur], kb[cur], hb[1 - cur], kb[1 - cur], L.ms_m, L.ms_k,
                 xm, xk, L.pf_mlp, L.pf_mlp.numel() * 8, None, 0)
            cur = 1 - cur
            pfd = (L.down_m,) if nxt is None else (L.down_m, nxt.as_m)
            ksd = self.fused_swiglu_ksplit
            if ksd and I_ % 512 == 0 and I_ <= 3072 and pro_fits(I_, ksd):
                # the down GEMV computes its SwiGLU operand row itself
                Pd = torch.empty(ksd, R, H, dtype=torch.int32, device=dev)
                nsd, std = ksd, R * H
                pf = []
                for t in pfd:
                    pf += [t, t.numel() * t.element_size()]
                pf += [None, 0] * (2 - len(pfd))
                call("detllm_igemv_swiglu", L.wd, Pd, H, I_, ksd, std, Pg, nsg, stg, xm, xk,
                     L.gate_m, L.gate_k, L.up_m, L.up_k, L.ds_m, L.ds_k, ym, yk, 0, *pf)
            else:
                call("detllm_swiglu_quant", Pg, nsg, stg, R, I_, xm, xk, L.gate_m, L.gate_k,
                     L.up_m, L.up_k, L.ds_m, L.ds_k, y8, ym, yk, *self._next_gemm(L.wd, R), 0)
                Pd, nsd, std = self._gemm(y8, L.wd, pfd)
            if nxt is None:
                call("detllm_residual_normq", Pd, nsd, std, R, H, ym, yk, L.down_m, L.down_k, 20,
                     hb[cur], kb[cur], None, 0, x8, xm, xk, None, 0, 0, 0, 0)
                break
            N = nxt.wqkv.shape[0]
            P, ns, st = self._partials(R, N, H)
            call("detllm_igemv_resnormq", nxt.wqkv, P, R, N, H, ns, st, Pd, nsd, std, ym, yk,
                 L.down_m, L.down_k, 20, hb[cur], kb[cur], hb[1 - cur], kb[1 - cur], nxt.as_m,
                 nxt.as_k, xm, xk, nxt.pf_attn, nxt.pf_attn.numel() * 8, None, 0)
            cur = 1 - cur

    def _decode_scratch(self, B, S):
        """Global score scratch of the decode attention when the scores of a
        (row, kv-head) do not fit its 48 KiB of LDS."""
        G = self.n_q // self.n_kv
        Spad = (S + 15) // 16 * 16
        if G * Spad * 4 <= 48 * 1024:
            return None
        return torch.empty(B, self.n_q, Spad, dtype=torch.int32, device=self.device)

    def _attention(self, L, B, T, P, ns, st, xm, xk, pos, cache, S_past, S, static, attn):
        dev = self.device
        nq, nkv, hd, li = self.n_q, self.n_kv, self.hd, L.idx
        q8 = torch.empty(B, nq, T, hd, dtype=torch.int8, device=dev)
        tpos = torch.empty(B, nq, T, dtype=I64, device=dev)
        call("detllm_qkv_epilogue", P, ns, st, B, T, nq, nkv, xm, xk, pos,
             L.q_m, L.q_k, L.k_m, L.k_k, L.v_m, L.v_k, L.q_norm_m, L.q_norm_k,
             L.k_norm_m, L.k_norm_k, L.qs_m, L.qs_k, L.kq_m, L.kq_k, L.ks_m, L.ks_k,
             L.vq_m, L.vq_k, self.rope_cos, self.rope_sin, self.max_pos, q8, tpos, None,
             *cache.layer_args(li), cache.len_idx if static else None,
             0 if static else S_past, L.kq_est, self._err)
        valid = cache.valid_buf.view(torch.uint8)
        if T == 1:
            call("detllm_attn_decode", q8, tpos, *cache.layer_args(li), valid, cache.cap,
                 B, S, nq, nkv, cache.nslots if static else None,
                 self._decode_scratch(B, S), attn, self._err)
        else:
            call("detllm_attn_prefill", q8, tpos, *cache.layer_args(li), valid, cache.cap,
                 B, T, S_past, nq, nkv, attn)

    def _attention_seams(self, L, B, T, P, ns, st, xm, xk, pos, cache, S_past, S, attn):
        """Prefill attention through the overridable seams, as the
        reference's prefill branch runs it (model.py:382-402): K/V are
        requantised into the cache by the fused epilogue (which also yields
        q8 and its scale (qm, qk)); the scores come from _attn_scores, the
        probabilities from di_softmax, the context from _attn_context, query
        chunk by query chunk under the reference's memory budget. aux carries
        the reference's diagnostics (model.py:385-386)."""
        dev = self.device
        nq, nkv, hd, li = self.n_q, self.n_kv, self.hd, L.idx
        group = nq // nkv
        q8 = torch.empty(B, nq, T, hd, dtype=torch.int8, device=dev)
        tpos = torch.empty(B, nq, T, dtype=I64, device=dev)
        dbg = torch.empty(B, nq, T, 4, dtype=I64, device=dev)
        call("detllm_qkv_epilogue", P, ns, st, B, T, nq, nkv, xm, xk, pos,
             L.q_m, L.q_k, L.k_m, L.k_k, L.v_m, L.v_k, L.q_norm_m, L.q_norm_k,
             L.k_norm_m, L.k_norm_k, L.qs_m, L.qs_k, L.kq_m, L.kq_k, L.ks_m, L.ks_k,
             L.vq_m, L.vq_k, self.rope_cos, self.rope_sin, self.max_pos, q8, tpos, dbg,
             *cache.layer_args(li), None, S_past, L.kq_est, self._err)
        qm, qk = dbg[..., 0:1], dbg[..., 1:2]
        Pfull = P.view(ns, B, T, -1).sum(dim=0, dtype=torch.int32) if ns > 1 else \
            P.view(B, T, -1)
        nqc, nkc = nq * hd, nkv * hd
        Pq, Pk, Pv = Pfull[..., :nqc], Pfull[..., nqc:nqc + nkc], Pfull[..., nqc + nkc:]
        xm3, xk3 = xm.view(B, T, 1), xk.view(B, T, 1)
        positions = pos.view(B, T)
        q, qkk = self._qk_head_pipeline(Pq.contiguous(), xm3, xk3, L.q_m, L.q_k, L.q_norm_m,
                                        L.q_norm_k, nq, positions)
        kk, kkk = self._qk_head_pipeline(Pk.contiguous(), xm3, xk3, L.k_m, L.k_k, L.k_norm_m,
                                         L.k_norm_k, nkv, positions)
        aux = {"li": li, "q": q, "qkk": qkk, "kk": kk, "kkk": kkk, "Pv": Pv.contiguous(),
               "xm": xm3, "xk": xk3, "L": L}
        K8 = cache._gather(li, "k", S)
        V8 = cache._gather(li, "v", S)
        K8r = K8.repeat_interleave(group, dim=1).contiguous()
        V8r = V8.repeat_interleave(group, dim=1).contiguous()
        slot = torch.arange(S, device=dev)
        causal = slot[None, :] <= (S_past + torch.arange(T, device=dev))[:, None]
        mask = cache.valid_buf[:, None, None, :S] & causal[None, None]
        budget = max(1, (1 << 27) // max(1, B * nq * S))
        CH = T if T <= budget else max(128, budget)
        parts = []
        for qlo in range(0, T, CH):
            qhi = min(qlo + CH, T)
            scores, sm, sk = self._attn_scores(q8[:, :, qlo:qhi], qm[:, :, qlo:qhi],
                                               qk[:, :, qlo:qhi], K8r, L, group, aux)
            probs = ops.di_softmax(scores, sm, sk,
                                   mask[:, :, qlo:qhi].expand(B, nq, qhi - qlo, S))
            parts.append(self._attn_context(probs, V8r, L, aux))
        a = torch.cat(parts, dim=2) if len(parts) > 1 else parts[0]
        attn.copy_(a.permute(0, 2, 1, 3).reshape(B * T, nq * hd))

    def _after_attention(self, L, nxt, B, T, attn, h, k_res, x8, xm, xk):
        """attn: (context partials, nsplit, split_stride) as _attend returns."""
        dev = self.device
        R, H, nq, hd, I_ = B * T, self.hidden, self.n_q, self.hd, self.inter
        a8 = torch.empty(R, nq * hd, dtype=torch.int8, device=dev)
        am = torch.empty(R, dtype=I64, device=dev)
        ak = torch.empty(R, dtype=I64, device=dev)
        # decode sizes: the merge and the SwiGLU leave their scale fits to the
        # residual kernel after the next GEMM (same integers)
        dfit = 1 if R <= 64 else 0
        if attn[3] is not None:
            # the merge from the attention's row statistics: elementwise, in
            # 256-column pieces (no row reduction)
            call("detllm_merge_ext", attn[0], R, nq * hd, L.osc_m, L.os_k, L.attn_out_col_k,
                 attn[3], self.n_kv, a8, am, ak, *self._next_gemm(L.wo, R), dfit)
        else:
            call("detllm_merge_rowcol", *attn[:3], R, nq * hd, L.os_m, L.os_k,
                 L.attn_out_col_m, L.attn_out_col_k, a8, am, ak, *self._next_gemm(L.wo, R), dfit)
        P, ns, st = self._gemm(a8, L.wo, (L.pf_o,))
        call("detllm_residual_normq", P, ns, st, R, H, am, ak, L.o_m, L.o_k, 20, h, k_res,
             L.ms_m, L.ms_k, x8, xm, xk, *self._next_gemm(L.wgu, R), dfit)
        P, ns, st = self._gemm(x8, L.wgu, (L.pf_mlp,))
        y8 = torch.empty(R, I_, dtype=torch.int8, device=dev)
        ym = torch.empty(R, dtype=I64, device=dev)
        yk = torch.empty(R, dtype=I64, device=dev)
        call("detllm_swiglu_quant", P, ns, st, R, I_, xm, xk, L.gate_m, L.gate_k, L.up_m,
             L.up_k, L.ds_m, L.ds_k, y8, ym, yk, *self._next_gemm(L.wd, R), dfit)
        P, ns, st = self._gemm(y8, L.wd, (L.down_m,) if nxt is None else (L.down_m, nxt.as_m))
        sm_m, sm_k = (nxt.as_m, nxt.as_k) if nxt is not None else (None, 0)
        call("detllm_residual_normq", P, ns, st, R, H, ym, yk, L.down_m, L.down_k, 20, h, k_res,
             sm_m, sm_k, x8, xm, xk, *self._next_gemm(None if nxt is None else nxt.wqkv, R), dfit)

    # -- decoding (model.py:482-531) ------------------------------------------------
    def greedy_pick(self, logits_row: torch.Tensor) -> torch.Tensor:
        """Integer argmax of logits*head_m (int64) with the lowest-id tie-break."""
        lr = logits_row.to(device=self.device, dtype=torch.int32).contiguous()
        R = lr.shape[0]
        nch = -(-self.vocab // GREEDY_CHUNK)
        key = R
        sc = self._greedy_scratch.get(key)
        if sc is None or torch.cuda.is_current_stream_capturing():
            sc = (torch.empty(R, nch, dtype=I64, device=self.device),
                  torch.empty(R, nch, dtype=I64, device=self.device))
            if not torch.cuda.is_current_stream_capturing():
                self._greedy_scratch[key] = sc
        out = torch.empty(R, dtype=I64, device=self.device)
        call("detllm_greedy_pick", lr, self.head_m, R, self.vocab, GREEDY_CHUNK, sc[0], sc[1],
             out)
        return out

    @torch.no_grad()
    def generate(self, ids: torch.Tensor, max_new: int, guard: bool = False,
                 chunk_valid: torch.Tensor | None = None, stop_at_eos: bool = False,
                 use_graph: bool = False):
        """Greedy generation; ids int64 [B, T0] right-padded (pads False in
        chunk_valid). Returns (tokens [B, max_new], step_logits list of [B, V])."""
        dev = self.device
        B, T0 = ids.shape
        self._check_host_indices(ids, torch.zeros(1, dtype=I64))
        ids = ids.to(dev)
        if chunk_valid is None:
            chunk_valid = torch.ones(B, T0, dtype=torch.bool, device=dev)
        chunk_valid = chunk_valid.to(dev)
        positions = torch.arange(T0, device=dev).expand(B, T0)
        lens = chunk_valid.sum(dim=1)
        # prefill reads positions 0 .. T0 - 1 and decode step s (1 <= s <
        # max_new) position lens + s - 1; the reference's cos_t[positions]
        # raises IndexError at the first position >= max_pos, so refuse up
        # front rather than after that many steps
        last_pos = max(T0 - 1, int(lens.max()) + max_new - 2 if max_new > 1 else -1)
        if last_pos >= self.max_pos:
            raise IndexError(f"generation reaches position {last_pos}, outside the RoPE "
                             f"tables (size {self.max_pos})")
        last = (lens - 1).clamp(min=0)
        # the cache is sized for the whole generation up front: decoding then
        # only maps pages (no reallocation, no copy, one graph capture)
        cache = KVCache().plan(self, B, T0 + max_new)
        if guard:
            with NoFloatMode():
                first, _, _, cache = self._forward(ids, positions, cache, chunk_valid, last)
        else:
            first, _, _, cache = self._forward(ids, positions, cache, chunk_valid, last)
        step_logits = [first]
        cur = self.greedy_pick(first)
        out = [cur]
        if use_graph and max_new > 1:
            from .graphed import GraphedDecode
            gd = GraphedDecode(self, cache, lens)
            for _ in range(1, max_new):
                lg = gd.step(cur).clone()
                step_logits.append(lg)
                cur = self.greedy_pick(lg)
                out.append(cur)
            self.raise_if_device_error()
            return torch.stack(out, dim=1), step_logits
        ones = torch.ones(B, 1, dtype=torch.bool, device=dev)
        for step in range(1, max_new):
            pos = (lens + step - 1).unsqueeze(1)
            lg, _, _, cache = self.forward(cur.unsqueeze(1), pos, cache, ones, guard)
            step_logits.append(lg[:, 0])
            cur = self.greedy_pick(lg[:, 0])
            out.append(cur)
        self.raise_if_device_error()
        return torch.stack(out, dim=1), step_logits
