"""Graph-captured decode (the contract of the reference's graphed.py:43-132).

The whole decode step — 28 layers of fused HIP kernels plus the LM head — is
recorded once into a HIP graph (torch.cuda.CUDAGraph, which is hipGraph on
ROCm) and replayed per token. Static-shape decode stays bit-exact by
construction:
  * the cache's page tables cover a fixed bucketed capacity (256 * 2^n
    slots); attention scans the filled slots (a device-side slot count bounds
    the scan) and the validity mask excludes everything else, exactly as a
    length-wide computation;
  * the K/V write slot is a device scalar (``len_idx``), so every replay
    writes the same bytes to the same slot as the eager path;
  * pages are mapped into the tables as the steps reach them, in place, so
    the captured graph keeps running; bucket overflow widens the tables (no
    K/V bytes move) and the next step recaptures, as does a page pool that
    had to be reallocated.
The graph contains kernel launches only (no memset nodes, no host reads).

``mode`` and ``layer_compile`` are the reference's arguments
(graphed.py:44-45). mode="capture" (default) replays the whole-step graph;
mode="layers" runs the same static-capacity step as eager launches of the
fused layer kernels (where the reference hands per-layer graphs to
inductor). ``layer_compile`` is accepted for the same signature: the
reference compiles its generic layer with inductor, and here every layer is
already a fixed sequence of hand-fused kernels, so there is nothing to
compile. Both modes give the same bits.
"""

from __future__ import annotations

import torch

from ._lib import call
from .model import DEC_MAX_SLOTS, GREEDY_CHUNK, IntQwen3, KVCache

I64 = torch.int64


def _next_bucket(n: int) -> int:
    cap = 256
    while cap < n:
        cap *= 2
    return cap


class GraphedDecode:
    def __init__(self, model: IntQwen3, cache: KVCache, lens: torch.Tensor,
                 mode: str = "capture", layer_compile: bool = True):
        """cache: as returned by a prefill ``forward``; lens: int64 [B] true
        prompt lengths (the next token's position per row); mode "capture"
        (whole-step graph) or "layers" (eager static-capacity step)."""
        if getattr(model, "backend", None) != "rocm":
            raise ValueError("GraphedDecode drives the rocm backend's IntQwen3")
        if mode not in ("capture", "layers"):
            raise ValueError(f"unknown mode {mode!r}; expected 'capture' or 'layers'")
        self.mode = mode
        self.layer_compile = bool(layer_compile)
        self.model = model
        self.cache = cache
        dev = model.device
        self.B = cache.valid_buf.shape[0]
        self.length = cache.length
        self.steps = 0
        self.ids_buf = torch.zeros(self.B, 1, dtype=I64, device=dev)
        self.pos0 = lens.to(dev).to(I64).contiguous().view(self.B).clone()
        self.pos_buf = self.pos0.view(self.B, 1).clone()
        cache.len_idx = torch.zeros(1, dtype=I64, device=dev)
        cache.nslots = torch.zeros(1, dtype=I64, device=dev)
        nch = -(-model.vocab // GREEDY_CHUNK)
        self._pick_scratch = (torch.empty(self.B, nch, dtype=I64, device=dev),
                              torch.empty(self.B, nch, dtype=I64, device=dev))
        self.graph = None        # forward only (step)
        self.graph_pick = None   # forward + greedy pick into ids_buf (step_greedy)
        self.out = None
        self.out_pick = None
        self._grow_to(_next_bucket(self.length + 1))

    def _grow_to(self, cap: int):
        if self.length + 1 > DEC_MAX_SLOTS:
            raise IndexError(f"decode past {DEC_MAX_SLOTS} cache slots is not supported "
                             "(int32 accumulators of the decode attention)")
        self.cache.resize(cap)
        self.cache.static_cap = self.cache.cap   # a planned cache may already be wider
        self.graph = None   # a captured graph references the old tables
        self.graph_pick = None

    def _map_next(self):
        """Pages for this step's slot (a no-op within a mapped page); a pool
        reallocation invalidates the captured graphs."""
        gen = self.cache.pool_generation
        self.cache.map_slots(self.length + 1)
        if self.cache.pool_generation != gen:
            self.graph = None
            self.graph_pick = None

    def _prologue(self):
        """Validity flag, write slot, scanned-slot count and positions of this
        step, one kernel (graphed.py:112-131 does them as separate ops)."""
        c = self.cache
        call("detllm_decode_prologue", c.valid_buf.view(torch.uint8), c.valid_buf.shape[1],
             self.B, self.length, c.len_idx, c.nslots, self.pos_buf, self.pos0, self.steps)

    def _advance(self):
        self.length += 1
        self.steps += 1
        self.cache.length = self.length

    def _pick_into_ids(self, logits):
        m = self.model
        call("detllm_greedy_pick", logits, m.head_m, self.B, m.vocab, GREEDY_CHUNK,
             self._pick_scratch[0], self._pick_scratch[1], self.ids_buf.view(self.B))

    def _run(self):
        logits, _, _, _ = self.model.forward(self.ids_buf, self.pos_buf, self.cache)
        return logits

    def _capture(self):
        # warm-up: real executions of this same step (idempotent: they write
        # the same K/V bytes to the same slot)
        for _ in range(3):
            self._run()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.out = self._run()
        self.graph = g

    def _capture_pick(self):
        # warm-up as in _capture (the forward only: the pick would overwrite
        # this step's input ids), then one graph of the forward and the pick
        for _ in range(3):
            self._run()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.out_pick = self._run()
            self._pick_into_ids(self.out_pick[:, 0])
        self.graph_pick = g

    @torch.no_grad()
    def step(self, cur_ids: torch.Tensor) -> torch.Tensor:
        """cur_ids int64 [B] (device). Returns int32 logits [B, vocab]; the
        buffer is reused by the next step — clone to keep."""
        c = self.cache
        if self.length + 1 > c.static_cap:
            self._grow_to(_next_bucket(self.length + 1))
        self._map_next()
        self._prologue()
        self.ids_buf.copy_(cur_ids.view(self.B, 1))
        if self.mode == "layers":
            self.out = self._run()
        else:
            if self.graph is None:
                self._capture()
            self.graph.replay()
        self._advance()
        return self.out[:, 0]

    @torch.no_grad()
    def step_greedy(self, cur_ids: torch.Tensor | None = None) -> torch.Tensor:
        """One greedy decode step with the pick (IntQwen3.greedy_pick) inside
        the captured graph: it reads this step's ids from the buffer the
        previous pick wrote (cur_ids, int64 [B], seeds it on the first call).
        Returns the picked ids, int64 [B] (the next step's input buffer —
        clone to keep); the step's logits are in ``self.out_pick[:, 0]``.
        Same tokens and logits as ``greedy_pick(step(cur_ids))``."""
        c = self.cache
        if self.length + 1 > c.static_cap:
            self._grow_to(_next_bucket(self.length + 1))
        self._map_next()
        self._prologue()
        if cur_ids is not None:
            self.ids_buf.copy_(cur_ids.view(self.B, 1))
        if self.mode == "layers":
            self.out_pick = self._run()
            self._pick_into_ids(self.out_pick[:, 0])
        else:
            if self.graph_pick is None:
                self._capture_pick()
            self.graph_pick.replay()
        self._advance()
        return self.ids_buf.view(self.B)
