"""Graph-captured decode (the contract of the reference's graphed.py:43-132).

The whole decode step — 28 layers of fused HIP kernels plus the LM head — is
recorded once into a HIP graph (torch.cuda.CUDAGraph, which is hipGraph on
ROCm) and replayed per token. Static-shape decode stays bit-exact by
construction:
  * the cache has a fixed bucketed capacity (256 * 2^n); attention scans the
    filled slots (a device-side slot count bounds the scan) and the validity
    mask excludes everything else, exactly as a length-wide computation;
  * the K/V write slot is a device scalar (``len_idx``), so every replay
    writes the same bytes to the same slot as the eager path;
  * bucket overflow reallocates the cache (filled slots copied verbatim) and
    the next step recaptures.
The graph contains kernel launches only (no memset nodes, no host reads).
"""

from __future__ import annotations

import torch

from .model import IntQwen3, KVCache

I64 = torch.int64


def _next_bucket(n: int) -> int:
    cap = 256
    while cap < n:
        cap *= 2
    return cap


class GraphedDecode:
    def __init__(self, model: IntQwen3, cache: KVCache, lens: torch.Tensor):
        """cache: as returned by a prefill ``forward``; lens: int64 [B] true
        prompt lengths (the next token's position per row)."""
        self.model = model
        self.cache = cache
        dev = model.device
        self.B = cache.valid_buf.shape[0]
        self.length = cache.length
        self.ids_buf = torch.zeros(self.B, 1, dtype=I64, device=dev)
        self.pos_buf = lens.to(dev).view(self.B, 1).clone().to(I64)
        cache.len_idx = torch.zeros(1, dtype=I64, device=dev)
        cache.nslots = torch.zeros(1, dtype=I64, device=dev)
        self.graph = None
        self.out = None
        self._grow_to(_next_bucket(self.length + 1))

    def _grow_to(self, cap: int):
        self.cache.resize(cap)
        self.cache.static_cap = cap
        self.graph = None   # a captured graph references the old buffers

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

    @torch.no_grad()
    def step(self, cur_ids: torch.Tensor) -> torch.Tensor:
        """cur_ids int64 [B] (device). Returns int32 logits [B, vocab]; the
        buffer is reused by the next step — clone to keep."""
        c = self.cache
        if self.length + 1 > c.static_cap:
            self._grow_to(_next_bucket(self.length + 1))
        c.valid_buf[:, self.length] = True
        c.len_idx.fill_(self.length)
        c.nslots.fill_(self.length + 1)
        self.ids_buf.copy_(cur_ids.view(self.B, 1))
        if self.graph is None:
            self._capture()
        self.graph.replay()
        self.length += 1
        c.length = self.length
        self.pos_buf += 1
        return self.out[:, 0]
