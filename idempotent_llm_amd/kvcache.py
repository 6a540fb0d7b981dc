"""Paged int8 KV cache of the rocm runtime (the contract of the reference's
KVCache, src/detllm/model.py:67-102, with paged storage).

The reference keeps, per layer, one contiguous [B, n_kv, CAP, hd] K and V
buffer and grows them by reallocating and copying the filled prefix. Here
each layer owns a page pool and every row a page table:

* a page holds PAGE = 128 slots of all kv heads: K as [n_kv, 128 slots, 128]
  and V transposed as [n_kv, 128 channels, 128 slots] (the attention kernels
  read slot-contiguous bytes from both);
* ``table[b, j]`` (int32, device) is the page of row b's slots
  [128 j, 128 j + 128), -1 when not mapped; the same page ids serve every
  layer (each layer indexes its own pool with them);
* growing the cache maps free pages of the pool into the tables, so filled
  slots are never copied; only when a pool runs out of pages is it
  reallocated at twice the size (the pages keep their ids, and
  ``pool_generation`` tells a captured graph to capture again).

Slot semantics are the reference's: slot order is call order for every row,
``valid`` marks real tokens, ``length`` counts filled slots. Slots that are
not valid are never read as data by the kernels (their K/V bytes are
unspecified), which is why pools are not zero-filled.
"""

from __future__ import annotations

import numpy as np
import torch

PAGE = 128   # slots per page (csrc/common.h DI_PAGE)


class CacheRowsMismatch(RuntimeError, ValueError):
    """A batch whose row count differs from the rows the cache holds. The
    reference fails the same call in ``torch.cat([cache.valid, chunk_valid])``
    (a RuntimeError); here the check runs on the host before any kernel
    would index the page tables past their rows."""


class KVCache:
    def __init__(self):
        self.k_pools: list = []     # per layer [n_pages, n_kv, PAGE, hd] int8
        self.v_pools: list = []     # per layer [n_pages, n_kv, hd, PAGE] int8
        self.table = None           # [B, width] int32 device
        self._table_host = None     # numpy mirror of ``table``
        self.n_pages = 0            # pages handed out (ids 0 .. n_pages - 1)
        self.mapped = 0             # slots [0, mapped) are mapped on every row
        self.valid_buf = None       # [B, width * PAGE] bool
        self.length = 0
        self.static_cap = 0
        self.len_idx = None         # [1] int64 device: slot written by a graphed step
        self.nslots = None          # [1] int64 device: slots visible to a graphed step
        self.pool_generation = 0
        self._dims = None           # (n_layers, n_kv, hd, device)

    # -- reference-compatible surface ------------------------------------------
    @property
    def width(self) -> int:
        return 0 if self.table is None else int(self.table.shape[1])

    @property
    def cap(self) -> int:
        return self.width * PAGE

    @property
    def valid(self):
        return None if self.valid_buf is None else self.valid_buf[:, :self.length]

    def seq_len(self) -> int:
        return self.length

    @property
    def k8(self) -> list:
        """Per layer K in the reference layout [B, n_kv, length, hd] (a
        gathered copy, for inspection)."""
        return [self._gather(li, "k") for li in range(len(self.k_pools))]

    @property
    def v8(self) -> list:
        """Per layer V in the reference layout [B, n_kv, length, hd]."""
        return [self._gather(li, "v") for li in range(len(self.v_pools))]

    def _gather(self, li: int, which: str, S: int | None = None) -> torch.Tensor:
        """[B, n_kv, S, hd] of layer li (S defaults to ``length``); slots of
        pages that are not mapped read as 0."""
        S = self.length if S is None else S
        w = -(-S // PAGE)
        B = self.table.shape[0]
        tb = self.table[:, :w].long()
        ids = tb.clamp(min=0)
        if which == "k":
            pages = self.k_pools[li][ids]                       # [B, w, n_kv, PAGE, hd]
            out = pages.permute(0, 2, 1, 3, 4)
        else:
            pages = self.v_pools[li][ids]                       # [B, w, n_kv, hd, PAGE]
            out = pages.permute(0, 2, 1, 4, 3)
        n_kv, hd = out.shape[1], out.shape[-1]
        out = out.reshape(B, n_kv, w * PAGE, hd)[:, :, :S]
        live = (tb >= 0).repeat_interleave(PAGE, dim=1)[:, None, :S, None]
        return torch.where(live, out, torch.zeros_like(out))

    # -- storage ------------------------------------------------------------------
    def _ensure_pool(self, need_pages: int):
        n_layers, n_kv, hd, dev = self._dims
        have = self.k_pools[0].shape[0] if self.k_pools else 0
        if need_pages <= have:
            return
        new = max(need_pages, 2 * have)
        kp = [torch.empty(new, n_kv, PAGE, hd, dtype=torch.int8, device=dev)
              for _ in range(n_layers)]
        vp = [torch.empty(new, n_kv, hd, PAGE, dtype=torch.int8, device=dev)
              for _ in range(n_layers)]
        for li in range(len(self.k_pools)):
            kp[li][:self.n_pages] = self.k_pools[li][:self.n_pages]
            vp[li][:self.n_pages] = self.v_pools[li][:self.n_pages]
        self.k_pools, self.v_pools = kp, vp
        self.pool_generation += 1

    def _ensure_width(self, B: int, width: int):
        if self.table is not None and width <= self.width:
            return
        host = np.full((B, width), -1, dtype=np.int32)
        dev = self._dims[3]
        valid = torch.zeros(B, width * PAGE, dtype=torch.bool, device=dev)
        if self.table is not None:
            host[:, :self.width] = self._table_host
            valid[:, :self.valid_buf.shape[1]] = self.valid_buf
        self._table_host = host
        self.table = torch.from_numpy(host).to(dev)
        self.valid_buf = valid

    def map_slots(self, upto: int):
        """Map pages so every row's slots [0, upto) have one. Only new pages
        are written into the tables (in place: a captured graph keeps
        reading the same table buffer)."""
        if upto <= self.mapped:
            return
        need_w = -(-upto // PAGE)
        B = self._table_host.shape[0]
        assert need_w <= self.width, "map_slots beyond the table width"
        missing = np.argwhere(self._table_host[:, :need_w] < 0)
        if len(missing):
            self._ensure_pool(self.n_pages + len(missing))
            ids = np.arange(self.n_pages, self.n_pages + len(missing), dtype=np.int32)
            self._table_host[missing[:, 0], missing[:, 1]] = ids
            self.n_pages += len(missing)
            self.table.copy_(torch.from_numpy(self._table_host))
        self.mapped = need_w * PAGE

    def check_rows(self, B: int):
        """Raise CacheRowsMismatch unless the cache is empty or holds B rows."""
        if self._table_host is not None and self._table_host.shape[0] != B:
            raise CacheRowsMismatch(
                f"a batch of {B} rows cannot use a KV cache of "
                f"{self._table_host.shape[0]} rows")

    def _init(self, model, B: int):
        self.check_rows(B)
        if self._dims is None:
            self._dims = (model.n_layers, model.n_kv, model.hd, model.device)
            self._ensure_width(B, 1)

    def plan(self, model, B: int, slots: int) -> "KVCache":
        """Size the tables and the page pools for ``slots`` slots per row up
        front (a caller that knows its longest sequence, e.g. generate with
        max_new): growth up to that length then only maps pages — nothing is
        reallocated or copied and a captured decode graph is never
        captured again."""
        self._init(model, B)
        w = max(1, -(-slots // PAGE))
        self._ensure_width(B, w)
        self._ensure_pool(B * w)
        return self

    def reserve(self, model, B: int, need: int):
        """Dynamic (prefill / eager decode) growth: table width at least
        ``need`` slots (doubling), pages mapped for slots [0, need)."""
        self._init(model, B)
        if need > self.cap:
            self._ensure_width(B, max(-(-need // PAGE), 2 * self.width))
        self.map_slots(need)

    def resize(self, cap: int):
        """Static (graphed) capacity: the table covers ``cap`` slots; pages
        are mapped as the steps reach them (graphed.py)."""
        assert cap % PAGE == 0
        B = self._table_host.shape[0]
        self._ensure_width(B, cap // PAGE)

    def layer_args(self, li: int):
        """(K pool, V pool, table, width) of layer li for the C ABI."""
        return self.k_pools[li], self.v_pools[li], self.table, self.width


def pages_from_contiguous(kc: torch.Tensor, vc: torch.Tensor, seed: int | None = None):
    """Paged copy of a contiguous cache: kc [B, n_kv, cap, hd], vc (V^T)
    [B, n_kv, hd, cap] with cap % PAGE == 0 -> (k_pool, v_pool, table). With
    ``seed`` the page ids are a seeded permutation (rows interleaved, so
    lookups must go through the table)."""
    B, n_kv, cap, hd = kc.shape
    w = cap // PAGE
    n = B * w
    order = np.arange(n, dtype=np.int32)
    if seed is not None:
        order = np.random.default_rng(seed).permutation(n).astype(np.int32)
    table = torch.from_numpy(order.reshape(B, w)).to(kc.device)
    kp = torch.empty(n, n_kv, PAGE, hd, dtype=torch.int8, device=kc.device)
    vp = torch.empty(n, n_kv, hd, PAGE, dtype=torch.int8, device=kc.device)
    kpages = kc.reshape(B, n_kv, w, PAGE, hd).permute(0, 2, 1, 3, 4).reshape(n, n_kv, PAGE, hd)
    vpages = vc.reshape(B, n_kv, hd, w, PAGE).permute(0, 3, 1, 2, 4).reshape(n, n_kv, hd, PAGE)
    idx = table.reshape(-1).long()
    kp[idx] = kpages
    vp[idx] = vpages
    return kp, vp, table
