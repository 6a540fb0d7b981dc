"""Host logic of the paged KV cache (idempotent_llm_amd.kvcache) on the CPU:
page mapping, growth without moving filled pages, and the row-count check
that keeps a mismatched batch from reaching the kernels."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from idempotent_llm_amd.kvcache import PAGE, CacheRowsMismatch, KVCache


def _model():
    return SimpleNamespace(n_layers=2, n_kv=1, hd=128, device=torch.device("cpu"))


def test_rows_are_fixed_once_the_cache_holds_any():
    m = _model()
    c = KVCache()
    c.check_rows(5)                          # an empty cache takes any batch
    c.reserve(m, 2, 10)
    c.check_rows(2)
    for B in (1, 3):
        with pytest.raises(ValueError, match="rows"):
            c.reserve(m, B, 20)
        with pytest.raises(RuntimeError, match="rows"):  # the reference's torch.cat error class
            c.plan(m, B, 20)
    assert c._table_host.shape[0] == 2 and c.mapped == PAGE
    assert issubclass(CacheRowsMismatch, ValueError) and issubclass(CacheRowsMismatch, RuntimeError)


def test_growth_maps_pages_in_place():
    m = _model()
    c = KVCache().plan(m, 2, 3 * PAGE)
    assert c.width == 3 and c.mapped == 0
    gen = c.pool_generation
    c.map_slots(PAGE + 1)
    first = c._table_host.copy()
    assert (first[:, :2] >= 0).all() and (first[:, 2] < 0).all()
    assert len(np.unique(first[:, :2])) == 4
    c.map_slots(3 * PAGE)
    assert np.array_equal(c._table_host[:, :2], first[:, :2])   # filled pages never move
    assert c.pool_generation == gen                              # planned pool: no regrowth
    assert torch.equal(c.table, torch.from_numpy(c._table_host))
