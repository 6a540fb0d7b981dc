"""detllm_greedy_pick_noalloc — the allocation-free greedy pick — against
detllm_greedy_pick (the entry point with caller scratch), through the C ABI:
two calls in a row on the same GPU, the second with a smaller input (the
library's scratch keeps the first call's partials and must not leak them
into the second), plus the size limit."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
I64 = torch.int64


def _pick_with_scratch(rows, head_m, chunk=2048):
    from idempotent_llm_amd._lib import call
    R, V = rows.shape
    nch = -(-V // chunk)
    pv = torch.empty(R, nch, dtype=I64, device="cuda")
    pi = torch.empty(R, nch, dtype=I64, device="cuda")
    out = torch.empty(R, dtype=I64, device="cuda")
    call("detllm_greedy_pick", rows, head_m, R, V, chunk, pv, pi, out)
    return out


def _pick_noalloc(rows, head_m):
    from idempotent_llm_amd._lib import call
    R, V = rows.shape
    out = torch.full((R,), -1, dtype=I64, device="cuda")
    call("detllm_greedy_pick_noalloc", rows, head_m, R, V, out)
    return out


def test_noalloc_pick_matches_pick_twice_then_smaller():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from idempotent_llm_amd._lib import load
    from tiecases import EXPECTED, tie_cases
    load()
    print("[noalloc greedy pick]", flush=True)
    rng = np.random.default_rng(77)
    # call 1: 8 rows over the Qwen3 vocabulary (75 chunks each)
    V1 = 151936
    rows1 = torch.from_numpy(rng.integers(-(1 << 20), 1 << 20, (8, V1)).astype(np.int32)).cuda()
    hm1 = torch.from_numpy(rng.integers(1 << 14, 1 << 16, V1).astype(np.int64)).cuda()
    rows1[3, 151935] = 1 << 30                    # maximum in the last, partial chunk
    a = _pick_noalloc(rows1, hm1)
    b = _pick_with_scratch(rows1, hm1)
    assert a.tolist() == b.tolist()
    assert a[3].item() == 151935
    # call 2: fewer rows, a smaller vocabulary, real ties across chunks
    rows2, hm2 = tie_cases()
    rows2 = torch.from_numpy(rows2).cuda()
    hm2 = torch.from_numpy(hm2).cuda()
    a2 = _pick_noalloc(rows2, hm2)
    assert a2.tolist() == _pick_with_scratch(rows2, hm2).tolist() == EXPECTED
    # call 3: one row of the first shape again
    a3 = _pick_noalloc(rows1[5:6].contiguous(), hm1)
    assert a3.tolist() == b[5:6].tolist()


def test_noalloc_pick_rejects_sizes_beyond_its_scratch():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from idempotent_llm_amd._lib import load
    load()
    V = 2048 * 64
    R = 32768 // 64 + 1                           # one row more than the scratch holds
    rows = torch.zeros(R, V, dtype=torch.int32, device="cuda")
    hm = torch.ones(V, dtype=I64, device="cuda")
    with pytest.raises(RuntimeError, match="code -34"):
        _pick_noalloc(rows, hm)
    ok = _pick_noalloc(rows[: R - 1].contiguous(), hm)
    assert ok.tolist() == [0] * (R - 1)
