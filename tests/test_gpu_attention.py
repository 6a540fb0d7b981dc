"""GPU checks of the decode attention paths through the C-ABI: the fused
Q/K/V-epilogue + attention kernel (detllm_qkv_attn_decode) against the two
separate launches it replaces (detllm_qkv_epilogue, detllm_attn_decode),
which the model goldens pin to the reference CPU path. Exact equality of the
attention output and of every cache byte, for random cache contents, ragged
validity masks, scanned-slot bounds given on the host or on the device, and
score rows that need the global scratch."""

import numpy as np
import pytest
import torch

from idempotent_llm_amd import artifact as art

pytestmark = pytest.mark.gpu
I64 = torch.int64


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from idempotent_llm_amd import _lib
    _lib.load()


def _layer_params(dims, seed):
    t, cfg = art.make_artifact_tensors(dims, seed)
    p, Lc = "layers.0.", cfg["layers"][0]
    d = lambda n: torch.from_numpy(np.ascontiguousarray(t[p + n])).cuda()
    g = dict(q_m=d("q.m"), q_k=Lc["q"]["k"], k_m=d("k.m"), k_k=Lc["k"]["k"], v_m=d("v.m"),
             v_k=Lc["v"]["k"], q_norm_m=d("q_norm.m"), q_norm_k=Lc["q_norm_k"],
             k_norm_m=d("k_norm.m"), k_norm_k=Lc["k_norm_k"],
             qs_m=d("qs_m").reshape(-1).contiguous(), qs_k=Lc["qs_k"],
             kq_m=d("kq_m").reshape(-1).contiguous(), kq_k=d("kq_k").reshape(-1).contiguous(),
             ks_m=d("ks_m"), ks_k=d("ks_k"), vq_m=d("vq_m"), vq_k=d("vq_k"),
             cos=torch.from_numpy(t["rope.cos"]).cuda(), sin=torch.from_numpy(t["rope.sin"]).cuda())
    return g


def _run(dims, B, cap, S, slot, device_bounds, seed):
    from idempotent_llm_amd._lib import call
    prm = _layer_params(dims, seed)
    nq, nkv, hd = dims["n_q_heads"], dims["n_kv_heads"], 128
    rnd = torch.Generator().manual_seed(seed)
    ns = 2
    P = torch.randint(-(1 << 19), 1 << 19, (ns, B, (nq + 2 * nkv) * hd), generator=rnd,
                      dtype=torch.int32).cuda()
    xm = torch.randint(1 << 15, 1 << 16, (B,), generator=rnd, dtype=I64).cuda()
    xk = torch.randint(22, 30, (B,), generator=rnd, dtype=I64).cuda()
    pos = torch.randint(0, dims["max_pos"], (B,), generator=rnd, dtype=I64).cuda()
    k0 = torch.randint(-128, 128, (B, nkv, cap, hd), generator=rnd, dtype=torch.int8).cuda()
    v0 = torch.randint(-128, 128, (B, nkv, hd, cap), generator=rnd, dtype=torch.int8).cuda()
    valid = (torch.rand(B, cap, generator=rnd) < 0.8).cuda()
    valid[:, slot] = True
    vbytes = valid.view(torch.uint8)
    G = nq // nkv
    Spad = (S + 15) // 16 * 16
    scratch = (torch.empty(B, nq, Spad, dtype=torch.int32, device="cuda")
               if G * Spad * 4 > 48 * 1024 else None)
    slot_dev = torch.tensor([slot], dtype=I64, device="cuda") if device_bounds else None
    s_dev = torch.tensor([S], dtype=I64, device="cuda") if device_bounds else None
    S_host = cap if device_bounds else S
    common = (prm["q_m"], prm["q_k"], prm["k_m"], prm["k_k"], prm["v_m"], prm["v_k"],
              prm["q_norm_m"], prm["q_norm_k"], prm["k_norm_m"], prm["k_norm_k"], prm["qs_m"],
              prm["qs_k"], prm["kq_m"], prm["kq_k"], prm["ks_m"], prm["ks_k"], prm["vq_m"],
              prm["vq_k"], prm["cos"], prm["sin"], prm["cos"].shape[0])
    # separate launches
    ka, va = k0.clone(), v0.clone()
    q8 = torch.empty(B, nq, 1, hd, dtype=torch.int8, device="cuda")
    tpos = torch.empty(B, nq, 1, dtype=I64, device="cuda")
    out_a = torch.empty(B, nq * hd, dtype=I64, device="cuda")
    call("detllm_qkv_epilogue", P, ns, B * P.shape[2], B, 1, nq, nkv, xm, xk, pos, *common,
         q8, tpos, None, ka, va, cap, slot_dev, slot)
    call("detllm_attn_decode", q8, tpos, ka, va, vbytes, cap, B, S_host, nq, nkv, cap, s_dev,
         scratch, out_a)
    # fused launch
    kb, vb = k0.clone(), v0.clone()
    out_b = torch.empty(B, nq * hd, dtype=I64, device="cuda")
    call("detllm_qkv_attn_decode", P, ns, B * P.shape[2], B, nq, nkv, xm, xk, pos, *common,
         kb, vb, cap, slot_dev, slot, vbytes, cap, S_host, s_dev, scratch, out_b)
    torch.cuda.synchronize()
    assert torch.equal(ka, kb)
    assert torch.equal(va, vb)
    assert torch.equal(out_a, out_b)
    assert not torch.equal(ka, k0)          # the step's K slot was written
    assert out_a.abs().sum().item() > 0


@pytest.mark.parametrize("S,device_bounds", [(1, False), (17, False), (300, True), (512, False)])
def test_fused_decode_equals_separate_launches(S, device_bounds):
    print(f"[fused decode S={S} device_bounds={device_bounds}]", flush=True)
    _run(art.MID, B=3, cap=512, S=S, slot=S - 1, device_bounds=device_bounds, seed=S)


def test_fused_decode_scratch_path():
    """Scores of a (row, kv-head) beyond the 48 KiB LDS budget (S = 6200,
    G = 2) go through the global scratch in both paths."""
    print("[fused decode scratch S=6200]", flush=True)
    _run(art.MID, B=2, cap=6400, S=6200, slot=6199, device_bounds=False, seed=5)


def test_fused_decode_group1():
    dims = dict(art.TINY, n_q_heads=2, n_kv_heads=2)
    print("[fused decode G=1]", flush=True)
    _run(dims, B=2, cap=256, S=100, slot=99, device_bounds=True, seed=9)
