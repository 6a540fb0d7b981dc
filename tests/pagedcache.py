"""Paged copies of contiguous test caches for the kernels' paged KV layout."""

import numpy as np
import torch

PAGE = 128


def paged(kc, vc, valid=None, seed=0):
    """Contiguous K [B, n_kv, cap, 128] and V^T [B, n_kv, 128, cap] (numpy or
    torch, int8) -> (k_pool, v_pool, table, width[, valid]) on the GPU. cap is
    padded to a multiple of 128 (the padding slots are invalid) and the page
    ids are a seeded permutation, so every access goes through the table."""
    from idempotent_llm_amd.kvcache import pages_from_contiguous
    kc = torch.as_tensor(np.ascontiguousarray(kc) if isinstance(kc, np.ndarray) else kc).cuda()
    vc = torch.as_tensor(np.ascontiguousarray(vc) if isinstance(vc, np.ndarray) else vc).cuda()
    B, n_kv, cap, hd = kc.shape
    capp = -(-cap // PAGE) * PAGE
    if capp != cap:
        kc = torch.cat([kc, torch.zeros(B, n_kv, capp - cap, hd, dtype=torch.int8,
                                        device="cuda")], dim=2)
        vc = torch.cat([vc, torch.zeros(B, n_kv, hd, capp - cap, dtype=torch.int8,
                                        device="cuda")], dim=3)
    kp, vp, table = pages_from_contiguous(kc, vc, seed=seed)
    out = (kp, vp, table, capp // PAGE)
    if valid is None:
        return out
    v = torch.as_tensor(np.ascontiguousarray(valid) if isinstance(valid, np.ndarray)
                        else valid).to(torch.bool).cuda()
    if capp != cap:
        v = torch.cat([v, torch.zeros(B, capp - cap, dtype=torch.bool, device="cuda")], dim=1)
    return out + (v.contiguous(),)


def unpaged(kp, vp, table, S):
    """Contiguous K [B, n_kv, S, 128] and V [B, n_kv, S, 128] of a paged cache."""
    B, w = table.shape
    ids = table.long()
    k = kp[ids].permute(0, 2, 1, 3, 4).reshape(B, kp.shape[1], w * PAGE, 128)[:, :, :S]
    v = vp[ids].permute(0, 2, 1, 4, 3).reshape(B, vp.shape[1], w * PAGE, 128)[:, :, :S]
    return k, v
