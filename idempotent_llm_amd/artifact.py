"""Seeded synthetic inputs and random-init integer artifacts.

The reference's real artifact (``prepare.py``, a float calibration of the
Qwen3 checkpoint) needs the HF Hub, so every workload here is synthetic:

* ``splitmix64`` (Steele, Lea & Flood, OOPSLA 2014) is the only source of
  randomness; every tensor draws from its own stream, keyed by a master seed
  and the tensor's name, so a workload is reproducible on any machine.
* Gaussian-shaped integers use Irwin-Hall: the sum of 12 uniform 32-bit
  integers, centred and scaled by an integer sigma with one rounding shift —
  no libm or float on the data path.
* ``make_artifact`` writes ``model.safetensors`` + ``config.json`` in the
  schema that ``prepare.py:296-433`` writes and ``model.py:106-183`` reads.
  Scale mantissas are drawn from ranges that keep every int64 intermediate of
  the forward pass below 2^62 (QK-smoothing, QK-norm gamma and activation
  smoothing are kept small; see ``_MODEL_SCALES``).

The RoPE tables are the one float computation (offline, as in
``ops/rope.py:25-35``): float64 cos/sin rounded to int16 at 2^14.
"""

from __future__ import annotations

import json
import os
import zlib

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def splitmix64(seed: int, n: int) -> np.ndarray:
    """The first n outputs of splitmix64 started at ``seed`` (uint64)."""
    out = np.empty(n, dtype=np.uint64)
    s = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
    with np.errstate(over="ignore"):
        for c0 in range(0, n, _CHUNK):
            c1 = min(n, c0 + _CHUNK)
            z = s + (np.arange(c0 + 1, c1 + 1, dtype=np.uint64) * _GOLDEN)
            z = (z ^ (z >> np.uint64(30))) * _M1
            z = (z ^ (z >> np.uint64(27))) * _M2
            out[c0:c1] = z ^ (z >> np.uint64(31))
    return out


def stream_seed(seed: int, name: str) -> int:
    """Independent stream per (master seed, tensor name)."""
    key = (int(seed) * 0x100000001B3 + zlib.crc32(name.encode())) & 0xFFFFFFFFFFFFFFFF
    return int(splitmix64(key, 1)[0])


def rand_i8(seed: int, name: str, shape) -> np.ndarray:
    """~Uniform int8 in [-127, 127] (the byte -128 is folded onto -127)."""
    n = int(np.prod(shape))
    raw = splitmix64(stream_seed(seed, name), (n + 7) // 8).view(np.int8)[:n].copy()
    raw[raw == -128] = -127
    return raw.reshape(shape)


def uniform_int(seed: int, name: str, shape, lo: int, hi: int) -> np.ndarray:
    """~Uniform int64 in [lo, hi)."""
    n = int(np.prod(shape))
    u = splitmix64(stream_seed(seed, name), n)
    span = np.uint64(hi - lo)
    return (np.int64(lo) + (u % span).astype(np.int64)).reshape(shape)


def gauss_int(seed: int, name: str, shape, sigma: int) -> np.ndarray:
    """~round(N(0, sigma)) as int64 via integer Irwin-Hall (12 uniforms)."""
    n = int(np.prod(shape))
    u = splitmix64(stream_seed(seed, name), 6 * n).reshape(n, 6)
    lo = (u & np.uint64(0xFFFFFFFF)).astype(np.int64)
    hi = (u >> np.uint64(32)).astype(np.int64)
    s = lo.sum(axis=1) + hi.sum(axis=1) - (np.int64(6) << np.int64(32))
    v = (s * np.int64(sigma) + (np.int64(1) << np.int64(31))) >> np.int64(32)
    return v.reshape(shape)


def rope_tables(head_dim: int, max_pos: int, base: float):
    """Offline int16 cos/sin tables at 2^14, HF tiling (ops/rope.py:25-35)."""
    j = np.arange(0, head_dim // 2, dtype=np.float64)
    inv_freq = base ** (-2.0 * j / head_dim)
    ang = np.outer(np.arange(max_pos, dtype=np.float64), inv_freq)
    ang = np.concatenate([ang, ang], axis=-1)
    cos_t = np.round(np.cos(ang) * 16384.0).astype(np.int16)
    sin_t = np.round(np.sin(ang) * 16384.0).astype(np.int16)
    return cos_t, sin_t


# Dimensions: the Qwen3-0.6B shape and two small shapes used by parity tests.
QWEN3_0_6B = dict(n_layers=28, hidden=1024, n_q_heads=16, n_kv_heads=8, head_dim=128,
                  intermediate=3072, vocab=151936, max_pos=40960, rope_theta=1e6,
                  eos_token_id=151645)
MID = dict(n_layers=2, hidden=1024, n_q_heads=16, n_kv_heads=8, head_dim=128,
           intermediate=3072, vocab=4096, max_pos=2048, rope_theta=1e6, eos_token_id=4095)
TINY = dict(n_layers=2, hidden=256, n_q_heads=4, n_kv_heads=2, head_dim=128,
            intermediate=512, vocab=1000, max_pos=1024, rope_theta=1e6, eos_token_id=999)

# (lo, hi) mantissa ranges and shifts for the per-tensor scales. The
# products that could overflow int64 on the Q path are bounded by
# 2^23.5 (RMSNorm) * 2^12 (gamma) * 2^10 (QK smoothing) * 2^15 (norm_scale)
# * 2^0.5 (RoPE) < 2^62; MLP down input: 2^35 (swiglu) * 2^10 * 2^16 < 2^62.
_MODEL_SCALES = dict(
    w_m=(1 << 14, 1 << 16), w_k=24,
    embed_m=(1 << 15, 1 << 16), embed_k=(22, 27),
    gamma_m=(1 << 10, 1 << 12), gamma_k=11,
    qs_m=(1 << 8, 1 << 10), qs_k=9,
    smooth_m=(1 << 9, 1 << 11), smooth_k=10,
    ds_m=(1 << 8, 1 << 10), ds_k=9,
    kq_m=(1 << 15, 1 << 16), kq_k=(18, 21),
    ks_m=(1 << 15, 1 << 16), ks_k=(24, 27),
    vq_m=(1 << 15, 1 << 16), vq_k=(16, 20),
)


def make_artifact_tensors(dims: dict, seed: int):
    """Build the artifact's tensors and config (reference schema)."""
    sc = _MODEL_SCALES
    L_, H, nq, nkv, hd = (dims["n_layers"], dims["hidden"], dims["n_q_heads"],
                          dims["n_kv_heads"], dims["head_dim"])
    inter, V, max_pos = dims["intermediate"], dims["vocab"], dims["max_pos"]
    t: dict = {}
    cfg = {
        "model_id": f"random-init-seed{seed}",
        "n_layers": L_, "hidden": H, "n_q_heads": nq, "n_kv_heads": nkv,
        "head_dim": hd, "intermediate": inter, "vocab": V, "max_pos": max_pos,
        "rope_frac_bits": 14, "eos_token_id": dims["eos_token_id"],
        "layers": [],
    }
    t["embed.e8"] = rand_i8(seed, "embed.e8", (V, H))
    t["embed.m"] = uniform_int(seed, "embed.m", (V,), *sc["embed_m"])
    t["embed.k"] = uniform_int(seed, "embed.k", (V,), *sc["embed_k"])
    t["head.w8t"] = rand_i8(seed, "head.w8t", (H, V))
    t["head.m"] = uniform_int(seed, "head.m", (V,), *sc["w_m"])
    cfg["head"] = {"k": sc["w_k"], "min_m": int(t["head.m"].min())}
    cos_t, sin_t = rope_tables(hd, max_pos, dims["rope_theta"])
    t["rope.cos"] = cos_t
    t["rope.sin"] = sin_t
    shapes = {"q": (H, nq * hd), "k": (H, nkv * hd), "v": (H, nkv * hd),
              "o": (nq * hd, H), "gate": (H, inter), "up": (H, inter),
              "down": (inter, H)}
    for i in range(L_):
        p = f"layers.{i}."
        Lc: dict = {}
        for nm, shp in shapes.items():
            t[p + nm + ".w8t"] = rand_i8(seed, p + nm + ".w8t", shp)
            m = uniform_int(seed, p + nm + ".m", (shp[1],), *sc["w_m"])
            t[p + nm + ".m"] = m
            Lc[nm] = {"k": sc["w_k"], "min_m": int(m.min())}
        t[p + "q_norm.m"] = uniform_int(seed, p + "q_norm.m", (hd,), *sc["gamma_m"])
        t[p + "k_norm.m"] = uniform_int(seed, p + "k_norm.m", (hd,), *sc["gamma_m"])
        Lc["q_norm_k"] = sc["gamma_k"]
        Lc["k_norm_k"] = sc["gamma_k"]
        t[p + "qs_m"] = uniform_int(seed, p + "qs_m", (nkv, hd), *sc["qs_m"])
        Lc["qs_k"] = sc["qs_k"]
        for nm, n in (("as", H), ("ms", H), ("os", nq * hd)):
            t[p + nm + "_m"] = uniform_int(seed, p + nm + "_m", (n,), *sc["smooth_m"])
            Lc[nm + "_k"] = sc["smooth_k"]
        t[p + "ds_m"] = uniform_int(seed, p + "ds_m", (inter,), *sc["ds_m"])
        Lc["ds_k"] = sc["ds_k"]
        t[p + "kq_m"] = uniform_int(seed, p + "kq_m", (nkv, hd), *sc["kq_m"])
        t[p + "kq_k"] = uniform_int(seed, p + "kq_k", (nkv, hd), *sc["kq_k"])
        t[p + "ks_m"] = uniform_int(seed, p + "ks_m", (nkv,), *sc["ks_m"])
        t[p + "ks_k"] = uniform_int(seed, p + "ks_k", (nkv,), *sc["ks_k"])
        t[p + "vq_m"] = uniform_int(seed, p + "vq_m", (nkv,), *sc["vq_m"])
        t[p + "vq_k"] = uniform_int(seed, p + "vq_k", (nkv,), *sc["vq_k"])
        cfg["layers"].append(Lc)
    return t, cfg


def make_artifact(out_dir: str, dims: dict = QWEN3_0_6B, seed: int = 3) -> str:
    """Write a random-init artifact directory; returns its path."""
    from safetensors.numpy import save_file
    os.makedirs(out_dir, exist_ok=True)
    t, cfg = make_artifact_tensors(dims, seed)
    save_file({k: np.ascontiguousarray(v) for k, v in t.items()},
              os.path.join(out_dir, "model.safetensors"))
    with open(os.path.join(out_dir, "config.json"), "w") as f:
        json.dump(cfg, f, indent=1)
    return out_dir


def artifact_digest(out_dir: str) -> str:
    """sha256 of model.safetensors + config.json (provable comparability)."""
    import hashlib
    h = hashlib.sha256()
    for fn in ("model.safetensors", "config.json"):
        with open(os.path.join(out_dir, fn), "rb") as f:
            for blk in iter(lambda: f.read(1 << 24), b""):
                h.update(blk)
    return h.hexdigest()


# ---------------------------------------------------------------------------
# Prompts (scripts/demo.py:90-94 shapes: ids in [100, 50000))
# ---------------------------------------------------------------------------

def prompt_ids(seed: int, n: int, vocab: int, lo: int = 100, hi: int = 50000) -> np.ndarray:
    hi = min(hi, vocab)
    lo = min(lo, hi - 1)
    return uniform_int(seed, "prompt", (n,), lo, hi)


def co_prompts(seed: int, count: int, vocab: int, len_lo: int = 5, len_hi: int = 40):
    """Seeded random co-prompts of random lengths (scripts/demo.py:90-94)."""
    lens = uniform_int(seed, "co_prompt_lens", (count,), len_lo, len_hi)
    out = []
    hi = min(50000, vocab)
    for i, n in enumerate(lens):
        out.append(uniform_int(seed, f"co_prompt.{i}", (int(n),), min(100, hi - 1), hi))
    return out


def right_pad(seqs):
    """Right-padded ids [B, T] and valid mask [B, T] (model.py:8-17)."""
    T = max(len(s) for s in seqs)
    ids = np.zeros((len(seqs), T), dtype=np.int64)
    valid = np.zeros((len(seqs), T), dtype=bool)
    for i, s in enumerate(seqs):
        ids[i, :len(s)] = s
        valid[i, :len(s)] = True
    return ids, valid
