"""Demo chain hashes over int32 logits and token ids (scripts/demo.py:58-75).

h_0 = sha256(b"detllm-demo-v1"); h_i = sha256(h_{i-1} || bytes_i) where the
bytes are a logits row as little-endian int32, or a token id as 8 little-endian
bytes. Checkpoints report ``h.hex()[:16]``.
"""

from __future__ import annotations

import hashlib

import numpy as np

SEED = b"detllm-demo-v1"
CHECKPOINTS = (64, 128, 256, 512)


def _as_numpy(row):
    if hasattr(row, "detach"):
        row = row.detach().to("cpu").numpy()
    return np.ascontiguousarray(row, dtype="<i4")


class HashChain:
    """Incremental chain with checkpoint snapshots (scripts/demo.py:58-71)."""

    def __init__(self):
        self.h = hashlib.sha256(SEED).digest()
        self.steps: list[str] = []
        self.at: dict[int, str] = {}

    def update(self, data: bytes):
        self.h = hashlib.sha256(self.h + data).digest()
        self.steps.append(self.h.hex()[:16])
        if len(self.steps) in CHECKPOINTS:
            self.at[len(self.steps)] = self.steps[-1]

    def update_logits(self, row):
        self.update(_as_numpy(row).tobytes())

    def update_token(self, tok: int):
        self.update(int(tok).to_bytes(8, "little", signed=True))


def chain_hashes(rows) -> list[str]:
    c = HashChain()
    for r in rows:
        c.update_logits(r)
    return c.steps


def token_chain(toks) -> list[str]:
    c = HashChain()
    for t in toks:
        c.update_token(int(t))
    return c.steps
