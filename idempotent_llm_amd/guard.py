"""Float-leak guard (the contract of the reference's guard.py:16-32).

A TorchDispatchMode that raises ``FloatLeakError`` the moment a floating-point
tensor is produced or consumed by any torch op inside the guarded region.
HIP kernels reached through the C-ABI do not dispatch through torch; their
arguments and outputs are integer tensors, which the guard sees wherever torch
allocates or views them.
"""

from __future__ import annotations

import torch
from torch.utils._python_dispatch import TorchDispatchMode
from torch.utils._pytree import tree_flatten


class FloatLeakError(RuntimeError):
    pass


def _floats(obj):
    flat, _ = tree_flatten(obj)
    return [t for t in flat if isinstance(t, torch.Tensor) and t.is_floating_point()]


class NoFloatMode(TorchDispatchMode):
    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if _floats((args, kwargs)):
            raise FloatLeakError(f"float tensor consumed by {func}")
        out = func(*args, **kwargs)
        if _floats(out):
            raise FloatLeakError(f"float tensor produced by {func}")
        return out
