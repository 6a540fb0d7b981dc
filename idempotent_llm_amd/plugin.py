"""Register the "rocm" backend with the reference package, so callers of its
unchanged API reach this runtime.

After ``install()`` (or ``install(detllm_module)``):

* ``detllm.backends.canonical_backend("rocm")`` (and the alias "hip") is
  accepted (backends.py:17-34: BACKENDS / BACKEND_ALIASES gain the name);
* ``detllm.backends.int_gemm(a, b, "rocm")`` — and through it
  ``int_gemm_u8i8`` / ``int_gemm_u16i8`` (backends.py:138-164), which look
  ``int_gemm`` up at call time — runs the detllm_rocm::int_gemm operator;
  every other backend name goes to the original function unchanged;
* ``detllm.model.IntQwen3(artifact_dir, "rocm")`` returns this package's
  ``IntQwen3`` (the fused-kernel runtime with the same forward / generate /
  greedy_pick API, model.py:105-531) instead of the per-op reference class;
  subclasses of the reference class (diagnostic seam overrides such as
  scripts/attribute_error.py) are left to the reference class, which then
  runs its own per-op path with the rocm GEMM;
* ``detllm.graphed.GraphedDecode(model, cache, lens, mode, layer_compile)``
  given a rocm model returns this package's ``GraphedDecode``.

``uninstall()`` restores the originals. Installing twice is a no-op.
"""

from __future__ import annotations

import importlib

_MARK = "_detllm_rocm_plugin"


def _plain_new(cls, *args, **kwargs):
    return object.__new__(cls)


def _modules(pkg):
    if pkg is None:
        pkg = importlib.import_module("detllm")
    name = pkg.__name__
    return (importlib.import_module(name + ".backends"), importlib.import_module(name + ".model"),
            importlib.import_module(name + ".graphed"))


def install(pkg=None) -> None:
    B, M, G = _modules(pkg)
    if getattr(B, _MARK, None) is not None:
        return
    from . import backends as rb
    from .graphed import GraphedDecode as RocmGraphed
    from .model import IntQwen3 as RocmIntQwen3

    saved = {"BACKENDS": B.BACKENDS, "BACKEND_ALIASES": dict(B.BACKEND_ALIASES),
             "int_gemm": B.int_gemm, "model_int_gemm": getattr(M, "int_gemm", None),
             "model_new": M.IntQwen3.__dict__.get("__new__"),
             "graphed_new": G.GraphedDecode.__dict__.get("__new__")}
    if "rocm" not in B.BACKENDS:
        B.BACKENDS = tuple(B.BACKENDS) + ("rocm",)
    B.BACKEND_ALIASES.setdefault("hip", "rocm")
    orig_gemm = saved["int_gemm"]

    def int_gemm(a, b, backend):
        if backend == "rocm":
            return rb.int_gemm(a, b, "rocm")
        return orig_gemm(a, b, backend)

    int_gemm.__doc__ = orig_gemm.__doc__
    B.int_gemm = int_gemm
    if saved["model_int_gemm"] is not None:
        M.int_gemm = int_gemm
    ref_cls = M.IntQwen3

    def model_new(cls, artifact_dir=None, backend="reference", *args, **kwargs):
        if cls is ref_cls and B.canonical_backend(backend) == "rocm":
            return RocmIntQwen3(artifact_dir, "rocm")
        return object.__new__(cls)

    M.IntQwen3.__new__ = staticmethod(model_new)
    ref_graphed = G.GraphedDecode

    def graphed_new(cls, model=None, *args, **kwargs):
        if cls is ref_graphed and isinstance(model, RocmIntQwen3):
            return RocmGraphed(model, *args, **kwargs)
        return object.__new__(cls)

    G.GraphedDecode.__new__ = staticmethod(graphed_new)
    setattr(B, _MARK, saved)


def uninstall(pkg=None) -> None:
    B, M, G = _modules(pkg)
    saved = getattr(B, _MARK, None)
    if saved is None:
        return
    B.BACKENDS = saved["BACKENDS"]
    B.BACKEND_ALIASES.clear()
    B.BACKEND_ALIASES.update(saved["BACKEND_ALIASES"])
    B.int_gemm = saved["int_gemm"]
    if saved["model_int_gemm"] is not None:
        M.int_gemm = saved["model_int_gemm"]
    for cls, key in ((M.IntQwen3, "model_new"), (G.GraphedDecode, "graphed_new")):
        # deleting an assigned __new__ leaves CPython calling object.__new__
        # with the constructor's arguments; a pass-through restores behaviour
        cls.__new__ = saved[key] if saved[key] is not None else staticmethod(_plain_new)
    delattr(B, _MARK)
