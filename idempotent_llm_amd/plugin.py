"""Register the "rocm" backend with the reference package, so callers of its
unchanged API reach this runtime.

After ``install()`` (or ``install(detllm_module)``):

* ``detllm.backends.canonical_backend("rocm")`` (and the alias "hip") is
  accepted (backends.py:17-34: BACKENDS / BACKEND_ALIASES gain the name);
* ``detllm.backends.int_gemm(a, b, "rocm")`` runs the detllm_rocm::int_gemm
  operator; every other backend name goes to the original function
  unchanged. The package's modules that imported ``int_gemm`` by name
  (model.py:29, ops/di_matmul.py:18) are rebound to the same dispatcher,
  and ``int_gemm_u8i8`` / ``int_gemm_u16i8`` (backends.py:138-164) look the
  name up at call time;
* ``detllm.ops.di_linear`` / ``di_matmul(..., "rocm")`` (ops/di_matmul.py:
  22-40) run this package's quantiser, GEMM and requantiser kernels;
* the reference's device primitives ``detllm::isqrt_i64`` /
  ``detllm::ilog2_i64`` (ops/int_prims.py:96-136, Triton kernels registered
  for "cuda") get this package's HIP kernels as their "cuda" kernels, the
  registration point the reference itself uses; reference code that runs on
  the device (a seam override calling ``dyadic.norm_scale``, say) therefore
  launches no Triton kernel;
* ``detllm.model.IntQwen3(artifact_dir, "rocm")`` builds this package's
  runtime (the fused kernels and the whole-step HIP graph behind the same
  forward / generate / greedy_pick API, model.py:105-531), as an instance of
  a class deriving from both this package's ``IntQwen3`` and the reference
  class, so ``isinstance(m, detllm.model.IntQwen3)`` holds. A subclass of the
  reference class built with "rocm" (diagnostic seam overrides of
  ``_attn_scores`` / ``_attn_context`` / ``_lm_head``, model.py:430-432,
  :469-478, as in scripts/attribute_error.py) gets the same runtime with its
  overrides in front: its methods come first in the method order, then this
  package's, then the reference class's, so ``super()`` in an override
  reaches this package's seam. Reference methods this runtime has no
  counterpart for raise NotImplementedError instead of running the
  reference's per-op path;
* ``detllm.graphed.GraphedDecode(model, cache, lens, mode, layer_compile)``
  given a rocm model returns this package's ``GraphedDecode``.

``uninstall()`` restores the originals. Installing twice is a no-op.
"""

from __future__ import annotations

import importlib
import sys

_MARK = "_detllm_rocm_plugin"
_ROCM_CLS = "_detllm_rocm_class"


def _plain_new(cls, *args, **kwargs):
    return object.__new__(cls)


def _modules(pkg):
    if pkg is None:
        pkg = importlib.import_module("detllm")
    name = pkg.__name__
    return (importlib.import_module(name + ".backends"), importlib.import_module(name + ".model"),
            importlib.import_module(name + ".graphed"))


def _optional(name):
    try:
        return importlib.import_module(name)
    except ImportError:
        return None


def _package_modules(name):
    return [m for k, m in list(sys.modules.items())
            if m is not None and (k == name or k.startswith(name + "."))]


def _unsupported(name):
    def method(self, *args, **kwargs):
        raise NotImplementedError(
            f"{name} is part of the reference's per-op path; the rocm backend runs fused "
            "HIP kernels behind forward / generate / greedy_pick and the seams "
            "_attn_scores / _attn_context / _lm_head")
    method.__name__ = name
    return method


def _rocm_base(ref_cls, rocm_cls):
    """The class of a plain IntQwen3(dir, "rocm"): this package's runtime
    first, the reference class after it (for isinstance)."""
    ns = {"__module__": rocm_cls.__module__, "__doc__": rocm_cls.__doc__, _ROCM_CLS: True}
    for name, val in vars(ref_cls).items():
        if name.startswith("__") or hasattr(rocm_cls, name):
            continue
        if callable(val) or isinstance(val, (staticmethod, classmethod, property)):
            ns[name] = _unsupported(name)
    return type(ref_cls.__name__, (rocm_cls, ref_cls), ns)


def install(pkg=None) -> None:
    B, M, G = _modules(pkg)
    if getattr(B, _MARK, None) is not None:
        return
    pkg_name = B.__name__.rsplit(".", 1)[0]
    D = _optional(pkg_name + ".ops.di_matmul")
    PR = _optional(pkg_name + ".ops.int_prims")
    from . import backends as rb
    from . import ops as rops
    from . import torch_ops  # noqa: F401  (registers detllm_rocm::*)
    from .graphed import GraphedDecode as RocmGraphed
    from .model import IntQwen3 as RocmIntQwen3

    saved = {"BACKENDS": B.BACKENDS, "BACKEND_ALIASES": dict(B.BACKEND_ALIASES),
             "int_gemm": B.int_gemm, "rebound": [], "prims": [],
             "model_new": M.IntQwen3.__dict__.get("__new__"),
             "graphed_new": G.GraphedDecode.__dict__.get("__new__")}
    if "rocm" not in B.BACKENDS:
        B.BACKENDS = tuple(B.BACKENDS) + ("rocm",)
    B.BACKEND_ALIASES.setdefault("hip", "rocm")

    def rebind(mod, attr, new):
        saved["rebound"].append((mod, attr, getattr(mod, attr)))
        setattr(mod, attr, new)

    # int_gemm: the backends module and every module that imported the name
    orig_gemm = saved["int_gemm"]

    def int_gemm(a, b, backend):
        if backend == "rocm":
            return rb.int_gemm(a, b, "rocm")
        return orig_gemm(a, b, backend)

    int_gemm.__doc__ = orig_gemm.__doc__
    for mod in _package_modules(pkg_name):
        if getattr(mod, "int_gemm", None) is orig_gemm:
            rebind(mod, "int_gemm", int_gemm)

    # di_linear / di_matmul (ops/di_matmul.py:22-40): the whole composition
    # on this package's kernels for "rocm"
    if D is not None:
        orig_lin, orig_mm = D.di_linear, D.di_matmul

        def di_linear(x8, xm, xk, w8_t, wm, wk, backend):
            if backend == "rocm":
                return rops.di_linear(x8, xm, xk, w8_t, wm, wk, backend)
            return orig_lin(x8, xm, xk, w8_t, wm, wk, backend)

        def di_matmul(x, xm, xk, w8_t, wm, wk, backend):
            if backend == "rocm":
                return rops.di_matmul(x, xm, xk, w8_t, wm, wk, backend)
            return orig_mm(x, xm, xk, w8_t, wm, wk, backend)

        di_linear.__doc__, di_matmul.__doc__ = orig_lin.__doc__, orig_mm.__doc__
        for mod in _package_modules(pkg_name):
            for attr, orig, new in (("di_linear", orig_lin, di_linear),
                                    ("di_matmul", orig_mm, di_matmul)):
                if getattr(mod, attr, None) is orig:
                    rebind(mod, attr, new)

    # the reference's device primitives: this package's HIP kernels behind
    # their "cuda" registration (ops/int_prims.py:116-136)
    if PR is not None:
        import torch
        for name in ("isqrt_i64", "ilog2_i64"):
            opdef = getattr(PR, name, None)
            if opdef is None or not hasattr(opdef, "register_kernel"):
                continue
            prev = getattr(opdef, "_backend_fns", {}).get("cuda")
            loop = getattr(PR, "_" + name.split("_")[0] + "_loop", None)
            saved["prims"].append((opdef, prev if prev is not None else loop))
            rocm_op = getattr(torch.ops.detllm_rocm, name)

            def kernel(a, _op=rocm_op):
                return _op(a.to(torch.int64).contiguous())

            opdef.register_kernel("cuda")(kernel)

    # IntQwen3(dir, "rocm") and subclasses of it
    ref_cls = M.IntQwen3
    saved["base"] = _rocm_base(ref_cls, RocmIntQwen3)
    saved["combined"] = {ref_cls: saved["base"]}

    def model_new(cls, artifact_dir=None, backend="reference", *args, **kwargs):
        try:
            rocm = B.canonical_backend(backend) == "rocm"
        except (ValueError, TypeError):
            rocm = False    # the constructor raises as the reference does
        return object.__new__(_runtime_class(saved, cls) if rocm else cls)

    M.IntQwen3.__new__ = staticmethod(model_new)
    ref_graphed = G.GraphedDecode

    def graphed_new(cls, model=None, *args, **kwargs):
        if cls is ref_graphed and isinstance(model, RocmIntQwen3):
            return RocmGraphed(model, *args, **kwargs)
        return object.__new__(cls)

    G.GraphedDecode.__new__ = staticmethod(graphed_new)
    setattr(B, _MARK, saved)


def _runtime_class(saved, cls):
    if cls.__dict__.get(_ROCM_CLS):
        return cls
    combined = saved["combined"]
    got = combined.get(cls)
    if got is None:
        # cls's own methods first, then this package's runtime, then the
        # reference class (C3 order of (cls, base): cls, its bases below the
        # reference class, base, RocmIntQwen3, reference class)
        got = type(cls.__name__, (cls, saved["base"]),
                   {"__module__": cls.__module__, "__qualname__": cls.__qualname__,
                    "__doc__": cls.__doc__, _ROCM_CLS: True})
        combined[cls] = got
    return got


def runtime_class(cls, pkg=None) -> type:
    """The class an ``IntQwen3`` (or subclass) built with backend "rocm" is
    an instance of while the plugin is installed on ``pkg``."""
    B, M, _ = _modules(pkg)
    saved = getattr(B, _MARK, None)
    if saved is None:
        raise RuntimeError("the rocm plugin is not installed on this package")
    if not issubclass(cls, M.IntQwen3):
        raise TypeError(f"{cls!r} does not derive from {M.__name__}.IntQwen3")
    return _runtime_class(saved, cls)


def uninstall(pkg=None) -> None:
    B, M, G = _modules(pkg)
    saved = getattr(B, _MARK, None)
    if saved is None:
        return
    B.BACKENDS = saved["BACKENDS"]
    B.BACKEND_ALIASES.clear()
    B.BACKEND_ALIASES.update(saved["BACKEND_ALIASES"])
    for mod, attr, orig in reversed(saved["rebound"]):
        setattr(mod, attr, orig)
    for opdef, fn in saved["prims"]:
        if fn is not None:
            opdef.register_kernel("cuda")(fn)
    for cls, key in ((M.IntQwen3, "model_new"), (G.GraphedDecode, "graphed_new")):
        # deleting an assigned __new__ leaves CPython calling object.__new__
        # with the constructor's arguments; a pass-through restores behaviour
        cls.__new__ = saved[key] if saved[key] is not None else staticmethod(_plain_new)
    delattr(B, _MARK)
