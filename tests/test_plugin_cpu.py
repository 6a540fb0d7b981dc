"""The drop-in registration (idempotent_llm_amd.plugin) and the custom
operators' fake implementations, on the CPU.

The reference package is not imported here (its code is read, not run); a
stand-in package with the same module layout and public names takes its
place, holding only what the plugin touches:

* backends: BACKENDS, BACKEND_ALIASES, canonical_backend, int_gemm,
  int_gemm_u8i8 (backends.py:17-164);
* ops.int_prims: the device primitives isqrt_i64 / ilog2_i64 as custom ops
  whose "cuda" kernel stands for the reference's Triton kernels and counts
  its launches (ops/int_prims.py:96-136);
* ops.di_matmul: di_linear / di_matmul binding int_gemm by name at import
  (ops/di_matmul.py:18-40), re-exported by ops/__init__;
* model: IntQwen3 importing int_gemm by name (model.py:29), with seams that
  run reference code on the device (an int_gemm and a primitive) and a
  per-op method this runtime has no counterpart for;
* graphed: GraphedDecode."""

import math
import sys
import types

import pytest
import torch

_PRIMS = {}     # custom ops are defined once per process and name


def _prims(name):
    if name not in _PRIMS:
        ns = types.SimpleNamespace(TRITON_CALLS=0)

        def isqrt_loop(a: torch.Tensor) -> torch.Tensor:
            return torch.tensor([math.isqrt(v) for v in a.reshape(-1).tolist()],
                                dtype=torch.int64, device=a.device).view(a.shape)

        def ilog2_loop(a: torch.Tensor) -> torch.Tensor:
            return torch.tensor([v.bit_length() - 1 for v in a.reshape(-1).tolist()],
                                dtype=torch.int64, device=a.device).view(a.shape)

        for op, loop in (("isqrt_i64", isqrt_loop), ("ilog2_i64", ilog2_loop)):
            d = torch.library.custom_op(f"{name}::{op}", loop, mutates_args=())
            d.register_fake(lambda a: torch.empty_like(a, dtype=torch.int64))

            def triton_standin(a: torch.Tensor, _loop=loop) -> torch.Tensor:
                ns.TRITON_CALLS += 1
                return _loop(a)

            d.register_kernel("cuda")(triton_standin)
            setattr(ns, op, d)
            setattr(ns, "_" + op.split("_")[0] + "_loop", loop)
        _PRIMS[name] = ns
    return _PRIMS[name]


def _module(name, src, **glob):
    m = types.ModuleType(name)
    m.__dict__.update(glob)
    exec(src, m.__dict__)
    sys.modules[name] = m
    return m


def _standin(name="detllm_standin"):
    pkg = types.ModuleType(name)
    pkg.__path__ = []
    sys.modules[name] = pkg
    B = _module(name + ".backends", """
import torch
BACKENDS = ("reference", "cuda")
BACKEND_ALIASES = {"cpu": "reference"}
def canonical_backend(name):
    canon = BACKEND_ALIASES.get(name, name)
    if canon not in BACKENDS:
        raise ValueError(f"unknown backend {name!r}")
    return canon
def int_gemm(a, b, backend):
    if backend == "reference":
        return torch.matmul(a.to(torch.int32), b.to(torch.int32))
    raise ValueError(f"unknown backend {backend!r}")
def int_gemm_u8i8(p, b, backend):
    core = int_gemm((p - 64).to(torch.int8), b, backend)
    return core + b.to(torch.int32).sum(dim=-2, keepdim=True) * 64
""")
    ops = types.ModuleType(name + ".ops")
    ops.__path__ = []
    sys.modules[name + ".ops"] = ops
    pr = _prims(name)
    PR = _module(name + ".ops.int_prims", "", isqrt_i64=pr.isqrt_i64, ilog2_i64=pr.ilog2_i64,
                 _isqrt_loop=pr._isqrt_loop, _ilog2_loop=pr._ilog2_loop, STATE=pr)
    D = _module(name + ".ops.di_matmul", """
import torch
int_gemm = _B.int_gemm
def di_linear(x8, xm, xk, w8_t, wm, wk, backend):
    return int_gemm(x8, w8_t, backend), xm, xk, wm, wk
def di_matmul(x, xm, xk, w8_t, wm, wk, backend):
    # the reference's dyadic quantiser runs the device primitives
    _PR.ilog2_i64(x.abs().amax(dim=-1).clamp(min=1))
    x8 = x.clamp(-127, 127).to(torch.int8)
    return ("reference per-op path",) + di_linear(x8, xm, xk, w8_t, wm, wk, backend)
""", _B=B, _PR=PR)
    ops.di_linear, ops.di_matmul, ops.int_prims = D.di_linear, D.di_matmul, PR
    M = _module(name + ".model", """
import torch
int_gemm = _B.int_gemm
class IntQwen3:
    def __init__(self, artifact_dir, backend="reference"):
        self.backend = _B.canonical_backend(backend)
        self.artifact_dir = artifact_dir
    def _per_op_attention(self, q8):
        return _PR.ilog2_i64(q8.to(torch.int64).abs().clamp(min=1))
    def _lm_head(self, x8, xm, xk):
        return int_gemm(x8, self.head_w8t, self.backend)
    def _attn_scores(self, q8, qm, qk, K8r, L, group, aux=None):
        _PR.ilog2_i64(qm.clamp(min=1))
        raise AssertionError("the reference's default seam ran")
""", _B=B, _PR=PR)
    G = _module(name + ".graphed", """
class GraphedDecode:
    def __init__(self, model, cache, lens, mode="capture", layer_compile=True):
        self.model = model
""")
    pkg.backends, pkg.ops, pkg.model, pkg.graphed = B, ops, M, G
    return pkg


@pytest.fixture
def standin():
    pkg = _standin()
    yield pkg
    for k in [k for k in sys.modules if k.startswith("detllm_standin")]:
        del sys.modules[k]


def test_install_routes_rocm_and_leaves_the_rest(standin):
    from idempotent_llm_amd import plugin
    from idempotent_llm_amd.model import IntQwen3 as RocmIntQwen3
    B, M = standin.backends, standin.model
    D = sys.modules["detllm_standin.ops.di_matmul"]
    with pytest.raises(ValueError):
        B.canonical_backend("rocm")
    orig_gemm, orig_mm = B.int_gemm, D.di_matmul
    plugin.install(standin)
    plugin.install(standin)                       # idempotent
    assert B.canonical_backend("rocm") == "rocm" and B.canonical_backend("hip") == "rocm"
    assert B.canonical_backend("cpu") == "reference"
    a = torch.tensor([[1, -2], [3, 4]], dtype=torch.int8)
    b = torch.tensor([[5, 6], [-7, 8]], dtype=torch.int8)
    assert torch.equal(B.int_gemm(a, b, "reference"), a.int() @ b.int())
    # every module that imported int_gemm by name reaches the dispatcher
    assert M.int_gemm is B.int_gemm and D.int_gemm is B.int_gemm and B.int_gemm is not orig_gemm
    # di_linear / di_matmul: rebound in the module and the package namespace
    assert standin.ops.di_matmul is D.di_matmul and D.di_matmul is not orig_mm
    x = torch.tensor([[3, -200], [5, 7]], dtype=torch.int32)
    one = torch.ones(2, 1, dtype=torch.int64)
    ref = standin.ops.di_matmul(x, one, one * 0, b, one[:, 0], 20, "reference")
    assert ref[0] == "reference per-op path"
    ref = M.IntQwen3("dir", "reference")
    assert type(ref) is M.IntQwen3 and ref.backend == "reference"
    # "rocm" reaches this package's runtime (which needs a GPU: on the CPU it
    # refuses instead of falling back)
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="gfx950"):
            M.IntQwen3("dir", "rocm")
        with pytest.raises(Exception):             # no CPU kernel behind the rocm GEMM
            B.int_gemm(a, b, "rocm")
        with pytest.raises(Exception):
            standin.ops.di_matmul(x, one, one * 0, b, one[:, 0], 20, "rocm")

    class Sub(M.IntQwen3):                          # a diagnostic seam override
        def _lm_head(self, x8, xm, xk):
            return "override"
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="gfx950"):   # this runtime's constructor
            Sub("dir", "rocm")
    assert type(Sub("dir", "cpu")) is Sub                   # other backends: untouched
    plugin.uninstall(standin)
    with pytest.raises(ValueError):
        B.canonical_backend("rocm")
    assert B.int_gemm is orig_gemm and M.int_gemm is orig_gemm and D.int_gemm is orig_gemm
    assert D.di_matmul is orig_mm and standin.ops.di_matmul is orig_mm
    assert type(M.IntQwen3("dir", "cpu")) is M.IntQwen3
    assert RocmIntQwen3 is not M.IntQwen3


def test_subclass_runtime_class_order(standin):
    """A reference subclass built with "rocm" is an instance of a class whose
    method order is: the subclass's overrides, this package's runtime, the
    reference class; super() in an override reaches this package's seam, and
    reference methods without a counterpart here refuse instead of running
    the reference's per-op path."""
    from idempotent_llm_amd import plugin
    from idempotent_llm_amd.model import IntQwen3 as RocmIntQwen3
    M = standin.model

    class Mid(M.IntQwen3):
        def _attn_context(self, probs, V8r, L, aux=None):
            return "mid"

    class Leaf(Mid):
        def _lm_head(self, x8, xm, xk):
            return ("leaf", super()._lm_head)

    with pytest.raises(RuntimeError):
        plugin.runtime_class(Leaf, standin)         # not installed
    plugin.install(standin)
    try:
        base = plugin.runtime_class(M.IntQwen3, standin)
        cls = plugin.runtime_class(Leaf, standin)
        assert plugin.runtime_class(Leaf, standin) is cls and plugin.runtime_class(cls, standin) is cls
        mro = cls.__mro__
        assert mro[:4] == (cls, Leaf, Mid, base)
        assert mro.index(RocmIntQwen3) < mro.index(M.IntQwen3)
        assert issubclass(cls, Leaf) and issubclass(cls, RocmIntQwen3) and issubclass(cls, M.IntQwen3)
        # method resolution without running a constructor
        obj = object.__new__(cls)
        tag, sup = obj._lm_head(None, None, None)
        assert tag == "leaf" and sup.__func__ is RocmIntQwen3._lm_head
        assert obj._attn_context(None, None, None) == "mid"
        assert cls._attn_scores is RocmIntQwen3._attn_scores     # not the reference default
        assert cls._norm_quant is RocmIntQwen3._norm_quant
        with pytest.raises(NotImplementedError, match="per-op path"):
            obj._per_op_attention(torch.zeros(2, dtype=torch.int8))
        assert standin.ops.int_prims.STATE.TRITON_CALLS == 0
        with pytest.raises(TypeError):
            plugin.runtime_class(int, standin)
    finally:
        plugin.uninstall(standin)


def test_custom_ops_trace_with_integer_fakes():
    """Every detllm_rocm:: operator has a fake implementation: a function
    chaining them traces with fake CUDA tensors into a graph of opaque
    custom-op nodes whose outputs are integer tensors (int_prims.py:96-136
    is the reference's pattern)."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    from torch.fx.experimental.proxy_tensor import make_fx

    from idempotent_llm_amd import torch_ops  # noqa: F401
    ops = torch.ops.detllm_rocm
    R, H, I, V, n_q, n_kv = 3, 256, 512, 1000, 4, 2

    def layerish(ids, e8, em, ek, w, wgu, cm, gm, um, dm, head, head_m, err):
        h, k_res, x8, xm, xk = ops.embed_normq(ids, e8, em, ek, None, 0, err)
        P = ops.int_gemm(x8, w).unsqueeze(0)
        x8b, xmb, xkb = ops.residual_normq(P, xm, xk, cm, 20, 20, h, k_res, None, 0)
        Pg = ops.int_gemm(x8b, wgu).unsqueeze(0)
        y8, ym, yk = ops.swiglu_quant(Pg, xmb, xkb, gm, 20, um, 20, dm, 0)
        logits = ops.int_gemm(x8b, head)
        return ops.greedy_pick(logits, head_m), y8, ops.isqrt_i64(xk), ops.ilog2_i64(xm)

    with FakeTensorMode():
        c = lambda *s, dt=torch.int64: torch.empty(*s, dtype=dt, device="cuda")
        args = (c(R), c(V, H, dt=torch.int8), c(V), c(V), c(H, H, dt=torch.int8),
                c(H, 2 * I, dt=torch.int8), c(H), c(I), c(I), c(I),
                c(H, V, dt=torch.int8), c(V), c(1, dt=torch.int32))
        gm = make_fx(layerish, tracing_mode="fake")(*args)
    names = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    for op in ("embed_normq", "int_gemm", "residual_normq", "swiglu_quant", "greedy_pick",
               "isqrt_i64", "ilog2_i64"):
        assert any(f"detllm_rocm.{op}" in n for n in names), op
    for n in gm.graph.nodes:
        v = n.meta.get("val")
        for t in (v if isinstance(v, (tuple, list)) else [v]):
            if isinstance(t, torch.Tensor):
                assert not t.is_floating_point(), n
