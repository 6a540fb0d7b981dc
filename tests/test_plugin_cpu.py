"""The drop-in registration (idempotent_llm_amd.plugin) and the custom
operators' fake implementations, on the CPU.

The reference package is not imported here (its code is read, not run); a
stand-in package with the same module layout and public names — backends
(BACKENDS, BACKEND_ALIASES, canonical_backend, int_gemm, int_gemm_u8i8),
model (IntQwen3 importing int_gemm by name), graphed (GraphedDecode) — takes
its place, holding only what the plugin touches."""

import sys
import types

import numpy as np
import pytest
import torch


def _standin(name="detllm_standin"):
    pkg = types.ModuleType(name)
    pkg.__path__ = []
    B = types.ModuleType(name + ".backends")
    exec("""
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
""", B.__dict__)
    M = types.ModuleType(name + ".model")
    M.__dict__["_B"] = B
    exec("""
int_gemm = _B.int_gemm
class IntQwen3:
    def __init__(self, artifact_dir, backend="reference"):
        self.backend = _B.canonical_backend(backend)
        self.artifact_dir = artifact_dir
""", M.__dict__)
    G = types.ModuleType(name + ".graphed")
    exec("""
class GraphedDecode:
    def __init__(self, model, cache, lens, mode="capture", layer_compile=True):
        self.model = model
""", G.__dict__)
    pkg.backends, pkg.model, pkg.graphed = B, M, G
    for m in (pkg, B, M, G):
        sys.modules[m.__name__] = m
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
    with pytest.raises(ValueError):
        B.canonical_backend("rocm")
    plugin.install(standin)
    plugin.install(standin)                       # idempotent
    assert B.canonical_backend("rocm") == "rocm" and B.canonical_backend("hip") == "rocm"
    assert B.canonical_backend("cpu") == "reference"
    a = torch.tensor([[1, -2], [3, 4]], dtype=torch.int8)
    b = torch.tensor([[5, 6], [-7, 8]], dtype=torch.int8)
    assert torch.equal(B.int_gemm(a, b, "reference"), a.int() @ b.int())
    assert M.int_gemm is B.int_gemm               # the name model.py imported
    ref = M.IntQwen3("dir", "reference")
    assert type(ref) is M.IntQwen3 and ref.backend == "reference"
    # "rocm" reaches this package's runtime (which needs a GPU: on the CPU it
    # refuses instead of falling back)
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="gfx950"):
            M.IntQwen3("dir", "rocm")
        # the rocm GEMM has no CPU kernel either
        with pytest.raises(Exception):
            B.int_gemm(a, b, "rocm")

    class Sub(M.IntQwen3):                          # diagnostic subclasses stay reference-side
        pass
    assert type(Sub("dir", "rocm")) is Sub
    plugin.uninstall(standin)
    with pytest.raises(ValueError):
        B.canonical_backend("rocm")
    assert type(M.IntQwen3("dir", "cpu")) is M.IntQwen3
    assert RocmIntQwen3 is not M.IntQwen3


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
