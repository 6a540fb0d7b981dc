"""The drop-in boundary on the GPU: the detllm_rocm:: custom operators under
torch.compile(fullgraph=True) and NoFloatMode, their fake implementations
against the real kernels (torch.library.opcheck), and the plugin that lets
the reference's unchanged API (IntQwen3(dir, "rocm"), int_gemm(..., "rocm"),
GraphedDecode(model, ...)) reach this runtime."""

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


def _rnd(shape, lo, hi, dt, seed=0):
    g = np.random.default_rng(seed)
    return torch.from_numpy(g.integers(lo, hi, shape).astype(dt)).cuda()


def test_opcheck_fake_vs_real():
    """register_fake agrees with the kernels on shapes, dtypes and strides."""
    from idempotent_llm_amd import torch_ops  # noqa: F401
    ops = torch.ops.detllm_rocm
    a = _rnd((5, 64), -128, 128, np.int8, 1)
    b = _rnd((64, 48), -128, 128, np.int8, 2)
    h = _rnd((5, 256), -(1 << 20), 1 << 20, np.int32, 3)
    tests = ("test_schema", "test_faketensor")
    torch.library.opcheck(ops.int_gemm.default, (a, b), test_utils=tests)
    torch.library.opcheck(ops.int_gemm.default, (a.view(1, 5, 64), b.view(1, 64, 48)),
                          test_utils=tests)
    torch.library.opcheck(ops.norm_quant.default, (h, None, 0), test_utils=tests)
    logits = _rnd((3, 5000), -1000, 1000, np.int32, 4)
    head_m = _rnd((5000,), 1 << 14, 1 << 16, np.int64, 5)
    torch.library.opcheck(ops.greedy_pick.default, (logits, head_m), test_utils=tests)
    torch.library.opcheck(ops.isqrt_i64.default, (_rnd((100,), 0, 1 << 62, np.int64, 6),),
                          test_utils=tests)


def test_compile_fullgraph_under_no_float_mode():
    """A layer-shaped chain of the custom operators compiles with
    fullgraph=True (one graph, custom ops opaque) and gives the eager bits,
    with NoFloatMode active (the reference's compiled _layer, model.py:434-467,
    calling int_gemm(..., "rocm") is this case)."""
    from idempotent_llm_amd import torch_ops  # noqa: F401
    from idempotent_llm_amd.guard import NoFloatMode
    ops = torch.ops.detllm_rocm
    R, H, I = 4, 256, 512
    h0 = _rnd((R, H), -(1 << 20), 1 << 20, np.int32, 7)
    w = _rnd((H, H), -127, 128, np.int8, 8)
    wgu = _rnd((H, 2 * I), -127, 128, np.int8, 9)
    cm = _rnd((H,), 1 << 14, 1 << 15, np.int64, 10)
    gm = _rnd((I,), 1 << 14, 1 << 15, np.int64, 11)
    um = _rnd((I,), 1 << 14, 1 << 15, np.int64, 12)
    dm = torch.ones(I, dtype=I64, device="cuda")

    def block(h, k_res):
        x8, xm, xk = ops.norm_quant(h, None, 0)
        P = ops.int_gemm(x8, w).unsqueeze(0)
        x8b, xmb, xkb = ops.residual_normq(P, xm, xk, cm, 20, 20, h, k_res, None, 0)
        Pg = ops.int_gemm(x8b, wgu).unsqueeze(0)
        y8, ym, yk = ops.swiglu_quant(Pg, xmb, xkb, gm, 20, um, 20, dm, 0)
        return y8, ym + 1, yk, h.clone(), k_res.clone()

    outs = []
    for compiled in (False, True):
        fn = torch.compile(block, fullgraph=True, backend="aot_eager") if compiled else block
        h = h0.clone()
        k_res = torch.full((R,), 24, dtype=I64, device="cuda")
        with NoFloatMode():
            outs.append(fn(h, k_res))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_plugin_routes_reference_api(tmp_path):
    """With the plugin installed on a package laid out as the reference
    (stand-in, see test_plugin_cpu.py), IntQwen3(dir, "rocm") is this
    runtime and gives its bits, int_gemm(..., "rocm") is exact, and
    GraphedDecode(model, ...) is this package's graphed decode."""
    import sys

    from idempotent_llm_amd import plugin
    from idempotent_llm_amd.graphed import GraphedDecode as RocmGraphed
    from idempotent_llm_amd.model import IntQwen3 as RocmIntQwen3
    sys.path.insert(0, __import__("os").path.dirname(__file__))
    from test_plugin_cpu import _standin
    pkg = _standin("detllm_standin_gpu")
    d = str(tmp_path)
    art.make_artifact(d, art.TINY, seed=11)
    plugin.install(pkg)
    try:
        m = pkg.model.IntQwen3(d, "rocm")
        assert isinstance(m, RocmIntQwen3) and isinstance(m, pkg.model.IntQwen3)
        direct = RocmIntQwen3(d, "rocm")
        ids = torch.from_numpy(art.prompt_ids(110, 24, art.TINY["vocab"]))[None].cuda()
        pos = torch.arange(24, device="cuda")[None]
        assert torch.equal(m.forward(ids, pos)[0], direct.forward(ids, pos)[0])
        a = _rnd((33, 100), -128, 128, np.int8, 13)
        b = _rnd((100, 70), -128, 128, np.int8, 14)
        got = pkg.backends.int_gemm(a, b, "rocm")
        assert torch.equal(got.cpu().to(I64), a.cpu().to(I64) @ b.cpu().to(I64))
        p = _rnd((9, 21), 0, 129, np.int32, 15)
        v = _rnd((21, 6), -128, 128, np.int8, 16)
        assert torch.equal(pkg.backends.int_gemm_u8i8(p, v, "rocm").cpu().to(I64),
                           p.cpu().to(I64) @ v.cpu().to(I64))
        lg, _, _, cache = m.forward(ids, pos)
        gd = pkg.graphed.GraphedDecode(m, cache, torch.full((1,), 24, dtype=I64, device="cuda"))
        assert isinstance(gd, RocmGraphed)
        gd.step(m.greedy_pick(lg[:, -1]))
        m.raise_if_device_error()
    finally:
        plugin.uninstall(pkg)


class _Dispatched(__import__("torch.utils._python_dispatch", fromlist=["x"]).TorchDispatchMode):
    """Records the namespace of every operator dispatched while active."""

    def __init__(self):
        super().__init__()
        self.namespaces = set()

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        self.namespaces.add(getattr(func, "namespace", ""))
        return func(*args, **(kwargs or {}))


def test_plugin_reference_routes_reach_the_hip_kernels(tmp_path):
    """Through the reference package's unchanged API (stand-in layout, see
    test_plugin_cpu.py), with the plugin installed:
    * ops.di_matmul(..., "rocm") (ops/di_matmul.py:34-40, which imports
      int_gemm by name) equals the oracle's composition and dispatches none
      of the reference package's operators;
    * a subclass of the reference IntQwen3 overriding _lm_head with zeros
      (a ZeroHead diagnostic) runs this runtime: zero logits at every step
      of a graphed generation, greedy picks of id 0 (lowest-id tie-break);
    * a seam override that calls super() and a reference primitive on the
      device gets this runtime's bits, and the primitive runs this package's
      HIP kernel instead of the reference's Triton kernel (its stand-in
      counts launches: none while installed, one after uninstall)."""
    import sys

    from idempotent_llm_amd import plugin
    from idempotent_llm_amd.model import IntQwen3 as RocmIntQwen3
    from oracle import ops as oops
    sys.path.insert(0, __import__("os").path.dirname(__file__))
    from test_plugin_cpu import _standin
    name = "detllm_standin_routes"
    pkg = _standin(name)
    state = pkg.ops.int_prims.STATE
    d = str(tmp_path)
    art.make_artifact(d, art.TINY, seed=11)
    ids = torch.from_numpy(art.prompt_ids(110, 24, art.TINY["vocab"]))[None].cuda()
    pos = torch.arange(24, device="cuda")[None]
    plugin.install(pkg)
    try:
        rnd = np.random.default_rng(21)
        x = rnd.integers(-(1 << 30), 1 << 30, (37, 256)).astype(np.int64)
        xm = rnd.integers(1 << 15, 1 << 16, (37, 1)).astype(np.int64)
        xk = rnd.integers(20, 40, (37, 1)).astype(np.int64)
        w = rnd.integers(-127, 128, (256, 96)).astype(np.int8)
        wm = rnd.integers(1 << 14, 1 << 16, (96,)).astype(np.int64)
        cu = lambda a: torch.from_numpy(a).cuda()
        with _Dispatched() as rec:
            y8, m8, k8 = pkg.ops.di_matmul(cu(x), cu(xm), cu(xk), cu(w), cu(wm), 24, "rocm")
        oy, om, ok = oops.di_matmul(x, xm, xk, w, wm, 24)
        assert np.array_equal(y8.cpu().numpy(), oy)
        assert np.array_equal(m8.cpu().numpy(), om) and np.array_equal(k8.cpu().numpy(), ok)
        assert name not in rec.namespaces and "detllm_rocm" in rec.namespaces

        class ZeroHead(pkg.model.IntQwen3):
            def _lm_head(self, x8, xm, xk):
                return torch.zeros(*x8.shape[:-1], self.vocab, dtype=torch.int32,
                                   device=x8.device)

        z = ZeroHead(d, "rocm")
        assert isinstance(z, RocmIntQwen3) and isinstance(z, ZeroHead)
        with _Dispatched() as rec:
            lg = z.forward(ids, pos)[0]
        assert name not in rec.namespaces
        assert lg.shape == (1, 24, art.TINY["vocab"]) and not lg.any()
        toks, steps = z.generate(ids, 5, use_graph=True)
        assert toks.tolist() == [[0] * 5] and not any(s.any() for s in steps)

        calls = []

        class Probe(pkg.model.IntQwen3):
            def _attn_scores(self, q8, qm, qk, K8r, L, group, aux=None):
                calls.append(L.idx)
                lg2 = pkg.ops.int_prims.ilog2_i64(qm.clamp(min=1))
                want = [v.bit_length() - 1 for v in qm.clamp(min=1).reshape(-1).tolist()]
                assert lg2.is_cuda and lg2.reshape(-1).tolist() == want
                return super()._attn_scores(q8, qm, qk, K8r, L, group, aux)

        probe = Probe(d, "rocm")
        direct = RocmIntQwen3(d, "rocm")
        assert torch.equal(probe.forward(ids, pos)[0], direct.forward(ids, pos)[0])
        assert calls == list(range(art.TINY["n_layers"]))
        assert state.TRITON_CALLS == 0
        probe.raise_if_device_error()
    finally:
        plugin.uninstall(pkg)
    pkg.ops.int_prims.ilog2_i64(torch.ones(3, dtype=torch.int64, device="cuda"))
    assert state.TRITON_CALLS == 1
