"""The C-ABI library loads without a GPU and exports every symbol that
include/detllm_hip.h declares; the Python binding covers each with the
header's arity. Also the host-side API checks that need no GPU."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "detllm_hip.h")
LIB = os.path.join(ROOT, "idempotent_llm_amd", "libdetllm_hip.so")


def _declarations():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"int\s+(detllm_\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.S):
        params = [p for p in m.group(2).split(",") if p.strip()]
        decls[m.group(1)] = len(params)
    return decls


def test_header_declares_entry_points():
    decls = _declarations()
    assert len(decls) >= 20
    assert "detllm_igemm_nt" in decls and "detllm_attn_decode" in decls


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built (run build())")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    missing = [n for n in _declarations() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_matches_header_arity():
    from idempotent_llm_amd._lib import HOST_ONLY, SIGNATURES
    decls = _declarations()
    assert set(SIGNATURES) == set(decls)
    for name, n in decls.items():
        assert len(SIGNATURES[name]) == n, name
        if name not in HOST_ONLY:   # every entry that enqueues work takes a stream last
            assert SIGNATURES[name][-1] == "s", name


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built (run build())")
def test_gemv_plan_host_entry():
    """The K-split planner runs on the host (no GPU needed): 1..8 partials,
    1 for wide products, a multiple-of-64 chunk that the kernel accepts."""
    from idempotent_llm_amd._lib import gemv_plan
    for N, K in ((4096, 1024), (1024, 2048), (6144, 1024), (1024, 3072), (151936, 1024),
                 (1024, 256), (16, 16), (48, 4096)):
        ks = gemv_plan(8, N, K)
        assert 1 <= ks <= 8
        chunk = (K + ks - 1) // ks
        chunk = (chunk + 63) // 64 * 64
        assert (K + chunk - 1) // chunk == ks
    assert gemv_plan(1, 151936, 1024) == 1
    assert gemv_plan(1, 1024, 3072) > 1
    # several rows split K in two between one and four column groups per CU
    # (one row keeps one split there: the fused-operand kernels' plan)
    assert gemv_plan(8, 6144, 1024) == 2
    assert gemv_plan(1, 6144, 1024) == 1
    assert gemv_plan(8, 4096, 1024) == 1
    with pytest.raises(RuntimeError):
        gemv_plan(65, 1024, 1024)


def test_backend_names():
    # the reference's tests/test_ops.py:33-48, extended by "rocm"
    from idempotent_llm_amd.backends import BACKENDS, canonical_backend
    assert canonical_backend("cpu") == "reference"
    assert canonical_backend("hip") == "rocm"
    for name in BACKENDS:
        assert canonical_backend(name) == name
    for bad in ("mps", "metal", "CPU", "reference ", "ROCM"):
        with pytest.raises(ValueError):
            canonical_backend(bad)


def test_int_gemm_rejects_non_int8_and_other_backends():
    import torch

    from idempotent_llm_amd.backends import int_gemm
    a = torch.zeros(2, 3, dtype=torch.int8)
    with pytest.raises(AssertionError):
        int_gemm(a.to(torch.int32), torch.zeros(3, 2, dtype=torch.int8), "rocm")
    with pytest.raises(AssertionError):
        int_gemm(a, torch.zeros(4, 2, dtype=torch.int8), "rocm")
    with pytest.raises(ValueError):
        int_gemm(a, torch.zeros(3, 2, dtype=torch.int8), "reference")


def test_guard_fires_on_float():
    import torch

    from idempotent_llm_amd.guard import FloatLeakError, NoFloatMode
    with pytest.raises(FloatLeakError):
        with NoFloatMode():
            torch.ones(3).float() * 2.0
    with NoFloatMode():
        (torch.ones(3, dtype=torch.int64) * 2).sum()


def test_model_requires_gpu_loudly(tmp_path):
    import torch

    from idempotent_llm_amd import artifact as art
    from idempotent_llm_amd.model import IntQwen3
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    d = art.make_artifact(str(tmp_path), art.TINY, seed=1)
    with pytest.raises(RuntimeError):
        IntQwen3(d, backend="rocm")
    with pytest.raises(ValueError):
        IntQwen3(d, backend="cpu")


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    # No CPU fallback: with the shared library absent, loading it and every
    # call through the C-ABI raise LibraryMissing instead of computing.
    from idempotent_llm_amd import _lib
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "libdetllm_hip.so"))
    with pytest.raises(_lib.LibraryMissing, match="no CPU fallback"):
        _lib.load()
    with pytest.raises(_lib.LibraryMissing):
        _lib.gemv_plan(8, 1024, 1024)
    with pytest.raises(_lib.LibraryMissing):
        _lib.call("detllm_igemv_plan", 8, 1024, 1024)
