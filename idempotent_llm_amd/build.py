"""Build the HIP library (gfx950) and the host test shim, in-tree.

``libdetllm_hip.so``      — every kernel + the extern "C" boundary
                            (declared in include/detllm_hip.h);
``libdetllm_intops_host.so`` — intops.h compiled for the CPU, used by the
                            CPU test suite to check the integer routines the
                            kernels share.

hipcc compiles each .hip translation unit to an object in parallel, then
links one shared library. Flags: gfx950 only; packed-fp32 instruction
selection disabled (no float arithmetic is used, the flag guards against
compiler-generated v_pk_*_f32).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(os.path.dirname(PKG), "_build")
LIB = os.path.join(PKG, "libdetllm_hip.so")
HOST_LIB = os.path.join(PKG, "libdetllm_intops_host.so")
HIP_SOURCES = ("gemm.hip", "rowops.hip", "attention.hip")
ARCH = "gfx950"
HIPCC_FLAGS = ["-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-Wno-unused-result"]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build the library")


def _run(cmd):
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{p.stdout}\n{p.stderr}")
    return p


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hipcc = _hipcc()
    objs = []
    jobs = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        objs.append(obj)
        jobs.append([hipcc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for p in ex.map(_run, jobs):
            if verbose and p.stderr:
                print(p.stderr)
    tmp = LIB + ".tmp"
    _run([hipcc, "-shared", f"--offload-arch={ARCH}", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    build_host_shim()
    return LIB


def build_host_shim() -> str:
    gxx = shutil.which("g++") or "g++"
    tmp = HOST_LIB + ".tmp"
    _run([gxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-I", CSRC,
          os.path.join(CSRC, "intops_host.cpp"), "-o", tmp])
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


if __name__ == "__main__":
    print(build(verbose=True))
