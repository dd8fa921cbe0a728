"""Builds libcrispybits_hip.so (the C-ABI of include/crispybits_hip.h) for gfx950.

Each csrc/ translation unit is compiled with hipcc in parallel, then linked into
``crispybits_kernels/libcrispybits_hip.so`` next to this file, so the library is
in-tree (it travels with the source snapshot and is what ``_C`` loads).

Usage: ``python -m crispybits_kernels._build`` (from llm_quantization-kernel_amd/)
or ``crispybits_kernels._build.build()``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)                       # llm_quantization-kernel_amd/
CSRC = os.path.join(ROOT, "csrc")
OBJ_DIR = os.path.join(ROOT, "_build")
LIB_NAME = "libcrispybits_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = os.environ.get("CRISPYBITS_ARCH", "gfx950")

SOURCES = ["abi.cpp", "gemv_mfma.hip", "gemv_stream.hip", "gemv_generic.hip", "gemm.hip", "gemm_f16.hip", "unpack.hip", "quant.hip"]

# -packed-fp32-ops is disabled: the kernels never rely on v_pk_*_f32.
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-munsafe-fp-atomics",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wno-unused-result", "-I" + CSRC, "-I" + os.path.join(os.path.dirname(ROOT), "include")]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), *HIP_FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every HIP/C++ source and link the shared library; returns its path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    jobs = min(len(SOURCES), max(1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
