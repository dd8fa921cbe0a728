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

SOURCES = ["abi.cpp", "gemv_stream.hip", "gemv_any.hip", "gemm.hip", "gemm_f16.hip", "gemm_f32.hip",
           "unpack.hip", "quant.hip", "probe.hip"]

# -packed-fp32-ops is disabled: the kernels never rely on v_pk_*_f32.
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-munsafe-fp-atomics",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wno-unused-result", "-I" + CSRC, "-I" + os.path.join(os.path.dirname(ROOT), "include")]


# Per-file compiler flags beside HIP_FLAGS (none at present).
FILE_FLAGS: dict = {}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), *HIP_FLAGS, *FILE_FLAGS.get(src, []), "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


EXT_SOURCE = "torch_ext.cpp"


def _ext_path() -> str:
    import sysconfig
    return os.path.join(PKG_DIR, "_ext" + sysconfig.get_config_var("EXT_SUFFIX"))


def _torch_flags():
    """Include paths, defines and libraries of the installed torch (ROCm build) for a host-only
    C++ extension; no torch.utils.cpp_extension (it would hipify), no device code."""
    import sysconfig
    import torch
    tdir = os.path.dirname(torch.__file__)
    inc = [os.path.join(tdir, "include"), os.path.join(tdir, "include", "torch", "csrc", "api", "include"),
           sysconfig.get_paths()["include"], "/opt/rocm/include", os.path.join(os.path.dirname(ROOT), "include")]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    defs = ["-DTORCH_EXTENSION_NAME=_ext", "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
            "-DUSE_ROCM=1", "-D__HIP_PLATFORM_AMD__=1"]
    libdir = os.path.join(tdir, "lib")
    libs = [f"-L{libdir}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
            f"-Wl,-rpath,{libdir}"]
    return [f"-I{p}" for p in inc] + defs, libs


def _compile_ext(verbose: bool) -> str:
    obj = os.path.join(OBJ_DIR, "torch_ext.o")
    cflags, _ = _torch_flags()
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-w", *cflags, "-c",
           os.path.join(CSRC, EXT_SOURCE), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed for {EXT_SOURCE}:\n{r.stdout}\n{r.stderr}")
    return obj


def _run(cmd, verbose, what):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{r.stdout}\n{r.stderr}")


def build(verbose: bool = False) -> str:
    """Compile every HIP/C++ source, link the C-ABI library and the torch op module over it;
    returns the library's path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    jobs = min(len(SOURCES) + 1, max(1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(jobs) as ex:
        ext_obj = ex.submit(_compile_ext, verbose)
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
        ext_obj = ext_obj.result()
    tmp = LIB_PATH + ".tmp"
    _run([_hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp], verbose, "link")
    os.replace(tmp, LIB_PATH)
    _, libs = _torch_flags()
    ext = _ext_path()
    _run([os.environ.get("CXX", "g++"), "-shared", "-fPIC", ext_obj, "-o", ext + ".tmp", f"-L{PKG_DIR}",
          "-lcrispybits_hip", "-Wl,-rpath,$ORIGIN", *libs], verbose, "extension link")
    os.replace(ext + ".tmp", ext)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
