"""``crispybits_kernels._C`` -- the op bindings of the gfx950 kernels.

Drop-in for the reference's pybind11 module (Kernel/csrc/bindings.cpp:32-40): the same seven
functions with the same argument order (``packed_gemv``, ``packed_gemm``, ``fused_gate_up``,
``fused_qkv``, ``sm_count``, ``tile_n``, ``max_rho``), tensors in and tensors out, plus the
additive ``packed_gemm_gate_up``, ``unpack_codes``, ``quantize_pack``, ``decode_plan``,
``timer_start`` / ``timer_stop`` and ``stream_probe``.  They live in the compiled module ``_ext``
(csrc/torch_ext.cpp), a PyTorch-ROCm C++ extension over the C ABI of ``libcrispybits_hip.so``
(include/crispybits_hip.h); its tensor checks raise ``RuntimeError`` like ``TORCH_CHECK``, and the
kernels run on torch's current HIP stream of x's device.

Importing this module fails with ImportError when either library has not been built: there is
no CPU fallback.
"""
import os

LIB_NAME = "libcrispybits_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is not built (run crispybits_kernels._build.build())")

import torch  # noqa: E402,F401  (loads the torch libraries the extension links)

from ._ext import (ABI_VERSION, decode_plan, fused_gate_up, fused_qkv, max_rho, packed_gemm,  # noqa: E402
                   packed_gemm_gate_up, packed_gemv, quantize_pack, sm_count, stream_probe, tile_n, timer_start,
                   timer_stop, unpack_codes)

__all__ = ["packed_gemv", "packed_gemm", "fused_gate_up", "fused_qkv", "sm_count", "tile_n", "max_rho",
           "packed_gemm_gate_up", "unpack_codes", "quantize_pack", "decode_plan", "timer_start", "timer_stop", "stream_probe", "ABI_VERSION",
           "LIB_PATH"]
