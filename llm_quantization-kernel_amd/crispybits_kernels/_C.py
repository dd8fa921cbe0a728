"""``crispybits_kernels._C`` -- torch-facing binding of the gfx950 C-ABI library.

Drop-in for the reference's pybind11 module (Kernel/csrc/bindings.cpp:32-40): the
same seven functions with the same argument order, tensors in and tensors out,
plus additive entries (``unpack_codes``, ``fused_qkv`` with per-projection
widths, ``quantize_pack``).  Tensor checks restate host_utils.h:38-87 and raise ``RuntimeError``
like ``TORCH_CHECK``; the kernels run on torch's current HIP stream of x's device.

The compute is libcrispybits_hip.so (include/crispybits_hip.h); importing this
module fails with ImportError when the library has not been built, and there is
no CPU fallback.
"""
from __future__ import annotations

import ctypes
import math
import os

import torch

LIB_NAME = "libcrispybits_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is not built (run crispybits_kernels._build.build())")

_lib = ctypes.CDLL(LIB_PATH)

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64

_SIGS = {
    "cbk_last_error": (ctypes.c_char_p, []),
    "cbk_abi_version": (_I, []),
    "cbk_sm_count": (_I, [_I, ctypes.POINTER(_I)]),
    "cbk_tile_n": (_I, []),
    "cbk_max_rho": (_I, [_I, _I, _I, ctypes.POINTER(_I)]),
    "cbk_decode_plan": (_I, [_I, _L, _L, _I, _L, _L, _L, _I, _I, _I, _I, _I, _I, _I, _P]),
    "cbk_gemv_partial_floats": (_L, [_I, _L, _L, _L, _I, _I]),
    "cbk_packed_gemv": (_I, [_P, _I, _L, _L, _P, _P, _P, _P, _L, _I, _I, _I, _I, _I, _P, _P, _P, _I, _P]),
    "cbk_packed_gemv_noalloc": (_I, [_P, _I, _L, _L, _P, _P, _P, _P, _L, _I, _I, _I, _I, _I, _P, _I, _P]),
    "cbk_fused_gate_up": (_I, [_P, _I, _L, _L, _P, _P, _P, _P, _P, _P, _L, _I, _I, _I, _I, _P, _P, _P, _I, _P]),
    "cbk_fused_qkv": (_I, [_P, _I, _L, _L,
                           _P, _P, _P, _P, _L, _P, _P, _P, _P, _L, _P, _P, _P, _P, _L,
                           _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _I, _P]),
    "cbk_fused_qkv_mixed": (_I, [_P, _I, _L, _L,
                                 _P, _P, _P, _P, _L, _P, _P, _P, _P, _L, _P, _P, _P, _P, _L,
                                 _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _I, _P]),
    "cbk_packed_gemm": (_I, [_P, _I, _L, _L, _P, _P, _P, _P, _L, _I, _I, _I, _I, _P, _I, _P]),
    "cbk_unpack_codes": (_I, [_P, _L, _L, _I, _P, _I, _P]),
    "cbk_quantize_pack": (_I, [_P, _I, _L, _L, _I, _I, _I, _P, _P, _P, _I, _I, _P]),
    "cbk_timer_start": (_I, [_I]),
    "cbk_timer_stop": (_I, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I), ctypes.POINTER(ctypes.c_double), _I]),
}
for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(_lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args

ABI_VERSION = _lib.cbk_abi_version()
EXPORTS = tuple(_SIGS)

_DT = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
_KIND = {"gemv": 0, "qkv": 1, "gate_up": 2}


def _raise(rc: int):
    if rc != 0:
        raise RuntimeError(_lib.cbk_last_error().decode())


def _ptr(t):
    return None if t is None or t.numel() == 0 else t.data_ptr()


try:                                                   # the raw handle without a Stream object
    _raw_stream = torch._C._cuda_getCurrentRawStream
except AttributeError:                                 # pragma: no cover
    _raw_stream = None


def _stream(x: torch.Tensor) -> int:
    if _raw_stream is not None:
        return _raw_stream(x.get_device())
    return torch.cuda.current_stream(x.device).cuda_stream


def _check(cond: bool, msg: str):
    if not cond:
        raise RuntimeError(msg)


def _check_x(x: torch.Tensor, K: int):
    if x.is_cuda and x.dim() == 2 and x.is_contiguous() and x.size(1) == K and x.dtype in _DT:
        return
    _check(x.is_cuda, "x must be CUDA")
    _check(x.dim() == 2, "x must be [B,K]")
    _check(x.is_contiguous(), "x must be contiguous")
    _check(x.size(1) == K, "x K != in_features")
    _check(x.dtype in _DT, "x must be fp16/bf16/fp32")


def _weight_ok(x, packed, scales, zeros, bits, K, group_size) -> bool:
    """Every condition of _check_weight at once (the common, passing case; devices compared
    by index, -1 for a CPU tensor)."""
    dev, dt = x.get_device(), x.dtype
    return (packed.dtype == torch.int32 and packed.get_device() == dev and scales.get_device() == dev
            and zeros.get_device() == dev
            and scales.dtype == dt and zeros.dtype == dt and packed.dim() == 2 and scales.dim() == 2
            and packed.is_contiguous() and scales.is_contiguous() and zeros.is_contiguous()
            and scales.shape == zeros.shape and scales.size(0) == packed.size(0) and bits in (2, 3, 4)
            and group_size > 0 and group_size % 32 == 0 and packed.size(1) == -(-K // 32) * bits
            and scales.size(1) == -(-K // group_size))


def _check_weight(x, packed, scales, zeros, bits, K, group_size, name):
    if x.is_cuda and _weight_ok(x, packed, scales, zeros, bits, K, group_size):
        return
    _check(packed.is_cuda and scales.is_cuda and zeros.is_cuda, f"{name}: tensors must be CUDA")
    _check(packed.device == x.device, f"{name}: weight and activation on different devices")
    _check(scales.device == x.device and zeros.device == x.device, f"{name}: weight and activation on different devices")
    _check(packed.dtype == torch.int32, f"{name}: packed must be torch.int32")
    _check(packed.dim() == 2 and scales.dim() == 2, f"{name}: packed/scales must be 2-D")
    _check(packed.is_contiguous() and scales.is_contiguous() and zeros.is_contiguous(),
           f"{name}: weight tensors must be contiguous")
    _check(scales.shape == zeros.shape, f"{name}: scale/zero shape mismatch")
    _check(scales.size(0) == packed.size(0), f"{name}: metadata rows != output rows")
    _check(scales.dtype == x.dtype and zeros.dtype == x.dtype, f"{name}: metadata dtype must match x")
    _check(bits in (2, 3, 4), f"{name}: bits must be 2/3/4")
    _check(group_size > 0 and group_size % 32 == 0, f"{name}: group_size must be a positive multiple of 32")
    _check(packed.size(1) == math.ceil(K / 32) * bits,
           f"{name}: packed row must hold exactly ceil(K/32)*bits words (rows padded to 32 codes)")
    _check(scales.size(1) == math.ceil(K / group_size), f"{name}: expected ceil(K/group_size) groups")


def _bias(bias, x, N):
    if bias is None:
        return None
    if bias.numel() == 0:
        return None
    _check(bias.is_cuda and bias.device == x.device, "bias must be on x's device")
    _check(bias.numel() == N, "bias length must equal out_features")
    _check(bias.dtype == x.dtype, "bias dtype must match x")
    _check(bias.is_contiguous(), "bias must be contiguous")
    return bias


def _workspace(ws, x):
    if ws is None:
        return None
    if ws.numel() >= 2:
        _check(ws.is_cuda and ws.device == x.device, "workspace must be on x's device")
        _check(ws.dtype == torch.int32 and ws.is_contiguous(), "workspace must be contiguous int32")
        return ws
    return None


_PARTIAL_FLOATS = {}


def _partial(x, M, V, K, group_size, split_k):
    key = (_DT[x.dtype], M, V, K, group_size, int(split_k))
    n = _PARTIAL_FLOATS.get(key)
    if n is None:
        n = _PARTIAL_FLOATS[key] = _lib.cbk_gemv_partial_floats(*key)
    return torch.empty(n, dtype=torch.float32, device=x.device) if n > 0 else None


def packed_gemv(x, packed, scales, zeros, bias, bits, in_features, group_size, split_k, rho, act, workspace):
    bits, K, gs, split_k, rho, act = int(bits), int(in_features), int(group_size), int(split_k), int(rho), int(act)
    _check_x(x, K)
    _check_weight(x, packed, scales, zeros, bits, K, gs, "packed_gemv")
    _check(split_k >= 1, "split_k must be >= 1")
    _check(0 <= act <= 2, "act must be 0 (none), 1 (relu) or 2 (silu)")
    N, M = packed.size(0), x.size(0)
    b = _bias(bias, x, N)
    ws = _workspace(workspace, x)
    out = x.new_empty((M, N))
    if M == 0:
        return out
    part = _partial(x, M, N, K, gs, split_k)
    dev = x.get_device()
    rc = _lib.cbk_packed_gemv(x.data_ptr(), _DT[x.dtype], M, K, packed.data_ptr(), scales.data_ptr(),
                              zeros.data_ptr(), _ptr(b), N, bits, gs, split_k, rho, act, _ptr(ws), _ptr(part),
                              out.data_ptr(), dev, _raw_stream(dev) if _raw_stream is not None else _stream(x))
    if rc:
        _raise(rc)
    return out


def fused_gate_up(x, wg, sg, zg, wu, su, zu, bits, in_features, group_size, split_k, rho, workspace):
    bits, K, gs, split_k, rho = int(bits), int(in_features), int(group_size), int(split_k), int(rho)
    _check_x(x, K)
    _check_weight(x, wg, sg, zg, bits, K, gs, "fused_gate_up(gate)")
    _check_weight(x, wu, su, zu, bits, K, gs, "fused_gate_up(up)")
    _check(wg.shape == wu.shape, "gate/up packed shapes must match")
    _check(split_k >= 1, "split_k must be >= 1")
    ws = _workspace(workspace, x)
    N, M = wg.size(0), x.size(0)
    out = x.new_empty((M, N))
    if M == 0:
        return out
    part = _partial(x, M, 2 * N, K, gs, split_k)
    rc = _lib.cbk_fused_gate_up(x.data_ptr(), _DT[x.dtype], M, K, wg.data_ptr(), sg.data_ptr(),
                                zg.data_ptr(), wu.data_ptr(), su.data_ptr(), zu.data_ptr(), N, bits, gs, split_k,
                                rho, _ptr(ws), _ptr(part), out.data_ptr(), x.get_device(), _stream(x))
    if rc:
        _raise(rc)
    return out


def fused_qkv(x, wq, sq, zq, bq, wk, sk, zk, bk, wv, sv, zv, bv, rope_cos, rope_sin, head_dim, perm_hd,
              bits, in_features, group_size, split_k, rho, workspace):
    """``bits`` is one width (the reference's signature) or a (q, k, v) tuple of widths."""
    mixed = isinstance(bits, (tuple, list))
    bq_, bk_, bv_ = (int(b) for b in bits) if mixed else (int(bits),) * 3
    K, gs, split_k, rho = int(in_features), int(group_size), int(split_k), int(rho)
    head_dim, perm_hd = int(head_dim), int(perm_hd)
    _check_x(x, K)
    _check_weight(x, wq, sq, zq, bq_, K, gs, "fused_qkv(q)")
    _check_weight(x, wk, sk, zk, bk_, K, gs, "fused_qkv(k)")
    _check_weight(x, wv, sv, zv, bv_, K, gs, "fused_qkv(v)")
    _check(split_k >= 1, "split_k must be >= 1")
    B = x.size(0)
    if perm_hd > 0:
        _check(perm_hd % 2 == 0, "perm head_dim must be even")
        _check(wq.size(0) % perm_hd == 0 and wk.size(0) % perm_hd == 0, "Q/K widths must be multiples of head_dim")
    rope = rope_cos is not None and rope_cos.numel() > 0
    rc = rs = None
    if rope:
        _check(perm_hd > 0 and perm_hd == head_dim,
               "fused RoPE needs Q/K weights stored pair-interleaved with the same head_dim "
               "(ops.permute_for_rope / install_bitmap(fuse_rope=True))")
        _check(rope_cos.shape == rope_sin.shape, "cos/sin shape mismatch")
        _check(rope_cos.numel() == B * head_dim, "cos/sin must be [B, head_dim] (one row per x row)")
        rc = rope_cos.to(device=x.device, dtype=torch.float32).contiguous()
        rs = rope_sin.to(device=x.device, dtype=torch.float32).contiguous()
    nq, nk, nv = wq.size(0), wk.size(0), wv.size(0)
    b = (_bias(bq, x, nq), _bias(bk, x, nk), _bias(bv, x, nv))
    ws = _workspace(workspace, x)
    outs = [x.new_empty((B, n)) for n in (nq, nk, nv)]
    if B == 0:
        return outs
    part = _partial(x, B, nq + nk + nv, K, gs, split_k)
    common = (x.data_ptr(), _DT[x.dtype], B, K,
              wq.data_ptr(), sq.data_ptr(), zq.data_ptr(), _ptr(b[0]), nq,
              wk.data_ptr(), sk.data_ptr(), zk.data_ptr(), _ptr(b[1]), nk,
              wv.data_ptr(), sv.data_ptr(), zv.data_ptr(), _ptr(b[2]), nv,
              _ptr(rc), _ptr(rs), head_dim if rope else 0, perm_hd)
    tail = (_ptr(ws), _ptr(part), outs[0].data_ptr(), outs[1].data_ptr(), outs[2].data_ptr(),
            x.get_device(), _stream(x))
    if bq_ == bk_ == bv_:
        _raise(_lib.cbk_fused_qkv(*common, bq_, gs, split_k, rho, *tail))
    else:
        _raise(_lib.cbk_fused_qkv_mixed(*common, bq_, bk_, bv_, gs, split_k, rho, *tail))
    return outs


def packed_gemm(x, packed, scales, zeros, bias, bits, in_features, group_size, act, use_tensor_cores):
    bits, K, gs, act = int(bits), int(in_features), int(group_size), int(act)
    _check_x(x, K)
    _check_weight(x, packed, scales, zeros, bits, K, gs, "packed_gemm")
    _check(0 <= act <= 2, "act must be 0 (none), 1 (relu) or 2 (silu)")
    N = packed.size(0)
    b = _bias(bias, x, N)
    out = torch.empty((x.size(0), N), dtype=x.dtype, device=x.device)
    if x.size(0) == 0:
        return out
    _raise(_lib.cbk_packed_gemm(x.data_ptr(), _DT[x.dtype], x.size(0), K, packed.data_ptr(), scales.data_ptr(),
                                zeros.data_ptr(), _ptr(b), N, bits, gs, act, 1 if use_tensor_cores else 0,
                                out.data_ptr(), x.get_device(), _stream(x)))
    return out


def unpack_codes(packed, bits, in_features):
    """Additive test hook: int32 codes [N, K] decoded on the device."""
    bits, K = int(bits), int(in_features)
    _check(packed.is_cuda and packed.dtype == torch.int32 and packed.is_contiguous() and packed.dim() == 2,
           "packed must be a contiguous 2-D CUDA int32 tensor")
    _check(packed.size(1) == math.ceil(K / 32) * bits, "packed row must hold exactly ceil(K/32)*bits words")
    out = torch.empty((packed.size(0), K), dtype=torch.int32, device=packed.device)
    _raise(_lib.cbk_unpack_codes(packed.data_ptr(), packed.size(0), K, bits, out.data_ptr(), packed.device.index,
                                 _stream(packed)))
    return out


def quantize_pack(weight, bits, group_size=128, dtype=torch.float16, scheme=0):
    """Additive: the format producer on the device -- (packed int32 [N, ceil(K/32)*bits],
    scales, zeros [N, ceil(K/g)] in ``dtype``) of a CUDA weight [N, K], bit-identical to
    reference.quantize_affine + pack_codes (reference.py:10-55) on the CPU (scheme 0), or
    to the paper quantizer crispybits_quant/affine.py:28-71 (scheme 1)."""
    bits, gs, scheme = int(bits), int(group_size), int(scheme)
    _check(weight.is_cuda and weight.dim() == 2, "weight must be a 2-D CUDA tensor")
    _check(weight.dtype in _DT, "weight must be fp16/bf16/fp32")
    _check(dtype in _DT, "scales/zeros dtype must be fp16/bf16/fp32")
    w = weight.contiguous()
    N, K = w.shape
    G = math.ceil(K / gs) if gs > 0 else 0
    packed = torch.empty((N, math.ceil(K / 32) * bits), dtype=torch.int32, device=w.device)
    scales = torch.empty((N, G), dtype=dtype, device=w.device)
    zeros = torch.empty((N, G), dtype=dtype, device=w.device)
    _raise(_lib.cbk_quantize_pack(w.data_ptr(), _DT[w.dtype], N, K, bits, gs, scheme, packed.data_ptr(),
                                  scales.data_ptr(), zeros.data_ptr(), _DT[dtype], w.device.index, _stream(w)))
    return packed, scales, zeros


def _device_index() -> int:
    return torch.cuda.current_device()


def sm_count() -> int:
    v = _I()
    _raise(_lib.cbk_sm_count(_device_index(), ctypes.byref(v)))
    return v.value


def tile_n() -> int:
    return _lib.cbk_tile_n()


def max_rho(bits, kind="gemv") -> int:
    if kind not in _KIND:
        raise RuntimeError("kind must be 'gemv', 'qkv' or 'gate_up'")
    v = _I()
    _raise(_lib.cbk_max_rho(_device_index(), int(bits), _KIND[kind], ctypes.byref(v)))
    return v.value


PLAN_FAMILIES = {1: "stream", 2: "bstream", 3: "mfma", 4: "generic"}


def decode_plan(dtype, batch, in_features, group_size, out_features, bits, kind, split_k, rho):
    """Additive policy query: the launch a decode call would make, as a tuple (kernel family,
    K splits, workgroups, threads per workgroup, LDS bytes, launches per call).
    ``out_features`` / ``bits`` are one value, or (q, k, v) tuples for kind "qkv"."""
    if kind not in _KIND:
        raise RuntimeError("kind must be 'gemv', 'qkv' or 'gate_up'")
    ns = tuple(int(n) for n in out_features) if isinstance(out_features, (tuple, list)) else (int(out_features),) * 3
    bs = tuple(int(b) for b in bits) if isinstance(bits, (tuple, list)) else (int(bits),) * 3
    out = (ctypes.c_int32 * 6)()
    _raise(_lib.cbk_decode_plan(_DT[dtype], int(batch), int(in_features), int(group_size), *ns, *bs, _KIND[kind],
                                int(split_k), int(rho), _device_index(), out))
    return (PLAN_FAMILIES.get(out[0], "?"),) + tuple(out[1:])


def timer_start(capacity: int = 4096):
    """Arm the library's per-launch kernel timer (measurement hook, see cbk_timer_start)."""
    _raise(_lib.cbk_timer_start(int(capacity)))


def timer_stop():
    """Disarm the timer; returns (total_ms, per-launch durations in ms)."""
    total, n = ctypes.c_double(), _I()
    cap = 1 << 16
    buf = (ctypes.c_double * cap)()
    _raise(_lib.cbk_timer_stop(ctypes.byref(total), ctypes.byref(n), buf, cap))
    return total.value, list(buf[:min(n.value, cap)])
