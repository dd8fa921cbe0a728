"""CPU emulation of the packed-linear kernels -- TEST INFRASTRUCTURE ONLY.

Restates /root/reference/Crispybits/Kernel/crispybits_kernels/emulator.py:15-144 with
numpy cores computed in float64 (a stricter checker than the reference's fp32
einsum; parity with the HIP kernels is tolerance-based, see the tests).

The module exposes the HIP backend's function names and argument order
(packed_gemv, packed_gemm, fused_gate_up, fused_qkv, sm_count, tile_n, max_rho, and
packed_gemm_gate_up),
taking and returning torch CPU tensors, so tests can inject it with
``crispybits_kernels.ops.set_backend(oracle.emulator)`` to exercise the host
logic of ops.py / integration.py without a GPU.  Product code never imports it.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import reference as R
from .reference import unpack_codes

IS_EMULATOR = True
# Device constants of the MI355X build this oracle stands in for.
SM_COUNT = 256          # CUs on one MI355X
TILE_N = 16             # virtual rows per decode job tile of the HIP GEMV
MAX_RHO = 8


def sm_count():
    return SM_COUNT


def tile_n():
    return TILE_N


def max_rho(bits, kind="gemv"):
    if kind not in ("gemv", "qkv", "gate_up"):
        raise RuntimeError("kind must be 'gemv', 'qkv' or 'gate_up'")
    return MAX_RHO


def decode_plan(dtype, batch, in_features, group_size, out_features, bits, kind, split_k, rho):
    """Launch-plan query of the HIP backend (its ``decode_plan``), for the host logic of the
    tuner on the CPU: one job per 16 virtual rows and K split, splits clamped to the 32-code
    chunks, rho ignored (as the streaming kernels ignore it)."""
    if kind not in ("gemv", "qkv", "gate_up"):
        raise RuntimeError("kind must be 'gemv', 'qkv' or 'gate_up'")
    ns = out_features if isinstance(out_features, (tuple, list)) else (out_features,)
    v = sum(ns) if kind == "qkv" else (2 * ns[0] if kind == "gate_up" else ns[0])
    P = max(1, min(int(split_k), math.ceil(in_features / 32)))
    return ("stream", P, math.ceil(v / TILE_N) * P, 256, 0, 2 if P > 1 else 1)


# ----------------------------------------------------------------------------- numpy cores

def silu64(v: np.ndarray) -> np.ndarray:
    """v * sigmoid(v) in float64 (common.cuh:15-19 SiLU), evaluated without overflow:
    e = exp(-|v|) <= 1, sigmoid(v) = 1 / (1 + e) for v >= 0 and e / (1 + e) for v < 0."""
    v = np.asarray(v, dtype=np.float64)
    e = np.exp(-np.abs(v))
    return v * np.where(v >= 0, 1.0 / (1.0 + e), e / (1.0 + e))


def act64(v: np.ndarray, act: int) -> np.ndarray:
    if act == 1:
        return np.maximum(v, 0.0)
    if act == 2:
        return silu64(v)
    return v


def dequant64(packed: np.ndarray, scales: np.ndarray, zeros: np.ndarray, bits: int, K: int,
              gs: int) -> np.ndarray:
    """float64 W-hat = (q - z) * s; metadata already rounded to the storage dtype."""
    q = unpack_codes(packed, bits, K).astype(np.float64)
    g = np.arange(K) // gs
    return (q - zeros.astype(np.float64)[:, g]) * scales.astype(np.float64)[:, g]


def dequant64_fast(packed: np.ndarray, scales: np.ndarray, zeros: np.ndarray, bits: int, K: int,
                   gs: int) -> np.ndarray:
    """dequant64 through unpack_codes_by_slot and per-group broadcasting on the host cores
    (torch float64, no repeated metadata arrays); the same float64 values
    (tests/test_oracle_format.py)."""
    q = torch.from_numpy(np.ascontiguousarray(R.unpack_codes_by_slot(packed, bits, K)))
    N = q.shape[0]
    G = scales.shape[1]
    s = torch.from_numpy(np.asarray(scales, dtype=np.float64))
    z = torch.from_numpy(np.asarray(zeros, dtype=np.float64))
    if K == G * gs:
        W = q.view(N, G, gs).to(torch.float64)
        W.sub_(z[:, :, None]).mul_(s[:, :, None])
        return W.view(N, K).numpy()
    g = torch.arange(K) // gs
    return ((q.to(torch.float64) - z[:, g]) * s[:, g]).numpy()


def split_bounds(C: int, split_k: int):
    """Chunk range of split s: [floor(C*s/P), floor(C*(s+1)/P)) (packed_gemv.cu:94-95)."""
    P = max(1, min(int(split_k), C))
    return [((C * s) // P, (C * (s + 1)) // P) for s in range(P)]


def gemv_partials64(x: np.ndarray, packed, scales, zeros, bits, K, gs, split_k) -> np.ndarray:
    """[P, B, V] float64 partial sums over the K splits (emulator.py:48-67)."""
    W = dequant64(packed, scales, zeros, bits, K, gs)
    C = math.ceil(K / 32)
    parts = []
    for c0, c1 in split_bounds(C, split_k):
        k0, k1 = c0 * 32, min(c1 * 32, K)
        parts.append(x[:, k0:k1] @ W[:, k0:k1].T)
    return np.stack(parts)


def unperm_index(n: int, hd: int) -> np.ndarray:
    """Stored row r -> original row (common.cuh:66-70, emulator.py:96-101)."""
    r = np.arange(n)
    if hd <= 0:
        return r
    head, p = r // hd, r % hd
    return head * hd + np.where(p % 2 == 1, p // 2 + hd // 2, p // 2)


# ----------------------------------------------------------------------------- torch adapters

def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().to(torch.float64).numpy()


def _out(a: np.ndarray, like: torch.Tensor) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(device=like.device, dtype=like.dtype)


def _check(x, packed, scales, zeros, bits, K, gs, name):
    assert x.dim() == 2 and x.shape[1] == K and x.is_contiguous(), f"{name}: bad x"
    assert x.dtype in (torch.float16, torch.bfloat16, torch.float32), f"{name}: x dtype"
    assert packed.dtype == torch.int32 and packed.is_contiguous(), f"{name}: packed must be contiguous int32"
    assert bits in (2, 3, 4), f"{name}: bits"
    assert gs > 0 and gs % 32 == 0, f"{name}: group_size must be a positive multiple of 32"
    assert packed.shape[1] == math.ceil(K / 32) * bits, f"{name}: packed row must be ceil(K/32)*bits words"
    assert scales.shape == zeros.shape and scales.shape[0] == packed.shape[0], f"{name}: metadata shape"
    assert scales.shape[1] == math.ceil(K / gs), f"{name}: groups"
    assert scales.dtype == x.dtype and zeros.dtype == x.dtype, f"{name}: metadata dtype must match x"


def _check_ws(ws):
    if ws is not None and ws.numel() >= 2:
        assert ws.dtype == torch.int32
        assert ws[:2].tolist() == [0, 0], "workspace not reset (was it shared across streams?)"


def _bias64(b, n):
    if b is None or b.numel() == 0:
        return np.zeros(n)
    assert b.numel() == n, "bias length must equal out_features"
    return _np(b)


def _partials(x, rows, s, z, bits, K, gs, split_k):
    return gemv_partials64(_np(x), rows.cpu().numpy(), _np(s), _np(z), bits, K, gs, split_k)


def packed_gemv(x, packed, scales, zeros, bias, bits, K, gs, split_k, rho, act, ws):
    _check(x, packed, scales, zeros, bits, K, gs, "packed_gemv"); _check_ws(ws)
    acc = _partials(x, packed, scales, zeros, bits, K, gs, split_k).sum(0)
    return _out(act64(acc + _bias64(bias, packed.shape[0])[None], int(act)), x)


def fused_gate_up(x, wg, sg, zg, wu, su, zu, bits, K, gs, split_k, rho, ws):
    _check(x, wg, sg, zg, bits, K, gs, "gate"); _check(x, wu, su, zu, bits, K, gs, "up"); _check_ws(ws)
    assert wg.shape == wu.shape
    g = _partials(x, wg, sg, zg, bits, K, gs, split_k).sum(0)
    u = _partials(x, wu, su, zu, bits, K, gs, split_k).sum(0)
    return _out(silu64(g) * u, x)


def fused_qkv(x, wq, sq, zq, bq, wk, sk, zk, bk, wv, sv, zv, bv, rope_cos, rope_sin, head_dim, perm_hd,
              bits, K, gs, split_k, rho, ws):
    ws_bits = bits if isinstance(bits, (tuple, list)) else (bits, bits, bits)
    for w, s, z, n, b in ((wq, sq, zq, "q", ws_bits[0]), (wk, sk, zk, "k", ws_bits[1]),
                          (wv, sv, zv, "v", ws_bits[2])):
        _check(x, w, s, z, b, K, gs, n)
    _check_ws(ws)
    rope = rope_cos is not None and rope_cos.numel() > 0
    if perm_hd > 0:
        assert perm_hd % 2 == 0 and wq.shape[0] % perm_hd == 0 and wk.shape[0] % perm_hd == 0
    if rope:
        assert perm_hd > 0 and perm_hd == head_dim, "fused RoPE needs pair-interleaved Q/K"
        assert rope_cos.numel() == x.shape[0] * head_dim
        cos, sin = _np(rope_cos).reshape(x.shape[0], head_dim), _np(rope_sin).reshape(x.shape[0], head_dim)
    outs = []
    for i, (w, s, z, b) in enumerate(((wq, sq, zq, bq), (wk, sk, zk, bk), (wv, sv, zv, bv))):
        n = w.shape[0]
        y = _partials(x, w, s, z, ws_bits[i], K, gs, split_k).sum(0) + _bias64(b, n)[None]
        hd = perm_hd if i < 2 else 0
        orig = unperm_index(n, hd)
        if rope and i < 2:
            partner = y[:, np.arange(n) ^ 1]
            d = orig % head_dim
            c, sn = cos[:, d], sin[:, d]
            y = np.where(d[None] < head_dim // 2, y * c - partner * sn, y * c + partner * sn)
        out = np.empty_like(y)
        out[:, orig] = y
        outs.append(_out(out, x))
    return outs


def rope64(y: np.ndarray, cos: np.ndarray, sin: np.ndarray, head_dim: int) -> np.ndarray:
    """HF rotate-half RoPE in float64 on un-permuted outputs y [M, H*head_dim] with cos/sin
    [M, head_dim], one row per x row (apply_rope_reference, Kernel/crispybits_kernels/
    ops.py:224-231; the fused epilogue's rotation, packed_gemv.cu:69-79)."""
    M, W = y.shape
    t = y.reshape(M, W // head_dim, head_dim)
    h = head_dim // 2
    rot = np.concatenate([-t[..., h:], t[..., :h]], axis=-1)
    return (t * cos[:, None, :] + rot * sin[:, None, :]).reshape(M, W)


def round_to(a: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """Round a float64 array once to ``dtype`` and back (RN-even)."""
    return torch.from_numpy(a).to(dtype).to(torch.float64).numpy()


def gemm_weight64(packed, scales, zeros, bits, K, gs, dtype, use_tensor_cores):
    """W-hat of the prefill GEMM (packed_gemm.cu:56,143; emulator.py:141-142).

    With the matrix-core path W-hat is RN_T((q - z) * s); the product is exact in
    float64 (an integer in [-15, 15] times a 16-bit float), so rounding it once
    to T equals the reference's RN_T(fp32 product).
    """
    W = dequant64(packed, scales, zeros, bits, K, gs)
    if use_tensor_cores and dtype in (torch.float16, torch.bfloat16):
        W = round_to(W, dtype)
    return W


def packed_gemm(x, packed, scales, zeros, bias, bits, K, gs, act, use_tensor_cores):
    _check(x, packed, scales, zeros, bits, K, gs, "packed_gemm")
    W = gemm_weight64(packed.cpu().numpy(), _np(scales), _np(zeros), bits, K, gs, x.dtype, use_tensor_cores)
    y = _np(x) @ W.T + _bias64(bias, packed.shape[0])[None]
    return _out(act64(y, int(act)), x)


def packed_gemm_gate_up(x, wg, sg, zg, wu, su, zu, bits, K, gs):
    """The reference's prefill gate-up (ops.py:216-220): the gate GEMM with SiLU and the up
    GEMM, each stored in x's dtype, multiplied in that dtype."""
    assert wg.shape == wu.shape
    g = packed_gemm(x, wg, sg, zg, None, bits, K, gs, 2, True)
    u = packed_gemm(x, wu, su, zu, None, bits, K, gs, 0, True)
    return g * u
