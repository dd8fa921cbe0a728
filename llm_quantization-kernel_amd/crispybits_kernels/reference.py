"""Offline quantizer / packer of the packed-linear format (torch, any device).

Produces the weights the kernels consume -- the reference's
Kernel/crispybits_kernels/reference.py:10-94 interface (quantize_affine,
dequantize, pack_codes, unpack_codes, pack_linear_dict, dequantized_weight,
write_packed_dir).  This is the format's producer, used when preparing a model;
it is never called by the op path (ops.py), which runs only the HIP kernels.

The quantizer formula is the format definition and follows reference.py:10-27
step for step (fp32, round-half-even, clamp); the bit packing is vectorised over
bit planes: a chunk's 32 codes are expanded to their 32*bits LSB-first bits, which
regrouped 32 at a time are exactly the chunk's ``bits`` words.  For a CUDA weight,
``quantize_pack`` / ``pack_linear_dict`` run the HIP producer instead (quant.hip).
"""
from __future__ import annotations

import math
from pathlib import Path
from typing import Dict, Iterable, Optional

import torch

_ROW_BLOCK = 256        # rows per vectorised block (bounds the bit-plane temporaries)


def quantize_affine(w: torch.Tensor, bits: int, group_size: int = 128):
    """Group-wise asymmetric min/max quantization -> (q int32 [N,K], scale fp32 [N,G], zero fp32 [N,G])."""
    assert bits in (2, 3, 4)
    N, K = w.shape
    G = math.ceil(K / group_size)
    wf = w.float()
    if G * group_size != K:
        wf = torch.cat([wf, wf[:, K - 1:K].expand(N, G * group_size - K)], dim=1)
    g = wf.reshape(N, G, group_size)
    qmax = float((1 << bits) - 1)
    lo, hi = g.amin(-1), g.amax(-1)
    scale = ((hi - lo) / qmax).clamp_min(1e-8)
    zero = torch.round(-lo / scale).clamp(0, qmax)
    q = torch.clamp(torch.round(g / scale[..., None]) + zero[..., None], 0, qmax)
    return q.reshape(N, G * group_size)[:, :K].to(torch.int32), scale, zero


def dequantize(q: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, group_size: int) -> torch.Tensor:
    """fp32 (q - z) * s with per-group metadata."""
    K = q.shape[1]
    gidx = torch.arange(K, device=q.device) // group_size
    return (q.float() - zeros.float()[:, gidx]) * scales.float()[:, gidx]


def pack_codes(q: torch.Tensor, bits: int) -> torch.Tensor:
    """Codes [N, K] -> int32 [N, ceil(K/32)*bits]: per row an LSB-first bitstream,
    rows padded to whole 32-code chunks."""
    assert bits in (2, 3, 4)
    N, K = q.shape
    C = math.ceil(K / 32)
    out = torch.empty(N, C * bits, dtype=torch.int32, device=q.device)
    shifts = torch.arange(bits, device=q.device, dtype=torch.int64)
    weights = torch.ones(32, dtype=torch.int64, device=q.device) << torch.arange(32, device=q.device)
    for r0 in range(0, N, _ROW_BLOCK):
        qb = q[r0:r0 + _ROW_BLOCK].to(torch.int64) & ((1 << bits) - 1)
        n = qb.shape[0]
        if C * 32 != K:
            qb = torch.cat([qb, qb.new_zeros(n, C * 32 - K)], dim=1)
        planes = (qb.view(n, C, 32, 1) >> shifts) & 1                 # bit i of code j at j*bits + i
        words = (planes.reshape(n, C, bits, 32) * weights).sum(-1)     # 32 consecutive bits per word
        words = torch.where(words >= 2 ** 31, words - 2 ** 32, words)
        out[r0:r0 + n] = words.reshape(n, C * bits).to(torch.int32)
    return out


def unpack_codes(packed: torch.Tensor, bits: int, K: int) -> torch.Tensor:
    """int32 [N, ceil(K/32)*bits] -> codes int32 [N, K]."""
    N, W = packed.shape
    C = W // bits
    out = torch.empty(N, K, dtype=torch.int32, device=packed.device)
    bit = torch.arange(32, device=packed.device, dtype=torch.int64)
    weights = torch.ones(bits, dtype=torch.int64, device=packed.device) << torch.arange(bits, device=packed.device)
    for r0 in range(0, N, _ROW_BLOCK):
        wb = packed[r0:r0 + _ROW_BLOCK].to(torch.int64) & 0xFFFFFFFF
        n = wb.shape[0]
        planes = (wb.view(n, C * bits, 1) >> bit) & 1                  # row bitstream, LSB first
        codes = (planes.reshape(n, C * 32, bits) * weights).sum(-1)
        out[r0:r0 + n] = codes[:, :K].to(torch.int32)
    return out


def quantize_pack(weight: torch.Tensor, bits: int, group_size: int = 128, dtype=torch.float16):
    """(packed, scales, zeros) of one weight on its own device.  A CUDA weight is
    quantized and packed by the HIP producer (``_C.quantize_pack``), bit-identical to
    this module's CPU path -- torch's own GPU division by a scalar is a multiply by the
    reciprocal, which moves some scales by an ulp and with them some codes."""
    if weight.is_cuda:
        from . import _C
        return _C.quantize_pack(weight.detach(), bits, group_size, dtype)
    q, s, z = quantize_affine(weight, bits, group_size)
    return pack_codes(q, bits), s.to(dtype), z.to(dtype)


def pack_linear_dict(weight: torch.Tensor, bits: int, group_size: int = 128,
                     bias: Optional[torch.Tensor] = None, dtype=torch.float16) -> Dict:
    """One linear -> the on-disk dict (packed/scales/zeros/bits/group_size/in/out/bias)."""
    packed, s, z = quantize_pack(weight, bits, group_size, dtype)
    return dict(packed=packed.cpu(), scales=s.cpu(), zeros=z.cpu(),
                bits=bits, group_size=group_size, in_features=weight.shape[1], out_features=weight.shape[0],
                bias=None if bias is None else bias.detach().to(dtype).cpu())


def dequantized_weight(d: Dict) -> torch.Tensor:
    q = unpack_codes(d["packed"], d["bits"], d["in_features"])
    return dequantize(q, d["scales"], d["zeros"], d["group_size"])


def write_packed_dir(model: torch.nn.Module, out_dir: str, bits_options: Iterable[int] = (2, 3, 4),
                     group_size: int = 128, dtype=torch.float16) -> None:
    """block_{i:03d}_w{b}.pt per block and width: {linear name: packed dict}."""
    from .integration import _blocks
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    for i, block in enumerate(_blocks(model)):
        linears = {n: m for n, m in block.named_modules() if isinstance(m, torch.nn.Linear)}
        for b in bits_options:
            data = {n: pack_linear_dict(m.weight.detach(), b, group_size, m.bias, dtype) for n, m in linears.items()}
            torch.save(data, out / f"block_{i:03d}_w{b}.pt")
