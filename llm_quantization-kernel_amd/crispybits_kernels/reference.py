"""Offline quantizer / packer of the packed-linear format (torch, any device).

Produces the weights the kernels consume -- the reference's
Kernel/crispybits_kernels/reference.py:10-94 interface (quantize_affine,
dequantize, pack_codes, unpack_codes, pack_linear_dict, dequantized_weight,
write_packed_dir) -- and the paper's checkpoint format of
quantization/crispybits_quant (affine_quantize_weight, pack_codes_continuous,
pack_block, write_checkpoint_dir; pack_checkpoint.py).  This is the format's
producer, used when preparing a model; it is never called by the op path
(ops.py), which runs only the HIP kernels.

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


def affine_quantize_weight(w: torch.Tensor, bits: int, group_size: int = 128, eps: float = 1e-8):
    """The paper quantizer of quantization/crispybits_quant/affine.py:28-71 (the producer
    behind its pack_checkpoint.py), vectorised: per group of real columns min <= 0 <= max,
    scale = (max - min) / qmax (1 where below eps), zero = clamp(round(-min / scale)),
    q = clamp(round(w / scale + zero)) -- the zero added before rounding.  fp32 throughout;
    returns (q int32 [N,K], scale fp32 [N,G], zero fp32 [N,G])."""
    assert bits in (2, 3, 4)
    N, K = w.shape
    G = math.ceil(K / group_size)
    wf = w.float()
    if G * group_size != K:        # pad with the row's last value: min/max over real columns unchanged
        wf = torch.cat([wf, wf[:, K - 1:K].expand(N, G * group_size - K)], dim=1)
    g = wf.reshape(N, G, group_size)
    qmax = float((1 << bits) - 1)
    lo, hi = g.amin(-1).clamp(max=0.0), g.amax(-1).clamp(min=0.0)
    scale = (hi - lo) / qmax
    scale = torch.where(scale < eps, torch.ones_like(scale), scale)
    zero = torch.round(-lo / scale).clamp(0, qmax)
    q = torch.round(g / scale[..., None] + zero[..., None]).clamp(0, qmax)
    return q.reshape(N, G * group_size)[:, :K].to(torch.int32), scale, zero


def pack_codes_continuous(q: torch.Tensor, bits: int) -> torch.Tensor:
    """Codes [N, K] -> int32 [N, ceil(K*bits/32)]: the unpadded row bitstream of
    crispybits_quant/packing.py:28-59 (equal to pack_codes when K % 32 == 0)."""
    assert bits in (2, 3, 4)
    N, K = q.shape
    W = (K * bits + 31) // 32
    out = torch.empty(N, W, dtype=torch.int32, device=q.device)
    shifts = torch.arange(bits, device=q.device, dtype=torch.int64)
    weights = torch.ones(32, dtype=torch.int64, device=q.device) << torch.arange(32, device=q.device)
    for r0 in range(0, N, _ROW_BLOCK):
        qb = q[r0:r0 + _ROW_BLOCK].to(torch.int64) & ((1 << bits) - 1)
        n = qb.shape[0]
        stream = ((qb.unsqueeze(-1) >> shifts) & 1).reshape(n, K * bits)       # bit i of code k at k*bits + i
        stream = torch.cat([stream, stream.new_zeros(n, W * 32 - K * bits)], dim=1)
        words = (stream.reshape(n, W, 32) * weights).sum(-1)
        out[r0:r0 + n] = torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32)
    return out


def unpack_codes_continuous(packed: torch.Tensor, K: int, bits: int) -> torch.Tensor:
    """int32 [N, ceil(K*bits/32)] -> codes int32 [N, K] (packing.py:62-80)."""
    N, W = packed.shape
    out = torch.empty(N, K, dtype=torch.int32, device=packed.device)
    bit = torch.arange(32, device=packed.device, dtype=torch.int64)
    weights = torch.ones(bits, dtype=torch.int64, device=packed.device) << torch.arange(bits, device=packed.device)
    for r0 in range(0, N, _ROW_BLOCK):
        wb = packed[r0:r0 + _ROW_BLOCK].to(torch.int64) & 0xFFFFFFFF
        n = wb.shape[0]
        stream = ((wb.unsqueeze(-1) >> bit) & 1).reshape(n, W * 32)[:, :K * bits]
        out[r0:r0 + n] = (stream.reshape(n, K, bits) * weights).sum(-1).to(torch.int32)
    return out


def continuous_to_chunked(packed: torch.Tensor, bits: int, K: int) -> torch.Tensor:
    """A continuous-bitstream weight (crispybits_quant/packing.py) in the kernels' format.
    Both put code k at bit k*bits of the row's bitstream and leave the bits past K*bits
    zero; the chunked rows are only longer (whole 32-code chunks), so the conversion is a
    zero pad of each row to ceil(K/32)*bits words."""
    chunked = math.ceil(K / 32) * bits
    p = packed.to(torch.int32)
    if p.shape[1] < chunked:
        p = torch.nn.functional.pad(p, (0, chunked - p.shape[1]))
    return p.contiguous()


SCHEMES = ("kernel", "affine")


def quantize_pack(weight: torch.Tensor, bits: int, group_size: int = 128, dtype=torch.float16,
                  scheme: str = "kernel"):
    """(packed, scales, zeros) of one weight on its own device, in the kernels' chunked
    format.  ``scheme`` "kernel" is this module's quantize_affine (reference.py:10-27);
    "affine" is the paper quantizer (affine_quantize_weight).  A CUDA weight is quantized
    and packed by the HIP producer (``_C.quantize_pack``), bit-identical to the CPU path --
    torch's own GPU division by a scalar is a multiply by the reciprocal, which moves some
    scales by an ulp and with them some codes."""
    if scheme not in SCHEMES:
        raise ValueError(f"scheme must be one of {SCHEMES}")
    if weight.is_cuda:
        from . import _C
        return _C.quantize_pack(weight.detach(), bits, group_size, dtype, scheme=SCHEMES.index(scheme))
    quant = quantize_affine if scheme == "kernel" else affine_quantize_weight
    q, s, z = quant(weight, bits, group_size)
    return pack_codes(q, bits), s.to(dtype), z.to(dtype)


def pack_linear_dict(weight: torch.Tensor, bits: int, group_size: int = 128,
                     bias: Optional[torch.Tensor] = None, dtype=torch.float16, scheme: str = "kernel") -> Dict:
    """One linear -> the on-disk dict (packed/scales/zeros/bits/group_size/in/out/bias)."""
    packed, s, z = quantize_pack(weight, bits, group_size, dtype, scheme)
    return dict(packed=packed.cpu(), scales=s.cpu(), zeros=z.cpu(),
                bits=bits, group_size=group_size, in_features=weight.shape[1], out_features=weight.shape[0],
                bias=None if bias is None else bias.detach().to(dtype).cpu())


def dequantized_weight(d: Dict) -> torch.Tensor:
    q = unpack_codes(d["packed"], d["bits"], d["in_features"])
    return dequantize(q, d["scales"], d["zeros"], d["group_size"])


def write_packed_dir(model: torch.nn.Module, out_dir: str, bits_options: Iterable[int] = (2, 3, 4),
                     group_size: int = 128, dtype=torch.float16, bitmap: Optional[Iterable[int]] = None) -> None:
    """block_{i:03d}_w{b}.pt per block and width: {linear name: packed dict}.  With ``bitmap``
    (additive) block i is written at width bitmap[i] only, the files install_bitmap reads for
    that bitmap."""
    from .integration import _blocks
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    widths = None if bitmap is None else [int(b) for b in bitmap]
    for i, block in enumerate(_blocks(model)):
        linears = {n: m for n, m in block.named_modules() if isinstance(m, torch.nn.Linear)}
        for b in (bits_options if widths is None else (widths[i],)):
            data = {n: pack_linear_dict(m.weight.detach(), b, group_size, m.bias, dtype) for n, m in linears.items()}
            torch.save(data, out / f"block_{i:03d}_w{b}.pt")


def pack_block(block: torch.nn.Module, bits: int, group_size: int = 128) -> Dict:
    """The paper's per-block checkpoint dict (crispybits_quant/model_utils.py:54-70): every
    nn.Linear of the block by its dotted name, quantized by affine_quantize_weight, packed
    as the continuous bitstream, scales and zeros in the weight's dtype.  CUDA weights are
    quantized by the HIP producer (scheme "affine") and re-laid out as the continuous
    bitstream, bit-identical to the CPU path."""
    out = {}
    for name, m in block.named_modules():
        if not isinstance(m, torch.nn.Linear):
            continue
        w = m.weight.detach()
        N, K = w.shape
        packed, s, z = quantize_pack(w, bits, group_size, w.dtype, scheme="affine")
        if K % 32:
            packed = pack_codes_continuous(unpack_codes(packed, bits, K), bits)
        out[name] = dict(packed=packed.cpu(), scales=s.cpu(), zeros=z.cpu(), bits=bits, group_size=group_size,
                         out_features=N, in_features=K,
                         bias=None if m.bias is None else m.bias.detach().cpu())
    return out


def write_checkpoint_dir(model: torch.nn.Module, out_dir: str, bitmap, group_size: int = 128,
                         model_name: str = "") -> None:
    """pack_checkpoint.py:19-29: block_{i:03d}.pt (one width per block, pack_block) and
    manifest.json {model, group_size, bitmap, blocks}.  install_bitmap reads this layout."""
    import json
    from .integration import _blocks
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    blocks = _blocks(model)
    if len(blocks) != len(bitmap):
        raise ValueError("bitmap length does not match model")
    manifest = {"model": model_name, "group_size": group_size, "bitmap": [int(b) for b in bitmap], "blocks": []}
    for i, (block, bits) in enumerate(zip(blocks, bitmap)):
        torch.save(pack_block(block, int(bits), group_size), out / f"block_{i:03d}.pt")
        manifest["blocks"].append(f"block_{i:03d}.pt")
    with open(out / "manifest.json", "w") as f:
        json.dump(manifest, f, indent=2)

