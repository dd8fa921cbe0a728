"""On-disk packed dict -> device PackedLinearWeight (Kernel/crispybits_kernels/io.py:5-15).

Besides the kernels' own chunked layout (reference.py:37-55, ceil(K/32)*bits words per row)
this accepts the continuous bitstream that the paper's checkpoint packer writes
(quantization/crispybits_quant/packing.py:24-25, ceil(K*bits/32) words per row) and pads its
rows to the chunked length (code k sits at bit k*bits in both); the two coincide when
K % 32 == 0.
"""
import math

import torch

from .ops import PackedLinearWeight


def chunked_packed(packed: torch.Tensor, bits: int, in_features: int) -> torch.Tensor:
    """The kernels' layout of a packed tensor in either on-disk layout (by its row length)."""
    W = packed.shape[1]
    chunked = math.ceil(in_features / 32) * bits
    if W == chunked:
        return packed
    if W == (in_features * bits + 31) // 32:
        from .reference import continuous_to_chunked
        return continuous_to_chunked(packed, bits, in_features)
    raise ValueError(f"packed has {W} words per row; W{bits} with in_features={in_features} needs "
                     f"{chunked} (chunked) or {(in_features * bits + 31) // 32} (continuous)")


def from_packed_dict(d: dict, device="cuda", dtype=torch.float16) -> PackedLinearWeight:
    bias = d.get("bias")
    bits, K = int(d["bits"]), int(d["in_features"])
    return PackedLinearWeight(
        packed=chunked_packed(d["packed"], bits, K).to(device=device, dtype=torch.int32).contiguous(),
        scales=d["scales"].to(device=device, dtype=dtype).contiguous(),
        zeros=d["zeros"].to(device=device, dtype=dtype).contiguous(),
        bits=bits,
        group_size=int(d["group_size"]),
        in_features=K,
        out_features=int(d["out_features"]),
        bias=None if bias is None else bias.to(device=device, dtype=dtype).contiguous(),
    )
