"""On-disk packed dict -> device PackedLinearWeight (Kernel/crispybits_kernels/io.py:5-15)."""
import torch

from .ops import PackedLinearWeight


def from_packed_dict(d: dict, device="cuda", dtype=torch.float16) -> PackedLinearWeight:
    bias = d.get("bias")
    return PackedLinearWeight(
        packed=d["packed"].to(device=device, dtype=torch.int32).contiguous(),
        scales=d["scales"].to(device=device, dtype=dtype).contiguous(),
        zeros=d["zeros"].to(device=device, dtype=dtype).contiguous(),
        bits=int(d["bits"]),
        group_size=int(d["group_size"]),
        in_features=int(d["in_features"]),
        out_features=int(d["out_features"]),
        bias=None if bias is None else bias.to(device=device, dtype=dtype).contiguous(),
    )
