"""Host op API of the packed W2/W3/W4 linears on MI355X (gfx950).

The public surface is the reference's (Kernel/crispybits_kernels/ops.py:1-321): the
weight record ``PackedLinearWeight``, the module ``PackedLinear``, the ops
``packed_linear`` / ``fused_qkv`` / ``fused_gate_up``, the RoPE row-order helpers, the
split-K rule and the device queries, with the same arguments and the same ValueError /
RuntimeError behaviour.  How they run is this build's own:

* **Call routing.**  A call is decode (the streaming GEMV kernels) when its flattened
  batch has at most ``decode_threshold`` rows, else prefill (the MFMA GEMM).  The K split
  of a decode call is the caller's request, or with ``split_k=None`` the policy's
  (``policy_split_k``: no split, retuned for MI355X -- see ``POLICY_SPLIT_K``).
* **RoPE layout.**  ``rope_row_order`` / ``rope_inverse_order`` are closed forms (stored
  row 2i of a head is original row i, stored row 2i+1 is original row i + head_dim/2).
  The prefill fallback of ``fused_qkv`` rotates the projection while it is still in the
  stored, pair-interleaved order -- a stored pair is (y_d, y_{d+h}), one complex number
  of the rotation -- and restores the original column order with one reshape-transpose
  (``_original_columns``) instead of an index gather.
* **Modules** keep their ``PackedLinearWeight`` cached and rebuild it when a buffer is
  replaced (``.to()``, ``permute_for_rope_``).

Retuned or additive, relative to the reference:
  * ``DECODE_THRESHOLD = 16``: the batched streaming GEMV reads each weight once for up
    to 16 batch rows, 3-4x faster than the prefill GEMM's 128-row tiles at M = 9..16
    (the reference uses 4, ops.py:23).
  * ``fused_qkv`` takes per-projection widths (the reference raises ValueError,
    ops.py:240-241); the kernel dispatches the width per workgroup.
  * The split-K rule counts decode jobs per ``BATCH_TILE`` batch rows, and the policy a
    ``split_k=None`` call takes requests no split (``POLICY_SPLIT_K``, measured at 256 CUs).
  * ``set_backend`` takes "cuda" (alias "hip") or a module object with the ``_C``
    functions -- the hook the CPU tests use to inject the oracle.  No emulator ships in
    the product: ``set_backend("emulator")`` raises RuntimeError.
"""
from __future__ import annotations

import os
import warnings
from dataclasses import dataclass, replace
from functools import lru_cache
from typing import Optional, Tuple

import torch
import torch.nn as nn

try:
    from . import _C as _CUDA
    _IMPORT_ERROR = None
except Exception as e:  # pragma: no cover - reported by _check_ext
    _CUDA = None
    _IMPORT_ERROR = e

_C = _CUDA
if os.environ.get("CRISPYBITS_BACKEND", "").lower() == "emulator":
    warnings.warn("CRISPYBITS_BACKEND=emulator: no CPU emulator ships with the MI355X build; using the HIP kernels")

DECODE_THRESHOLD = 16
ACT = {"none": 0, None: 0, "relu": 1, "silu": 2}
KINDS = ("gemv", "qkv", "gate_up")
BATCH_TILE = 16          # batch rows of one decode job


# ----------------------------------------------------------------------------- backend

def set_backend(name):
    """"cuda" / "hip": the gfx950 library.  A module object: its ``packed_gemv`` /
    ``packed_gemm`` / ``fused_*`` / ``sm_count`` / ``tile_n`` / ``max_rho`` serve every op
    (the tests pass the CPU oracle this way)."""
    global _C
    if not isinstance(name, str):
        _C = name
    elif name in ("cuda", "hip"):
        _C = _CUDA
    elif name == "emulator":
        raise RuntimeError("the CPU emulator is test infrastructure (oracle.emulator); "
                           "pass the module object to set_backend to use it")
    else:
        raise ValueError(name)
    for cached in (tile_n, _sm_count_for):
        cached.cache_clear()


def backend_name() -> str:
    return "emulator" if getattr(_C, "IS_EMULATOR", False) else "cuda"


def _check_ext():
    if _C is None:
        raise RuntimeError(f"crispybits HIP library is not built: {_IMPORT_ERROR}")


# ----------------------------------------------------------------------------- weights

@dataclass
class PackedLinearWeight:
    """One packed linear: int32 codes [N, ceil(K/32)*bits], scales and zeros
    [N, ceil(K/group_size)] in the activation dtype, optional bias [N], and the head_dim
    its rows are stored pair-interleaved with (0 when in original order)."""
    packed: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor
    bits: int
    group_size: int
    in_features: int
    out_features: int
    bias: Optional[torch.Tensor] = None
    rope_perm_head_dim: int = 0

    def cuda(self, device=None, dtype=torch.float16):
        """A copy on ``device`` (default: the current GPU) with int32 codes and metadata
        and bias in ``dtype``, every tensor contiguous."""
        dev = torch.device(device if device is not None else "cuda")

        def moved(t, dt):
            return None if t is None else t.to(device=dev, dtype=dt).contiguous()

        return replace(self, packed=moved(self.packed, torch.int32), scales=moved(self.scales, dtype),
                       zeros=moved(self.zeros, dtype), bias=moved(self.bias, dtype))


def new_workspace(device) -> torch.Tensor:
    """The reference's per-module int32[2] job-queue words.  The HIP kernels assign jobs
    statically, accept it and never write it, so it stays [0, 0]."""
    return torch.zeros(2, dtype=torch.int32, device=device)


# ----------------------------------------------------------------------------- RoPE layout

def _check_heads(out_features: int, head_dim: int):
    if head_dim % 2 or out_features % head_dim:
        raise ValueError("out_features must be a multiple of an even head_dim")


def rope_row_order(out_features: int, head_dim: int, device=None) -> torch.Tensor:
    """Stored row p <- original row order[p]: within a head, stored 2i holds original i and
    stored 2i+1 holds original i + head_dim/2 (each rotate-half pair side by side)."""
    _check_heads(out_features, head_dim)
    p = torch.arange(out_features)
    within = p % head_dim
    return (p - within + (within >> 1) + (within & 1) * (head_dim // 2)).to(device)


def rope_inverse_order(out_features: int, head_dim: int, device=None) -> torch.Tensor:
    """Original row o -> its stored row: 2d for the first half of a head, 2(d - h) + 1 for
    the second (d = o mod head_dim, h = head_dim / 2)."""
    _check_heads(out_features, head_dim)
    o = torch.arange(out_features)
    d = o % head_dim
    h = head_dim // 2
    return (o - d + torch.where(d < h, 2 * d, 2 * (d - h) + 1)).to(device)


def permute_for_rope(w: PackedLinearWeight, head_dim: int) -> PackedLinearWeight:
    """The weight with its rows stored pair-interleaved for ``head_dim`` (what the fused
    RoPE epilogue needs: a row's rotate-half partner is the adjacent row)."""
    if w.rope_perm_head_dim:
        if w.rope_perm_head_dim != head_dim:
            raise ValueError("weight already permuted with a different head_dim")
        return w
    order = rope_row_order(w.out_features, head_dim, w.packed.device)

    def rows(t):
        return None if t is None else t.index_select(0, order).contiguous()

    return replace(w, packed=rows(w.packed), scales=rows(w.scales), zeros=rows(w.zeros), bias=rows(w.bias),
                   rope_perm_head_dim=head_dim)


def _original_columns(y: torch.Tensor, head_dim: int) -> torch.Tensor:
    """Columns of y [M, n] in stored (pair-interleaved) order -> original order: per head,
    the stored [h, 2] pairs transposed to [2, h]."""
    M, n = y.shape
    return y.view(M, n // head_dim, head_dim // 2, 2).transpose(-1, -2).reshape(M, n)


def _unpermute_cols(y: torch.Tensor, w: PackedLinearWeight) -> torch.Tensor:
    """Kernel-order outputs of a permuted weight -> original column order."""
    return _original_columns(y, w.rope_perm_head_dim) if w.rope_perm_head_dim else y


def apply_rope_reference(t: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, head_dim: int) -> torch.Tensor:
    """HF rotate-half RoPE of t [M, H*head_dim] (original column order) with cos/sin
    [M, head_dim], computed in fp32 and rounded once to t's dtype."""
    M, W = t.shape
    h = head_dim // 2
    halves = t.float().reshape(M, W // head_dim, 2, h)
    a, b = halves[:, :, 0], halves[:, :, 1]
    c = cos.float().reshape(M, 1, 2, h)
    s = sin.float().reshape(M, 1, 2, h)
    out = torch.stack((a * c[:, :, 0] - b * s[:, :, 0], b * c[:, :, 1] + a * s[:, :, 1]), dim=2)
    return out.view(M, W).to(t.dtype)


def _rope_stored(y: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, head_dim: int) -> torch.Tensor:
    """RoPE of a pair-interleaved projection y [M, n] (stored order), returned in the original
    column order: the same fp32 arithmetic and single rounding as un-permuting first and
    then ``apply_rope_reference``."""
    M, n = y.shape
    h = head_dim // 2
    pairs = y.float().reshape(M, n // head_dim, h, 2)
    a, b = pairs[..., 0], pairs[..., 1]                       # (y_d, y_{d+h}), d < h
    c = cos.float().reshape(M, 1, 2, h)
    s = sin.float().reshape(M, 1, 2, h)
    out = torch.stack((a * c[:, :, 0] - b * s[:, :, 0], b * c[:, :, 1] + a * s[:, :, 1]), dim=2)
    return out.view(M, n).to(y.dtype)


# ----------------------------------------------------------------------------- split-K policy

@lru_cache(maxsize=None)
def tile_n() -> int:
    """Virtual rows of one decode job tile (B_N of the split-K rule)."""
    _check_ext()
    return int(_C.tile_n())


@lru_cache(maxsize=None)
def _sm_count_for(device_index: int) -> int:
    if backend_name() == "emulator":
        return int(_C.sm_count())
    return torch.cuda.get_device_properties(device_index).multi_processor_count


def virtual_rows(kind: str, *out_features: int) -> int:
    """Rows one decode call produces: N (gemv), nq + nk + nv (qkv), 2N (gate_up)."""
    if kind == "gemv":
        return out_features[0]
    if kind == "qkv":
        return sum(out_features)
    if kind == "gate_up":
        return 2 * out_features[0]
    raise ValueError(kind)


def candidate_split_k(batch: int, n: int, bn: int, sms: int, rho: int, max_split: Optional[int] = None) -> int:
    """The underfill rule (ops.py:155-163): with C_out = batch * ceil(n / bn) decode jobs and
    a target of rho * sms, split K into ceil(target / C_out) parts when C_out falls short,
    else not at all; optionally capped at max_split."""
    target = max(1, int(rho)) * sms
    jobs = batch * -(-n // bn)
    if jobs >= target:
        return 1
    parts = max(1, -(-target // jobs))
    return parts if max_split is None else min(max_split, parts)


# The split a decode call requests when the caller passes split_k=None.  The reference's
# policy is the underfill rule above (split K when fewer than rho * SMs decode jobs exist).
# Retuned for MI355X it requests no split at any shape: a decode workgroup here already spreads
# K over up to 16 slice waves, and a K split adds a round trip of fp32 partials through the L2
# plus a second finish pass.  Measured (W3, graph replays over >= 1 GiB of rotating weights,
# 25 shapes with N from 64 to 14336 and K from 1024 to 28672): at batch 1 a requested split never
# beat split 1 (the underfill rule's picks cost up to +97 % at 256 CUs, e.g. 4096 -> 512: 3.9 us
# unsplit, 7.7 us at its 8 splits); at batch 3..16 the batched planner adds splits itself where
# its own fill rule finds idle CUs.  The underfill rule stays available as candidate_split_k.
POLICY_SPLIT_K = 1


def policy_split_k(batch: int, v_rows: int, k: int, rho: int = 1, max_split: Optional[int] = None) -> int:
    """The policy's K split for a decode call of `batch` rows, `v_rows` virtual rows and K = `k`
    (POLICY_SPLIT_K, within [1, ceil(k / 32)] and `max_split`)."""
    del batch, v_rows, rho
    pk = POLICY_SPLIT_K if max_split is None else min(POLICY_SPLIT_K, max_split)
    return max(1, min(pk, -(-k // 32)))


def _k_splits(split_k: Optional[int], rho: int, batch: int, v_rows: int, k: int, x: torch.Tensor) -> int:
    """K splits of a decode call: the caller's split clamped to [1, chunks], or for
    split_k=None the policy's (policy_split_k)."""
    chunks = -(-k // 32)
    if split_k is not None:
        return max(1, min(int(split_k), chunks))
    return policy_split_k(batch, v_rows, k, rho)


# ----------------------------------------------------------------------------- ops

def _as_matrix(x: torch.Tensor):
    """x as a contiguous [M, K] matrix and its leading dims (None when already 2-D)."""
    if x.dim() == 2:
        return (x if x.is_contiguous() else x.contiguous()), None
    return x.reshape(-1, x.shape[-1]).contiguous(), x.shape[:-1]


def _restore(y: torch.Tensor, lead) -> torch.Tensor:
    return y if lead is None else y.view(*lead, y.shape[-1])


def _linear(x2, w: PackedLinearWeight, split_k, rho, act: int, threshold, workspace, use_tensor_cores):
    """One projection of a 2-D activation, decode or prefill by its row count."""
    if x2.shape[0] <= threshold:
        pk = _k_splits(split_k, rho, x2.shape[0], w.out_features, w.in_features, x2)
        return _C.packed_gemv(x2, w.packed, w.scales, w.zeros, w.bias, w.bits, w.in_features, w.group_size,
                              pk, rho, act, workspace)
    return _C.packed_gemm(x2, w.packed, w.scales, w.zeros, w.bias, w.bits, w.in_features, w.group_size,
                          act, use_tensor_cores)


def packed_linear(x: torch.Tensor, w: PackedLinearWeight, split_k: Optional[int] = None, rho: int = 1,
                  act: Optional[str] = None, decode_threshold: int = DECODE_THRESHOLD,
                  workspace: Optional[torch.Tensor] = None, use_tensor_cores: bool = True):
    """act(x W-hat^T + bias) for x [..., K]: the decode GEMV up to ``decode_threshold``
    flattened rows, the prefill GEMM beyond."""
    _check_ext()
    if w.rope_perm_head_dim:
        raise ValueError("this weight is stored RoPE-permuted; use fused_qkv (or _unpermute_cols)")
    x2, lead = _as_matrix(x)
    return _restore(_linear(x2, w, split_k, rho, ACT[act], decode_threshold, workspace, use_tensor_cores), lead)


def fused_gate_up(x: torch.Tensor, gate: PackedLinearWeight, up: PackedLinearWeight,
                  split_k: Optional[int] = None, rho: int = 1, decode_threshold: int = DECODE_THRESHOLD,
                  workspace: Optional[torch.Tensor] = None):
    """silu(x G^T) * (x U^T).  Decode: one kernel over interleaved gate/up rows, the
    product formed in fp32 and rounded once.  Prefill: the reference's two GEMMs (SiLU in
    the gate's epilogue) multiplied in the activation dtype, with its double rounding
    (ops.py:216-220) -- for fp16 / bf16 activations as one GEMM launch whose epilogue forms
    the product of the two rounded factors."""
    _check_ext()
    if gate.bits != up.bits:
        raise ValueError("fused Gate/Up requires the same precision for Gate and Up within a block")
    x2, lead = _as_matrix(x)
    M = x2.shape[0]
    if M <= decode_threshold:
        pk = _k_splits(split_k, rho, M, 2 * gate.out_features, gate.in_features, x2)
        y = _C.fused_gate_up(x2, gate.packed, gate.scales, gate.zeros, up.packed, up.scales, up.zeros,
                             gate.bits, gate.in_features, gate.group_size, pk, rho, workspace)
    elif hasattr(_C, "packed_gemm_gate_up"):
        y = _C.packed_gemm_gate_up(x2, gate.packed, gate.scales, gate.zeros, up.packed, up.scales, up.zeros,
                                   gate.bits, gate.in_features, gate.group_size)
    else:   # a backend with the reference's seven functions only (e.g. its emulator)
        y = _C.packed_gemm(x2, gate.packed, gate.scales, gate.zeros, None, gate.bits, gate.in_features,
                           gate.group_size, ACT["silu"], True)
        y.mul_(_C.packed_gemm(x2, up.packed, up.scales, up.zeros, None, up.bits, up.in_features,
                              up.group_size, ACT["none"], True))
    return _restore(y, lead)


def fused_qkv(x: torch.Tensor, q: PackedLinearWeight, k: PackedLinearWeight, v: PackedLinearWeight,
              split_k: Optional[int] = None, rho: int = 1,
              rope: Optional[Tuple[torch.Tensor, torch.Tensor, int]] = None,
              decode_threshold: int = DECODE_THRESHOLD, workspace: Optional[torch.Tensor] = None):
    """Q, K and V of one attention layer.  Decode: one kernel (GQA widths, biases, and with
    ``rope=(cos, sin, head_dim)`` HF rotate-half RoPE on Q/K stored pair-interleaved).
    Prefill: three GEMMs, then RoPE on the stored layout and the original column order."""
    _check_ext()
    if not (q.in_features == k.in_features == v.in_features and q.group_size == k.group_size == v.group_size):
        raise ValueError("Q/K/V must share in_features and group_size")
    if q.rope_perm_head_dim != k.rope_perm_head_dim or v.rope_perm_head_dim:
        raise ValueError("Q and K must be permuted with the same head_dim; V must not be permuted")
    perm = q.rope_perm_head_dim
    x2, lead = _as_matrix(x)
    M = x2.shape[0]
    cos2 = sin2 = None
    head_dim = 0
    if rope is not None:
        cos, sin, head_dim = rope
        head_dim = int(head_dim)
        if perm != head_dim:
            raise ValueError("fused RoPE needs Q/K permuted with permute_for_rope(w, head_dim) "
                             "(install_bitmap(fuse_rope=True) does this)")
        pre = x.shape[:-1]                    # one cos/sin row per activation row
        cos2 = cos.expand(*pre, head_dim).reshape(M, head_dim)
        sin2 = sin.expand(*pre, head_dim).reshape(M, head_dim)
    if M <= decode_threshold:
        pk = _k_splits(split_k, rho, M, q.out_features + k.out_features + v.out_features, q.in_features, x2)
        rc = None if cos2 is None else cos2.float().contiguous()
        rs = None if sin2 is None else sin2.float().contiguous()
        bits = q.bits if q.bits == k.bits == v.bits else (q.bits, k.bits, v.bits)
        outs = _C.fused_qkv(x2, q.packed, q.scales, q.zeros, q.bias, k.packed, k.scales, k.zeros, k.bias,
                            v.packed, v.scales, v.zeros, v.bias, rc, rs, head_dim, perm, bits, q.in_features,
                            q.group_size, pk, rho, workspace)
    else:
        outs = []
        for i, w in enumerate((q, k, v)):
            y = _linear(x2, w, None, 1, 0, 0, None, True)
            if i < 2 and cos2 is not None:
                y = _rope_stored(y, cos2, sin2, head_dim)
            elif w.rope_perm_head_dim:
                y = _original_columns(y, w.rope_perm_head_dim)
            outs.append(y)
    return tuple(_restore(o, lead) for o in outs)


def sm_count():
    _check_ext()
    return int(_C.sm_count())


def max_rho(bits: int, kind: str = "gemv"):
    _check_ext()
    return int(_C.max_rho(bits, kind))


# ----------------------------------------------------------------------------- module

class PackedLinear(nn.Module):
    """nn.Linear stand-in over a packed weight: buffers ``packed``, ``scales``, ``zeros``,
    ``bias`` (persistent) and ``workspace`` (not), the decode policy (``split_k``,
    ``rho``) and an epilogue activation ``act``."""

    def __init__(self, w: PackedLinearWeight, split_k: Optional[int] = None, rho: int = 1, act: Optional[str] = None):
        super().__init__()
        for name in ("packed", "scales", "zeros", "bias"):
            self.register_buffer(name, getattr(w, name))
        self.register_buffer("workspace", new_workspace(w.packed.device), persistent=False)
        self.bits = int(w.bits)
        self.group_size = int(w.group_size)
        self.in_features = int(w.in_features)
        self.out_features = int(w.out_features)
        self.rope_perm_head_dim = int(w.rope_perm_head_dim)
        self.split_k = None if split_k is None else int(split_k)
        self.rho = int(rho)
        self.act = act
        self._spec: Optional[PackedLinearWeight] = None

    def weight_spec(self) -> PackedLinearWeight:
        """The module's weight as a PackedLinearWeight (cached; rebuilt when a buffer or the
        RoPE layout changed)."""
        s = self._spec
        b = self._buffers
        if (s is None or s.packed is not b["packed"] or s.scales is not b["scales"] or s.zeros is not b["zeros"]
                or s.bias is not b["bias"] or s.rope_perm_head_dim != self.rope_perm_head_dim):
            s = self._spec = PackedLinearWeight(b["packed"], b["scales"], b["zeros"], self.bits, self.group_size,
                                                self.in_features, self.out_features, b["bias"],
                                                self.rope_perm_head_dim)
        return s

    def permute_for_rope_(self, head_dim: int):
        """In place: store the rows pair-interleaved for the fused RoPE epilogue."""
        w = permute_for_rope(self.weight_spec(), head_dim)
        self.packed, self.scales, self.zeros, self.bias = w.packed, w.scales, w.zeros, w.bias
        self.rope_perm_head_dim = head_dim
        return self

    def forward(self, x):
        return packed_linear(x, self.weight_spec(), self.split_k, self.rho, self.act, workspace=self.workspace)

    def extra_repr(self):
        layout = f", pair-interleaved(head_dim={self.rope_perm_head_dim})" if self.rope_perm_head_dim else ""
        act = f", act={self.act}" if self.act else ""
        return (f"{self.in_features} -> {self.out_features}, W{self.bits} g{self.group_size}, "
                f"split_k={self.split_k}, rho={self.rho}{act}{layout}")
