"""Model surgery for Hugging Face causal LMs: packed linears in, fused decode paths on.

``install_bitmap(model, packed_dir, bitmap)`` keeps the reference's interface and file
layout (Kernel/crispybits_kernels/integration.py:201-218): block i's linears come from
``block_{i:03d}_w{bits}.pt`` (or the paper's ``block_{i:03d}.pt`` + ``manifest.json``), each
becomes a ``PackedLinear``, and with ``fuse`` the block's decode paths are fused.  The
mechanism is this build's own:

* **Validate, then install, per block.**  A block's file is read and every entry checked
  (width against the bitmap, target is an ``nn.Linear``) before any of its modules is
  replaced, so a bad entry never leaves a half-converted block.
* **Fusion rules.**  Each block is offered to a short list of rules (``_FUSIONS``), each
  recognising one pattern and rewriting it: Q/K/V of an attention into one ``FusedQKV``
  owner with three slot modules; a SiLU-gated MLP into ``FusedLlamaMLP`` (gate and up in one
  decode pass); an OPT ``fc1`` followed by ReLU into the GEMV's ReLU epilogue.
* **Fused RoPE through module hooks.**  When RoPE is fused, a forward pre-hook on the
  attention evaluates Q/K/V of its ``hidden_states`` with Q/K rotated by its
  ``position_embeddings`` (``FusedQKV.prime``) and passes the attention *identity tables*
  (cos = 1, sin = 0) in their place, so the model's own rotation leaves the pre-rotated Q/K
  exactly as they are (q * 1 + rotate_half(q) * 0 = q); a forward hook (always called)
  drops whatever the slots did not take.  No modeling function is patched and nothing
  outside the converted modules changes.
"""
from __future__ import annotations

import inspect
import json
from pathlib import Path
from typing import Dict, List, Optional

import torch
import torch.nn as nn

from .io import from_packed_dict
from .ops import PackedLinear, fused_gate_up, fused_qkv, new_workspace

_DECODER_PATHS = (("model", "layers"), ("model", "decoder", "layers"))


def _blocks(model) -> List[nn.Module]:
    """The decoder blocks of a LLaMA-family (model.layers) or OPT (model.decoder.layers) LM."""
    for path in _DECODER_PATHS:
        node = model
        for attr in path:
            node = getattr(node, attr, None)
            if node is None:
                break
        if node is not None:
            return list(node)
    raise ValueError("Supported integration targets are Hugging Face LLaMA-family and OPT causal LMs")


def _get(root: nn.Module, name: str):
    node = root
    for attr in name.split("."):
        node = getattr(node, attr, None)
        if node is None:
            return None
    return node


def _set_by_dotted_name(root: nn.Module, name: str, module: nn.Module):
    parent, _, leaf = name.rpartition(".")
    setattr(_get(root, parent) if parent else root, leaf, module)


# ----------------------------------------------------------------------------- fused Q/K/V

class _Parked:
    """Outputs of one fused Q/K/V evaluation waiting for their slots."""
    __slots__ = ("source", "version", "outs", "rotated")

    def __init__(self, source, outs, rotated):
        self.source, self.version, self.outs, self.rotated = source, source._version, list(outs), rotated

    def matches(self, x, idx):
        return self.source is x and self.version == x._version and self.outs[idx] is not None


class FusedQKV(nn.Module):
    """Q/K/V of one attention layer served by one fused decode call.

    The attention's ``q_proj`` / ``k_proj`` / ``v_proj`` become slots (``_QKVProxy``) drawing
    on this owner.  ``prime(x, cos, sin)`` evaluates Q/K/V of x with Q/K rotated and parks the
    three outputs; a slot called with the parked input takes its output once.  Unprimed, the
    first slot call evaluates all three (no rotation) and parks the other two.  A slot called
    with another input while rotated outputs are parked raises RuntimeError: the model would
    rotate that input's Q/K a second time."""

    def __init__(self, q: PackedLinear, k: PackedLinear, v: PackedLinear, split_k=None, rho: int = 1,
                 rope_head_dim: int = 0):
        super().__init__()
        self.q, self.k, self.v = q, k, v
        self.split_k, self.rho = split_k, int(rho)
        self.rope_head_dim = int(rope_head_dim)
        self.register_buffer("workspace", new_workspace(q.packed.device), persistent=False)
        self._parked: Optional[_Parked] = None
        self._identity = None       # ((shape, dtype, device), cos = 1, sin = 0)

    @property
    def pending(self) -> bool:
        """Whether outputs of an evaluation are still waiting for their slots."""
        return self._parked is not None

    def compute(self, x, rope=None):
        return fused_qkv(x, self.q.weight_spec(), self.k.weight_spec(), self.v.weight_spec(), self.split_k,
                         self.rho, rope=rope, workspace=self.workspace)

    def prime(self, x, cos, sin):
        """Evaluate rotated Q/K and V of ``x`` ahead of the slots (the fused RoPE path)."""
        self._parked = _Parked(x, self.compute(x, rope=(cos, sin, self.rope_head_dim)), True)

    def release(self):
        self._parked = None

    def take(self, x, idx: int):
        p = self._parked
        if p is None or not p.matches(x, idx):
            if p is not None and p.rotated:
                self._parked = None
                raise RuntimeError("CrispyBits fused RoPE: q/k/v_proj received a different tensor than the one "
                                   "primed by the attention hook; install with fuse_rope=False for this model")
            p = self._parked = _Parked(x, self.compute(x), False)
        out, p.outs[idx] = p.outs[idx], None
        if not any(o is not None for o in p.outs):
            self._parked = None
        return out

    def identity_tables(self, cos, sin):
        """cos = 1 and sin = 0 of the given tables' shape and dtype (kept between calls)."""
        key = (tuple(cos.shape), cos.dtype, cos.device, tuple(sin.shape), sin.dtype)
        if self._identity is None or self._identity[0] != key:
            self._identity = (key, torch.ones_like(cos), torch.zeros_like(sin))
        return self._identity[1], self._identity[2]


class _QKVProxy(nn.Module):
    """The q_proj / k_proj / v_proj slot of a FusedQKV owner (the owner is not a registered
    child, so its parameters are not listed twice)."""

    def __init__(self, owner: FusedQKV, idx: int):
        super().__init__()
        object.__setattr__(self, "_owner", owner)
        self.idx = idx
        src = (owner.q, owner.k, owner.v)[idx]
        self.in_features, self.out_features = src.in_features, src.out_features

    def forward(self, x):
        return self._owner.take(x, self.idx)

    def extra_repr(self):
        return f"slot {'qkv'[self.idx]} of crispybits_qkv, {self.in_features} -> {self.out_features}"


def _takes_position_embeddings(attn: nn.Module) -> bool:
    try:
        return "position_embeddings" in inspect.signature(attn.forward).parameters
    except (TypeError, ValueError):
        return False


def _install_rope_hooks(attn: nn.Module, owner: FusedQKV):
    """Prime the owner from the attention's inputs and hand the attention identity tables."""

    def before(module, args, kwargs):
        hs = kwargs["hidden_states"] if "hidden_states" in kwargs else (args[0] if args else None)
        in_kwargs = "position_embeddings" in kwargs
        pe = kwargs["position_embeddings"] if in_kwargs else (args[1] if len(args) > 1 else None)
        if hs is None or not isinstance(pe, (tuple, list)) or len(pe) != 2:
            return None                     # nothing to fuse with: the slots evaluate unrotated
        cos, sin = pe
        owner.prime(hs, cos, sin)
        ident = owner.identity_tables(cos, sin)
        if in_kwargs:
            return args, {**kwargs, "position_embeddings": ident}
        return (args[0], ident, *args[2:]), kwargs

    def after(module, args, kwargs, output):
        owner.release()

    attn.register_forward_pre_hook(before, with_kwargs=True)
    attn.register_forward_hook(after, with_kwargs=True, always_call=True)


def _head_dim(attn) -> int:
    hd = getattr(attn, "head_dim", None)
    if hd is None and hasattr(attn, "config"):
        cfg = attn.config
        hd = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
    return int(hd) if hd else 0


# ----------------------------------------------------------------------------- fused MLP

class FusedLlamaMLP(nn.Module):
    """A SiLU-gated MLP whose gate and up projections run as one decode pass."""

    def __init__(self, gate: PackedLinear, up: PackedLinear, down: PackedLinear, split_k=None, rho: int = 1):
        super().__init__()
        self.gate_proj, self.up_proj, self.down_proj = gate, up, down
        self.split_k, self.rho = split_k, int(rho)
        self.register_buffer("workspace", new_workspace(gate.packed.device), persistent=False)

    def forward(self, x):
        hidden = fused_gate_up(x, self.gate_proj.weight_spec(), self.up_proj.weight_spec(), self.split_k, self.rho,
                               workspace=self.workspace)
        return self.down_proj(hidden)


# ----------------------------------------------------------------------------- fusion rules

def _all_packed(mod, names) -> bool:
    return mod is not None and all(isinstance(getattr(mod, n, None), PackedLinear) for n in names)


def _activation_named(mod, names) -> bool:
    return mod is not None and type(mod).__name__ in names


def _fuse_attention(block, i, tuning, fuse_rope) -> bool:
    attn = getattr(block, "self_attn", None)
    if not _all_packed(attn, ("q_proj", "k_proj", "v_proj")):
        return False
    cfg = tuning.get(f"block.{i}.self_attn.qkv", {})
    rope_hd = 0
    rotary = hasattr(block, "mlp") and not hasattr(block, "fc1")       # LLaMA family; OPT has no RoPE
    if fuse_rope and rotary and _takes_position_embeddings(attn):
        hd = _head_dim(attn)
        if hd and hd % 2 == 0 and attn.q_proj.out_features % hd == 0 and attn.k_proj.out_features % hd == 0:
            attn.q_proj.permute_for_rope_(hd)
            attn.k_proj.permute_for_rope_(hd)
            rope_hd = hd
    owner = FusedQKV(attn.q_proj, attn.k_proj, attn.v_proj, cfg.get("split_k"), cfg.get("rho", 1), rope_hd)
    attn.crispybits_qkv = owner
    attn.q_proj, attn.k_proj, attn.v_proj = (_QKVProxy(owner, j) for j in range(3))
    if rope_hd:
        _install_rope_hooks(attn, owner)
    return True


def _fuse_swiglu(block, i, tuning, fuse_rope) -> bool:
    mlp = getattr(block, "mlp", None)
    if not (_all_packed(mlp, ("gate_proj", "up_proj", "down_proj"))
            and _activation_named(getattr(mlp, "act_fn", None), ("SiLU", "SiLUActivation"))):
        return False
    cfg = tuning.get(f"block.{i}.mlp.gate_up", {})
    block.mlp = FusedLlamaMLP(mlp.gate_proj, mlp.up_proj, mlp.down_proj, cfg.get("split_k"), cfg.get("rho", 1))
    return True


def _fuse_relu_fc1(block, i, tuning, fuse_rope) -> bool:
    if not (isinstance(getattr(block, "fc1", None), PackedLinear)
            and _activation_named(getattr(block, "activation_fn", None), ("ReLU",))):
        return False
    block.fc1.act = "relu"
    block.activation_fn = nn.Identity()
    return True


_FUSIONS = (_fuse_attention, _fuse_swiglu, _fuse_relu_fc1)


# ----------------------------------------------------------------------------- install

def _block_file(packed_dir: Path, i: int, bits: int) -> Path:
    """block_{i:03d}_w{bits}.pt (write_packed_dir, reference.py:85-94), else the one-width
    block_{i:03d}.pt of the paper's pack_checkpoint.py:26."""
    for name in (f"block_{i:03d}_w{bits}.pt", f"block_{i:03d}.pt"):
        path = packed_dir / name
        if path.exists():
            return path
    raise FileNotFoundError(f"neither block_{i:03d}_w{bits}.pt nor block_{i:03d}.pt in {packed_dir}")


def install_bitmap(model: nn.Module, packed_dir: str, bitmap, device="cuda", dtype=torch.float16,
                   tuning: Optional[Dict] = None, fuse: bool = True, fuse_rope: bool = True):
    """Replace every linear of block i with its packed weights of width ``bitmap[i]`` (the
    bitmap of ``manifest.json`` when None), then fuse each block's decode paths."""
    root = Path(packed_dir)
    if bitmap is None:
        with open(root / "manifest.json") as f:
            bitmap = json.load(f)["bitmap"]
    blocks = _blocks(model)
    if len(blocks) != len(bitmap):
        raise ValueError("bitmap length does not match model")
    tuning = tuning or {}
    for i, (block, bits) in enumerate(zip(blocks, bitmap)):
        bits = int(bits)
        entries = torch.load(_block_file(root, i, bits), map_location="cpu", weights_only=True)
        for name, d in entries.items():
            if int(d["bits"]) != bits:
                raise ValueError(f"block {i}: '{name}' is packed at W{int(d['bits'])}, the bitmap asks for W{bits}")
            if not isinstance(_get(block, name), nn.Linear):
                raise ValueError(f"block {i}: '{name}' is not an nn.Linear in this model")
        for name, d in entries.items():
            cfg = tuning.get(f"block.{i}.{name}", {})
            _set_by_dotted_name(block, name, PackedLinear(from_packed_dict(d, device=device, dtype=dtype),
                                                          split_k=cfg.get("split_k"), rho=int(cfg.get("rho", 1))))
        if fuse:
            for rule in _FUSIONS:
                rule(block, i, tuning, fuse_rope)
    return model


def load_tuning(path: Optional[str]):
    if not path:
        return {}
    with open(path) as f:
        return json.load(f)


def save_tuning(tuning: Dict, path: str):
    with open(path, "w") as f:
        json.dump(tuning, f, indent=2, sort_keys=True)
