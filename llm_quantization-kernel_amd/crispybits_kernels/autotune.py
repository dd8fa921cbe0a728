"""(rho, split_k) tuner for the decode kernels (Kernel/crispybits_kernels/autotune.py:1-169 interface).

For each rho in 1..max_rho the split-K rule's pick is timed; with ``exhaustive``
every split in EXHAUSTIVE_PK is timed too.  ``best`` is the fastest rule pick,
``oracle`` the fastest point measured, and ``regret = best/oracle - 1``.
Candidates that launch the same (split, workgroup count) are timed once.

Retuned for MI355X: splits are in units of the MFMA kernel's 128-code K unit, so
the grid stops at 32 (a 4096-wide row has 32 units); candidates are ranked by kernel
time from the library's per-dispatch timer (see ``_time``).
"""
from __future__ import annotations

import time
from dataclasses import asdict, dataclass
from math import ceil
from typing import Callable, Dict, List, Optional

import torch

from .ops import (BATCH_TILE, PackedLinear, PackedLinearWeight, candidate_split_k, fused_gate_up, fused_qkv,
                  max_rho, new_workspace, packed_linear, sm_count, tile_n, virtual_rows)

EXHAUSTIVE_PK = (1, 2, 3, 4, 6, 8, 12, 16, 24, 32)


@dataclass
class TuneResult:
    rho: int
    split_k: int
    ms: float
    c_out: int
    c_target: int
    policy: bool = True


@dataclass
class TuneReport:
    best: TuneResult
    oracle: TuneResult
    results: List[TuneResult]

    @property
    def regret(self) -> float:
        return self.best.ms / self.oracle.ms - 1.0


def _kernel_timer():
    """The HIP library's per-dispatch timer when the ops run on it, else None."""
    from . import ops
    C = ops._C
    if C is not None and C is ops._CUDA and hasattr(C, "timer_start"):
        return C
    return None


def _time(fn: Callable[[], object], warmup: int, iters: int) -> float:
    """Mean ms per call.  On the HIP library: the summed durations of the call's kernel
    launches (events recorded inside each dispatch; a split-K call counts its combine
    launch too), so the ranking sees the kernels and not the host's launch rate -- events
    around back-to-back calls (the reference's autotune.py:40-48) read the Python
    dispatch cost here, ~12 us per call, above every decode kernel.  Otherwise device
    events, or the wall clock on the CPU."""
    for _ in range(warmup):
        fn()
    C = _kernel_timer()
    if C is not None:
        torch.cuda.synchronize()
        C.timer_start(4 * iters + 16)
        try:
            for _ in range(iters):
                fn()
        finally:
            total, _ = C.timer_stop()
        return total / iters
    if torch.cuda.is_available() and torch.cuda.is_initialized():
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(iters):
            fn()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / iters
    start = time.perf_counter()
    for _ in range(iters):
        fn()
    return (time.perf_counter() - start) * 1e3 / iters


def _tune(run: Callable[[int, int], object], B: int, V: int, K: int, bits: int, kind: str,
          warmup: int, iters: int, max_split: Optional[int], exhaustive: bool = False) -> TuneReport:
    S, bn = sm_count(), tile_n()
    occ = max(1, max_rho(bits, kind))
    nchunks = ceil(K / 32)
    jobs_per_split = ceil(B / BATCH_TILE) * ceil(V / bn)
    results: List[TuneResult] = []
    timed: Dict[tuple, TuneResult] = {}

    def measure(rho: int, pk: int, policy: bool):
        pk = max(1, min(pk, nchunks))
        key = (pk, min(jobs_per_split * pk, rho * S))
        if key in timed:
            timed[key].policy = timed[key].policy or policy
            return
        ms = _time(lambda: run(pk, rho), warmup, iters)
        r = TuneResult(rho, pk, ms, jobs_per_split, rho * S, policy)
        timed[key] = r
        results.append(r)

    for rho in range(1, occ + 1):
        measure(rho, candidate_split_k(ceil(B / BATCH_TILE), V, bn, S, rho, max_split), True)
    if exhaustive:
        for rho in range(1, occ + 1):
            for pk in EXHAUSTIVE_PK:
                if max_split is None or pk <= max_split:
                    measure(rho, pk, False)
    best = min((r for r in results if r.policy), key=lambda r: r.ms)
    oracle = min(results, key=lambda r: r.ms)
    return TuneReport(best, oracle, results)


def tune_gemv(x: torch.Tensor, w: PackedLinearWeight, warmup: int = 10, iters: int = 50,
              max_split: Optional[int] = None, act: Optional[str] = None, exhaustive: bool = False) -> TuneReport:
    B = x.reshape(-1, x.shape[-1]).shape[0]
    ws = new_workspace(x.device)
    return _tune(lambda pk, rho: packed_linear(x, w, pk, rho, act, workspace=ws), B,
                 virtual_rows("gemv", w.out_features), w.in_features, w.bits, "gemv",
                 warmup, iters, max_split, exhaustive)


def tune_qkv(x, q: PackedLinearWeight, k: PackedLinearWeight, v: PackedLinearWeight,
             warmup: int = 10, iters: int = 50, max_split: Optional[int] = None,
             exhaustive: bool = False) -> TuneReport:
    B = x.reshape(-1, x.shape[-1]).shape[0]
    ws = new_workspace(x.device)
    V = virtual_rows("qkv", q.out_features, k.out_features, v.out_features)
    return _tune(lambda pk, rho: fused_qkv(x, q, k, v, pk, rho, workspace=ws), B, V, q.in_features,
                 max(q.bits, k.bits, v.bits), "qkv", warmup, iters, max_split, exhaustive)


def tune_gate_up(x, gate: PackedLinearWeight, up: PackedLinearWeight, warmup: int = 10, iters: int = 50,
                 max_split: Optional[int] = None, exhaustive: bool = False) -> TuneReport:
    B = x.reshape(-1, x.shape[-1]).shape[0]
    ws = new_workspace(x.device)
    return _tune(lambda pk, rho: fused_gate_up(x, gate, up, pk, rho, workspace=ws), B,
                 virtual_rows("gate_up", gate.out_features), gate.in_features, gate.bits, "gate_up",
                 warmup, iters, max_split, exhaustive)


@torch.no_grad()
def tune_model(model: torch.nn.Module, batch: int = 1, warmup: int = 10, iters: int = 50,
               max_split: Optional[int] = None, dtype=torch.float16, verbose: bool = False,
               exhaustive: bool = False) -> Dict[str, Dict]:
    """Tune every packed module of a model installed with install_bitmap; sets each
    module's split_k / rho and returns {"block.i.<name>": {"split_k", "rho"}}."""
    from .integration import FusedLlamaMLP, FusedQKV, _blocks
    cache: Dict[tuple, TuneReport] = {}
    tuning: Dict[str, Dict] = {}

    def sample(K, device):
        return torch.randn(batch, K, device=device, dtype=dtype)

    def once(key, fn):
        if key not in cache:
            cache[key] = fn()
        return cache[key].best

    for i, block in enumerate(_blocks(model)):
        fused_members = set()
        for m in block.modules():
            if isinstance(m, FusedQKV):
                fused_members.update(id(t) for t in (m.q, m.k, m.v))
            elif isinstance(m, FusedLlamaMLP):
                fused_members.update(id(t) for t in (m.gate_proj, m.up_proj))
        for name, mod in block.named_modules():
            if isinstance(mod, FusedQKV):
                specs = [t.weight_spec() for t in (mod.q, mod.k, mod.v)]
                key = ("qkv", tuple(s.bits for s in specs), specs[0].in_features, *(s.out_features for s in specs))
                r = once(key, lambda: tune_qkv(sample(specs[0].in_features, specs[0].packed.device), *specs,
                                               warmup=warmup, iters=iters, max_split=max_split,
                                               exhaustive=exhaustive))
                mod.split_k, mod.rho = r.split_k, r.rho
                tuning[f"block.{i}.self_attn.qkv"] = {"split_k": r.split_k, "rho": r.rho}
            elif isinstance(mod, FusedLlamaMLP):
                g, u = mod.gate_proj.weight_spec(), mod.up_proj.weight_spec()
                key = ("gate_up", g.bits, g.in_features, g.out_features)
                r = once(key, lambda: tune_gate_up(sample(g.in_features, g.packed.device), g, u, warmup=warmup,
                                                   iters=iters, max_split=max_split, exhaustive=exhaustive))
                mod.split_k, mod.rho = r.split_k, r.rho
                tuning[f"block.{i}.mlp.gate_up"] = {"split_k": r.split_k, "rho": r.rho}
            elif isinstance(mod, PackedLinear) and id(mod) not in fused_members:
                w = mod.weight_spec()
                key = ("gemv", w.bits, w.in_features, w.out_features, w.bias is not None, mod.act)
                r = once(key, lambda: tune_gemv(sample(w.in_features, w.packed.device), w, warmup=warmup,
                                                iters=iters, max_split=max_split, act=mod.act,
                                                exhaustive=exhaustive))
                mod.split_k, mod.rho = r.split_k, r.rho
                tuning[f"block.{i}.{name}"] = {"split_k": r.split_k, "rho": r.rho}
        if verbose:
            print(f"block {i} tuned")
    if verbose:
        for k, rep in cache.items():
            print(k, "best", asdict(rep.best), "oracle", asdict(rep.oracle), f"regret {rep.regret:+.1%}")
    return tuning
