"""Decode policy tuner for the packed linears.

Interface of Kernel/crispybits_kernels/autotune.py:1-169: ``TuneResult``, ``TuneReport``
(``best``, ``oracle``, ``results``, ``regret``), ``_time(fn, warmup, iters)``, ``tune_gemv``,
``tune_qkv``, ``tune_gate_up`` and ``tune_model`` (which sets each module's ``split_k`` /
``rho`` and returns the ``{"block.i.<name>": {"split_k", "rho"}}`` dict that
``install_bitmap(tuning=...)`` reads).  The search is this build's own and works in
*launches*:

* The candidate points are the split-K policy's pick (``ops.policy_split_k``) for every rho
  in 1..max_rho and, with ``exhaustive``, every split request of ``EXHAUSTIVE_PK`` at every
  rho.  Each point is mapped to the launch the library makes for it (``_C.decode_plan``:
  kernel family, K splits, workgroups, threads, LDS, launches per call); points that map to
  the same launch are one candidate, timed once, and a candidate is a policy candidate when
  any policy pick maps to it.  On the streaming kernels rho changes no launch, so it adds no
  timing.
* Time is kernel time: the summed dispatch durations of a call (a split call counts its
  combine launch), from the library's per-dispatch timer, so the ranking sees the kernels
  and not the host's launch rate.
* ``tune_model`` first lists the model's tunables (fused Q/K/V owners, fused MLPs and the
  packed linears outside them) with a shape signature each, tunes every distinct signature
  once, and then writes the winners back.
"""
from __future__ import annotations

import time
from dataclasses import asdict, dataclass, field
from math import ceil
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import torch

from . import ops
from .ops import (BATCH_TILE, PackedLinear, PackedLinearWeight, fused_gate_up, fused_qkv, policy_split_k,
                  max_rho, new_workspace, packed_linear, sm_count, tile_n, virtual_rows)

# Split requests of the exhaustive sweep: dense where the streaming kernels' launches differ
# (a K = 4096 row is 128 chunks, 11008 is 344), sparse beyond; duplicates of one launch cost
# nothing.
EXHAUSTIVE_PK = (1, 2, 3, 4, 5, 6, 8, 10, 12, 16, 20, 24, 32, 43, 64, 86)


@dataclass
class TuneResult:
    rho: int
    split_k: int
    ms: float
    c_out: int
    c_target: int
    policy: bool = True
    launch: Tuple = field(default=(), compare=False)


@dataclass
class TuneReport:
    best: TuneResult
    oracle: TuneResult
    results: List[TuneResult]

    @property
    def regret(self) -> float:
        return self.best.ms / self.oracle.ms - 1.0


def _kernel_timer():
    """The HIP library (its per-dispatch timer) when the ops run on it, else None."""
    C = ops._C
    if C is not None and C is ops._CUDA and hasattr(C, "timer_start"):
        return C
    return None


def _time(fn: Callable[[], object], warmup: int, iters: int) -> float:
    """Mean ms per call of ``fn``.  On the HIP library: the summed durations of the call's
    kernel launches, recorded inside each dispatch.  Otherwise device events around the
    calls, or the host clock on the CPU."""
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


def _launch(kind: str, batch: int, k: int, gs: int, widths: Sequence[int], bits, split: int, rho: int,
            dtype) -> Tuple:
    return tuple(ops._C.decode_plan(dtype, batch, k, gs, tuple(widths) if kind == "qkv" else widths[0], bits,
                                    kind, split, rho))


def _search(run: Callable[[int, int], object], kind: str, batch: int, k: int, gs: int, widths: Sequence[int],
            bits, dtype, warmup: int, iters: int, max_split: Optional[int], exhaustive: bool) -> TuneReport:
    sms, bn = sm_count(), tile_n()
    v_rows = virtual_rows(kind, *widths)
    batch_tiles = ceil(batch / BATCH_TILE)
    chunks = ceil(k / 32)
    widest = max(bits) if isinstance(bits, (tuple, list)) else bits
    rhos = range(1, max(1, max_rho(widest, kind)) + 1)
    points = [(rho, policy_split_k(batch, v_rows, k, rho, max_split), True) for rho in rhos]
    if exhaustive:
        points += [(rho, pk, False) for rho in rhos for pk in EXHAUSTIVE_PK if max_split is None or pk <= max_split]
    candidates: Dict[Tuple, List] = {}            # launch -> [rho, split, policy], first point first
    for rho, pk, policy in points:
        pk = max(1, min(pk, chunks))
        launch = _launch(kind, batch, k, gs, widths, bits, pk, rho, dtype)
        if launch in candidates:
            candidates[launch][2] |= policy
        else:
            candidates[launch] = [rho, pk, policy]
    c_out = batch_tiles * ceil(v_rows / bn)
    results = [TuneResult(rho, pk, _time(lambda: run(pk, rho), warmup, iters), c_out, rho * sms, policy, launch)
               for launch, (rho, pk, policy) in candidates.items()]
    best = min((r for r in results if r.policy), key=lambda r: r.ms)
    oracle = min(results, key=lambda r: r.ms)
    return TuneReport(best, oracle, results)


def _rows(x: torch.Tensor) -> int:
    return x.numel() // x.shape[-1]


def tune_gemv(x: torch.Tensor, w: PackedLinearWeight, warmup: int = 10, iters: int = 50,
              max_split: Optional[int] = None, act: Optional[str] = None, exhaustive: bool = False) -> TuneReport:
    ws = new_workspace(x.device)
    return _search(lambda pk, rho: packed_linear(x, w, pk, rho, act, workspace=ws), "gemv", _rows(x),
                   w.in_features, w.group_size, (w.out_features,), w.bits, x.dtype, warmup, iters, max_split,
                   exhaustive)


def tune_qkv(x, q: PackedLinearWeight, k: PackedLinearWeight, v: PackedLinearWeight,
             warmup: int = 10, iters: int = 50, max_split: Optional[int] = None,
             exhaustive: bool = False) -> TuneReport:
    ws = new_workspace(x.device)
    return _search(lambda pk, rho: fused_qkv(x, q, k, v, pk, rho, workspace=ws), "qkv", _rows(x), q.in_features,
                   q.group_size, (q.out_features, k.out_features, v.out_features), (q.bits, k.bits, v.bits),
                   x.dtype, warmup, iters, max_split, exhaustive)


def tune_gate_up(x, gate: PackedLinearWeight, up: PackedLinearWeight, warmup: int = 10, iters: int = 50,
                 max_split: Optional[int] = None, exhaustive: bool = False) -> TuneReport:
    ws = new_workspace(x.device)
    return _search(lambda pk, rho: fused_gate_up(x, gate, up, pk, rho, workspace=ws), "gate_up", _rows(x),
                   gate.in_features, gate.group_size, (gate.out_features,), gate.bits, x.dtype, warmup, iters,
                   max_split, exhaustive)


def _tunables(model, measure_qkv, measure_gate_up, measure_gemv):
    """{signature: (measure, [(tuning key, module), ...])} over the model's blocks, in block
    order: fused Q/K/V owners, fused MLPs, and packed linears not inside either."""
    from .integration import FusedLlamaMLP, FusedQKV, _blocks
    found: Dict[Tuple, Tuple[Callable[[], TuneReport], List]] = {}

    def add(sig, measure, key, module):
        found.setdefault(sig, (measure, []))[1].append((key, module))

    for i, block in enumerate(_blocks(model)):
        inside = set()
        for m in block.modules():
            if isinstance(m, FusedQKV):
                inside.update(map(id, (m.q, m.k, m.v)))
            elif isinstance(m, FusedLlamaMLP):
                inside.update(map(id, (m.gate_proj, m.up_proj)))
        for name, m in block.named_modules():
            if isinstance(m, FusedQKV):
                specs = tuple(t.weight_spec() for t in (m.q, m.k, m.v))
                sig = ("qkv", specs[0].in_features, specs[0].group_size,
                       tuple((s.bits, s.out_features, s.bias is not None) for s in specs))
                add(sig, lambda s=specs: measure_qkv(*s), f"block.{i}.self_attn.qkv", m)
            elif isinstance(m, FusedLlamaMLP):
                g, u = m.gate_proj.weight_spec(), m.up_proj.weight_spec()
                sig = ("gate_up", g.in_features, g.group_size, g.bits, g.out_features)
                add(sig, lambda g=g, u=u: measure_gate_up(g, u), f"block.{i}.mlp.gate_up", m)
            elif isinstance(m, PackedLinear) and id(m) not in inside:
                w = m.weight_spec()
                sig = ("gemv", w.in_features, w.group_size, w.bits, w.out_features, w.bias is not None, m.act)
                add(sig, lambda w=w, act=m.act: measure_gemv(w, act), f"block.{i}.{name}", m)
    return found


@torch.no_grad()
def tune_model(model: torch.nn.Module, batch: int = 1, warmup: int = 10, iters: int = 50,
               max_split: Optional[int] = None, dtype=torch.float16, verbose: bool = False,
               exhaustive: bool = False) -> Dict[str, Dict]:
    """Tune every packed module of a model converted by install_bitmap at ``batch`` rows;
    sets each module's split_k / rho and returns the tuning dict."""
    opts = dict(warmup=warmup, iters=iters, max_split=max_split, exhaustive=exhaustive)

    def sample(w: PackedLinearWeight):
        return torch.randn(batch, w.in_features, device=w.packed.device, dtype=dtype)

    found = _tunables(model,
                      lambda q, k, v: tune_qkv(sample(q), q, k, v, **opts),
                      lambda g, u: tune_gate_up(sample(g), g, u, **opts),
                      lambda w, act: tune_gemv(sample(w), w, act=act, **opts))
    tuning: Dict[str, Dict] = {}
    for sig, (measure, members) in found.items():
        report = measure()
        for key, module in members:
            module.split_k, module.rho = report.best.split_k, report.best.rho
            tuning[key] = {"split_k": report.best.split_k, "rho": report.best.rho}
        if verbose:
            print(sig, "best", asdict(report.best), "oracle", asdict(report.oracle), f"regret {report.regret:+.1%}",
                  f"({len(members)} module(s))")
    return tuning
