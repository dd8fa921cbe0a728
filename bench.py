#!/usr/bin/env python3
"""MI355X benchmark of the packed W2/W3/W4 linear kernels (one GPU).

Timed workload (the metric's W3 decode GEMV): one step
is one token (M = 1, fp16 activations) through the W3 decode GEMV of the three
Llama-2-7B-like shapes (K, N) = (4096, 4096), (4096, 11008), (11008, 4096),
group size 128, for 32 layers with distinct weight copies (1.29 GB of packed
weights, so the 256 MB Infinity Cache cannot serve repeats).  The 96 launches of
a step are captured once in a HIP graph; `value` is the whole-step throughput in
algorithmic GB/s (wall clock over K replays, inputs resident in HBM).

Correctness gate (before anything is timed): every launch configuration the run times -- each
candidate (split_k, rho) of the timed step, the timed graph's own outputs after its warm-up
replays, every sweep row, the fused modes and the stack's plans -- is checked against the
oracle's float64 dequant-matmul at the reference's bars (fp16 3e-3, bf16 2e-2); a miss exits
with status 3 and no result line.  The line records the checks in `correctness_checked`.

Also reported (outside the timed region): per-launch kernel durations from the
library's dispatch-recorded event timer for the full decode matrix (W2/W3/W4 x
M in {1,4,8} x the three shapes), the fused QKV / gate-up decode, the M=1024 and
M=2048 prefill GEMM, the roofline of the dominant kernel, and the CPU oracle
(dequant + matmul) on a bounded sample on the host cores.

Algorithmic bytes of one decode launch:
    N*ceil(K/32)*bits*4 (packed) + N*ceil(K/128)*2*2 (fp16 scales+zeros) + M*K*2 + M*N*2
Algorithmic FLOPs of one prefill launch: 2*M*N*K.

`roofline.traffic` (HBM bytes per launch of the dominant kernel) is read from
profiles/gemv_w3_m1_traffic.txt, written from two rocprofv3 --pmc passes
(FETCH_SIZE, WRITE_SIZE) over `bench.py --pmc-workload` scaled by the same
counters' reading for a copy of known size; null if that file is absent.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]
       python bench.py --pmc-workload [gemv|gemm]   (fixed launches for counter collection)
Prints one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "llm_quantization-kernel_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_w3_m1_traffic.txt")
PMC_COPY_BYTES = 256 << 20     # calibration copy of the counter passes
MFMA_F16_PEAK_TFS = 2500.0     # MI355X dense fp16 MFMA, published
MFMA_F32_PEAK_TFS = 157.3      # MI355X dense fp32 matrix, published
METRIC = "W3/W4 GEMV µs & HBM GB/s (% peak); M=1024 prefill GEMM TFLOP/s (% peak)"
SHAPES = [(4096, 4096), (4096, 11008), (11008, 4096)]          # (K, N)
LAYERS = 32
GS = 128


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_bytes(M, K, N, bits, gs=GS):
    return N * math.ceil(K / 32) * bits * 4 + N * math.ceil(K / gs) * 4 + M * K * 2 + M * N * 2


def make_weight(torch, N, K, bits, seed, device):
    """BASELINE inputs: W = randn(N, K, seed) * 0.02, group-affine quantized and packed."""
    from crispybits_kernels.ops import PackedLinearWeight
    from crispybits_kernels.reference import quantize_pack
    g = torch.Generator().manual_seed(seed)
    W = (torch.randn(N, K, generator=g) * 0.02).to(device)
    packed, s, z = quantize_pack(W, bits, GS)
    return PackedLinearWeight(packed, s, z, bits, GS, K, N)


def clone_weight(w):
    from dataclasses import replace
    return replace(w, packed=w.packed.clone(), scales=w.scales.clone(), zeros=w.zeros.clone())


def randx(torch, M, K, seed, device):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(M, K, generator=g).half().to(device)


class Gate:
    """Correctness gate: every launch configuration the bench times is first checked against the
    oracle's float64 dequant-matmul on the same inputs, as the reference benches refuse to time a
    wrong kernel (Kernel/scripts/bench_gemv.py:21-24, bench_prefill.py:19-22).  Bars: max|y - ref|
    / max|ref| below 3e-3 for fp16 and 2e-2 for bf16 outputs (Kernel/tests/test_correctness.py:10),
    both inside the brief's 1e-2 for fp16.  A miss ends the run with exit status 3 and no result
    line.  Prefill checks compare every 16th output row (the row within its 16-row group rotating),
    so every 128-row tile of the GEMM is covered."""
    BAR = {"torch.float16": 3e-3, "torch.bfloat16": 2e-2, "torch.float32": 1e-4}

    def __init__(self, torch):
        self.torch = torch
        self.cache = {}
        self.checks = 0
        self.worst = {}

    def weight64(self, w):
        """float64 W-hat of a packed weight (its metadata as stored), cached per weight object."""
        k = id(w)
        if k not in self.cache:
            from oracle import emulator as E
            W = E.dequant64_fast(w.packed.cpu().numpy(), w.scales.double().cpu().numpy(),
                                 w.zeros.double().cpu().numpy(), w.bits, w.in_features, w.group_size)
            self.cache[k] = (w, self.torch.from_numpy(W))
        return self.cache[k][1]

    def clear(self):
        self.cache.clear()

    @staticmethod
    def rows(M):
        if M <= 64:
            return None
        return [16 * i + (i % 16) for i in range(M // 16) if 16 * i + (i % 16) < M]

    def linear64(self, x, w, rows=None, round_w=None, act=None):
        """x W-hat^T in float64 for the given rows of x; W-hat rounded once to `round_w` (the
        matrix-core prefill's operand) when given."""
        torch = self.torch
        W = self.weight64(w)
        if round_w is not None:
            W = W.to(round_w).double()
        xs = x if rows is None else x[rows]
        y = xs.double().cpu() @ W.T
        if act == "silu":
            from oracle import emulator as E
            y = torch.from_numpy(E.silu64(y.numpy()))
        return y

    def check(self, tag, y, ref, rows=None):
        torch = self.torch
        yy = (y if rows is None else y[rows]).double().cpu()
        den = ref.abs().max().item()
        err = (yy - ref).abs().max().item() / (den + 1e-6)
        bar = self.BAR[str(y.dtype)]
        self.checks += 1
        key = str(y.dtype).replace("torch.", "")
        self.worst[key] = max(self.worst.get(key, 0.0), err)
        if not (err < bar and math.isfinite(err)):
            log(f"CORRECTNESS GATE: {tag}: rel err {err:.3e} >= {bar:.0e}; not timing")
            raise SystemExit(3)

    def gemv(self, tag, y, x, w, act=None):
        self.check(tag, y, self.linear64(x, w, act=act))

    def gemm(self, tag, y, x, w):
        rows = self.rows(x.shape[0])
        self.check(tag, y, self.linear64(x, w, rows, round_w=x.dtype), rows)

    def record(self):
        return {"checks": self.checks, "max_rel_err": {k: float(f"{v:.3e}") for k, v in self.worst.items()},
                "bar": {"fp16": 3e-3, "bf16": 2e-2},
                "reference": "oracle float64 dequant-matmul (oracle.emulator.dequant64_fast) on the same inputs; "
                             "every timed (shape, bits, M, split_k, rho) and sweep row checked once before it "
                             "is timed, the timed step's graph outputs (first and last layer copy) after its "
                             "warm-up replays; prefill rows sampled one per 16"}


def timed_kernels(C, fn, n_launch):
    """Run fn() (which makes n_launch library launches) with the dispatch timer armed."""
    C.timer_start(n_launch + 8)
    try:
        fn()
    finally:
        total, durs = C.timer_stop()
    return total, durs


def graph_launch_us(torch, fn, n_launch, replays=20):
    """Mean µs per launch of fn() (which makes n_launch launches), captured once as a HIP graph
    and replayed `replays` times between events recorded on the replay stream."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    g.replay()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(replays):
        g.replay()
    t1.record(stream)
    t1.synchronize()
    ms = t0.elapsed_time(t1)
    del g
    return ms * 1e3 / (replays * n_launch)


def best_config(torch, C, ops, x, ws, candidates, gate, base):
    """Pick (split_k, rho) with the shortest graph-replayed time over the layer copies; each
    candidate is checked against the oracle before it is timed."""
    best = None
    for sk, rho in candidates:
        gate.gemv(f"W{base.bits} M={x.shape[0]} {base.in_features}->{base.out_features} split_k={sk} rho={rho}",
                  ops.packed_linear(x, ws[0], sk, rho), x, base)
        us = graph_launch_us(torch, lambda: [ops.packed_linear(x, w, sk, rho) for w in ws], len(ws), replays=4)
        if best is None or us < best[0]:
            best = (us, sk, rho)
    return best[1], best[2]


def _median_ms(fn, warm=2, runs=5):
    for _ in range(warm):
        fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times) * 1e3


def cpu_baseline(torch, dev, base, xs):
    """The reference's CPU path on the host cores (dequantize + matmul, and the matmul alone) on
    the same seeded inputs as the GPU: the oracle's restatement of reference.py unpack_codes -> dequantize
    (reference.py:30-34,58-67; unpack by code slot, oracle.reference.unpack_codes_by_slot, then
    (q - z) s in fp32) followed by x.float() @ W.T (test_correctness.py:23-31), torch on every core
    this process may use.  Two numbers per config: dequant + matmul per call, and the matmul alone
    on a pre-dequantized fp32 W.  Configs 1, 2 and 4: 2 warm-up runs, median of 5; configs 3 and 5
    (5 and 7 weights): 1 warm-up, median of 3, config 5 on one block of the 32 (x 32 for a step)."""
    import numpy as np
    from oracle import reference as R
    affinity = len(os.sched_getaffinity(0))
    torch.set_num_threads(affinity)

    def host(w):
        return (w.packed.cpu().numpy(), w.scales.float().cpu(), w.zeros.float().cpu(), w.bits, w.in_features)

    def dequant(h):
        packed, s, z, bits, K = h
        q = torch.from_numpy(np.ascontiguousarray(R.unpack_codes_by_slot(packed, bits, K)))
        G = s.shape[1]
        return ((q.view(q.shape[0], G, GS).float() - z[:, :, None]) * s[:, :, None]).view(q.shape[0], K)

    def row(weights, x, flop_or_bytes, unit, warm=2, runs=5):
        hs = [host(w) for w in weights]
        xc = x.float().cpu()
        dense = [dequant(h) for h in hs]
        full = _median_ms(lambda: [xc @ dequant(h).T for h in hs], warm, runs)
        mm = _median_ms(lambda: [xc @ W.T for W in dense], warm, runs)
        rate = flop_or_bytes / (full * 1e-3)
        r = {"dequant_matmul_ms": round(full, 3), "matmul_only_ms": round(mm, 3)}
        if unit == "GB/s":
            r["GBps"] = round(rate / 1e9, 4)
        else:
            r["TFLOPs"] = round(rate / 1e12, 4)
            r["TFLOPs_matmul_only"] = round(flop_or_bytes / (mm * 1e-3) / 1e12, 4)
        return r

    res = {}
    # config 1: W4 GEMV M=1 4096 x 4096
    w1 = make_weight(torch, 4096, 4096, 4, 0, dev)
    x1 = randx(torch, 1, 4096, 1, dev)
    res["config1_w4_gemv_m1_4096x4096"] = row([w1], x1, gemv_bytes(1, 4096, 4096, 4), "GB/s")
    # config 2 (the timed workload): one layer-set of the step, the three W3 GEMVs at M = 1
    c2 = [row([w], x, gemv_bytes(1, w.in_features, w.out_features, w.bits), "GB/s") for w, x in zip(base, xs)]
    full2 = sum(r["dequant_matmul_ms"] for r in c2)
    nbytes2 = sum(gemv_bytes(1, w.in_features, w.out_features, w.bits) for w in base)
    res["config2_w3_gemv_m1_layer_set"] = {"dequant_matmul_ms": round(full2, 3),
                                           "matmul_only_ms": round(sum(r["matmul_only_ms"] for r in c2), 3),
                                           "GBps": round(nbytes2 / (full2 * 1e-3) / 1e9, 4),
                                           "per_shape": c2}
    # config 3: fused QKV (widths by seed) and fused gate-up (W3 2 x 11008) at M = 1
    qkv_bits = [int(b) for b in np.random.default_rng(0).choice([2, 3, 4], 3)]
    qkv = [make_weight(torch, 4096, 4096, b, s + 1, dev) for s, b in enumerate(qkv_bits)]
    res["config3_fused_qkv_m1"] = row(qkv, x1, sum(gemv_bytes(1, 4096, 4096, b) for b in qkv_bits), "GB/s", 1, 3)
    gu = [make_weight(torch, 11008, 4096, 3, 4, dev), make_weight(torch, 11008, 4096, 3, 5, dev)]
    res["config3_fused_gate_up_w3_m1"] = row(gu, x1, 2 * gemv_bytes(1, 4096, 11008, 3), "GB/s", 1, 3)
    del qkv, gu
    # config 4: the M = 1024 prefill GEMM, W4 4096 x 4096
    xg = randx(torch, 1024, 4096, 1, dev)
    res["config4_w4_gemm_m1024_4096x4096"] = row([w1], xg, 2.0 * 1024 * 4096 * 4096, "TFLOP/s")
    # config 5: one block of the Llama-2-7B stack at decode (bits of block 0 of the bitmap)
    bits0 = int(np.random.default_rng(0).choice([2, 3, 4], STACK_BLOCKS)[0])
    blk = [make_weight(torch, N, K, bits0, j, dev) for j, (_, N, K) in enumerate(STACK_LINEARS)]
    nb5 = sum(gemv_bytes(1, K, N, bits0) for _, N, K in STACK_LINEARS)
    hs = [host(w) for w in blk]
    xh, xi = randx(torch, 1, STACK_H, 1, "cpu").float(), randx(torch, 1, STACK_I, 2, "cpu").float()
    xin = [xi if K == STACK_I else xh for _, _, K in STACK_LINEARS]
    full5 = _median_ms(lambda: [x @ dequant(h).T for h, x in zip(hs, xin)], 1, 3)
    res["config5_stack_one_block_m1"] = {"dequant_matmul_ms": round(full5, 3), "bits": bits0,
                                         "step_estimate_ms": round(32 * full5, 1),
                                         "GBps": round(nb5 / (full5 * 1e-3) / 1e9, 4)}
    del blk, hs
    value = res["config2_w3_gemv_m1_layer_set"]["GBps"]
    return {"value": value, "unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port",
            "cpu_count": os.cpu_count(), "affinity": affinity, "torch_threads": torch.get_num_threads(),
            **res,
            "sample": "value = config 2 (the timed workload's metric) on one layer-set of the step (W3 GEMVs "
                      "4096x4096, 4096->11008, 11008->4096 at M=1): algorithmic bytes / dequant+matmul time.  "
                      "Rows for configs 1, 3, 4 and one block of config 5.  The oracle's restatement of "
                      "reference.py (unpack by code slot in torch int64 ops, fp32 dequant, torch fp32 matmul), "
                      "not reference.py itself; all on the affinity cores"}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="timed step + roofline only (no sweeps)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--sweeps", default="gemv,fused,probe,ablation,gemm,fp32,stack,model,producer",
                    help="comma-separated extra sweeps after the timed step (ignored with --quick); "
                         "'probe': a read-only streaming launch over each decode call's bytes; "
                         "also 'batched': batched decode at the library's own plans; 'dtypes': fp16 against "
                         "bf16 activations; 'splits': the split-K policy against every split request")
    ap.add_argument("--pmc-workload", nargs="?", const="gemv", choices=("gemv", "gemm", "bstream"),
                    help="run the fixed launch sequence of a counter pass and exit: gemv (default: the "
                         "W3 decode GEMV after a calibration copy), gemm (the M=1024 W4 prefill GEMM) or "
                         "bstream (the W3 batch-8 decode at 4096^2 and 11008->4096 after a calibration copy)")
    ap.add_argument("--trace-summary", nargs="+", metavar="FILE",
                    help="KERNEL_TRACE_CSV BENCH_JSON [UNTRACED_BENCH_JSON]: reduce a rocprofv3 kernel trace of a "
                         "bench run to the markdown tables under profiles/ (the default command's timed step, or "
                         "the batched sweep), with the tracer's inflation against an untraced run of the same "
                         "command when given, and exit")
    args = ap.parse_args()
    if args.trace_summary:
        trace_summary(*args.trace_summary, steps=args.steps, warmup=args.warmup)
        return
    if args.gpus != 1:
        print(f"bench.py: this build targets one MI355X; --gpus {args.gpus} is not supported "
              "(one GPU's share is the same kernel at a smaller N: column-parallel linears shard output rows, "
              "row-parallel ones K with an all-reduce of the fp32 partials)", file=sys.stderr)
        sys.exit(2)

    import torch
    from crispybits_kernels import ops
    if ops._CUDA is None:
        raise SystemExit(f"HIP library not built: {ops._IMPORT_ERROR}")
    C = ops._CUDA
    ops.set_backend("cuda")
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"device {torch.cuda.get_device_name(dev)}  CUs={C.sm_count()}")
    if args.pmc_workload == "gemm":
        pmc_workload_gemm(torch, ops, dev)
        return
    if args.pmc_workload == "bstream":
        pmc_workload_bstream(torch, ops, dev)
        return
    if args.pmc_workload:
        pmc_workload(torch, ops, dev)
        return

    # ---------------------------------------------------------------- timed workload
    bits = 3
    base = [make_weight(torch, N, K, bits, 0, dev) for K, N in SHAPES]
    layers = [[clone_weight(w) for w in base] for _ in range(LAYERS)]
    xs = [randx(torch, 1, K, 1, dev) for K, _ in SHAPES]
    torch.cuda.synchronize()
    pool_gb = sum(w.packed.numel() * 4 + w.scales.numel() * 4 for lw in layers for w in lw) / 1e9
    log(f"weights: {LAYERS} layers x 3 shapes, {pool_gb:.2f} GB packed")

    gate = Gate(torch)
    cand = [(1, 0), (1, 1), (1, 2), (2, 0), (None, 1)]
    cfg = [best_config(torch, C, ops, xs[s], [lw[s] for lw in layers], cand, gate, base[s]) for s in range(3)]
    log(f"per-shape (split_k, rho): {cfg}")

    def step_eager(keep=None):
        for li, lw in enumerate(layers):
            for s in range(3):
                y = ops.packed_linear(xs[s], lw[s], cfg[s][0], cfg[s][1])
                if keep is not None and li in (0, LAYERS - 1):
                    keep.append((li, s, y))

    step_eager()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    graph_outs = []
    with torch.cuda.graph(graph):
        step_eager(graph_outs)
    torch.cuda.synchronize()

    step_bytes = LAYERS * sum(gemv_bytes(1, K, N, bits) for K, N in SHAPES)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    # the graph that is timed: its outputs after the warm-up replays, against the oracle
    for li, s, y in graph_outs:
        K, N = SHAPES[s]
        gate.gemv(f"timed step graph, layer {li}, W{bits} M=1 {K}->{N} (split_k, rho)={cfg[s]}", y, xs[s], base[s])
    log(f"correctness gate: timed step passed ({gate.checks} checks)")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    value = step_bytes / (wall / args.steps) / 1e9
    log(f"timed: {args.steps} steps, {ms_per_step:.4f} ms/step, {value:.1f} GB/s")

    # ---------------------------------------------------------------- roofline of the dominant kernel
    # per shape: the 32 launches of that shape (one per layer copy) captured in a graph and
    # replayed between two events recorded on the stream the kernels run on; a launch's
    # duration is the replays' elapsed time over the launches, so it includes the gaps
    # between back-to-back kernels and can only understate the kernel's own rate
    total_ms, per_shape = 0.0, []
    for s, (K, N) in enumerate(SHAPES):
        us = graph_launch_us(torch, lambda s=s: [ops.packed_linear(xs[s], lw[s], cfg[s][0], cfg[s][1])
                                                 for lw in layers], LAYERS)
        total_ms += us * LAYERS * 1e-3
        per_shape.append({"K": K, "N": N, "bits": bits, "M": 1, "us": round(us, 3),
                          "GBps": round(gemv_bytes(1, K, N, bits) / (us * 1e-6) / 1e9, 1),
                          "split_k": cfg[s][0], "rho": cfg[s][1]})
    achieved = step_bytes / (total_ms * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic(),
                "achieved_step": round(value, 1), "frac_step": round(value / HBM_PEAK_GBS, 4),
                "kernel": "gemv_stream_kernel<GEMV, 3, 1> (W3 decode GEMV, M=1)",
                "bytes_per_launch_avg": round(step_bytes / (3 * LAYERS)),
                "avg_launch_us": round(total_ms * 1e3 / (3 * LAYERS), 3), "per_shape": per_shape,
                "timing": "HIP events on the launch stream around graph replays of 32 launches per shape; "
                          "achieved_step / frac_step: the step's algorithmic bytes over ms_per_step (wall clock "
                          "of the timed replays, gaps between kernels included)"}
    log(f"roofline: {achieved:.1f} GB/s = {achieved / HBM_PEAK_GBS:.1%} of HBM peak; {per_shape}")

    out = {"metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
           "config": {"workload": "W3 decode GEMV, M=1, 32 layers x {4096x4096, 4096->11008, 11008->4096}, "
                                  "g=128, one HIP graph per step", "bits": bits, "M": 1, "group_size": GS,
                      "shapes_KN": SHAPES, "layers": LAYERS, "weight_pool_GB": round(pool_gb, 3)},
           "roofline": roofline}

    del graph, graph_outs
    gate.clear()
    if not args.quick:
        todo = {w.strip() for w in args.sweeps.split(",") if w.strip()}
        if "gemv" in todo:
            out["gemv_sweep"] = gemv_sweep(torch, C, ops, dev, gate)
        if "batched" in todo:
            out["batched"] = batched_sweep(torch, C, ops, dev, gate)
        if "dtypes" in todo:
            out["dtypes"] = dtype_sweep(torch, C, ops, dev, gate)
        if "fused" in todo:
            out["fused"] = fused_sweep(torch, C, ops, dev, gate)
        if "probe" in todo:
            out["probe"] = probe_sweep(torch, C, dev, out.get("gemv_sweep"), out.get("fused"))
        if "ablation" in todo:
            out["ablation"] = ablation_sweep(torch, C, ops, dev, gate)
        if "splits" in todo:
            out["split_policy"] = split_sweep(torch, C, ops, dev, gate)
        if "gemm" in todo:
            out["gemm"] = gemm_sweep(torch, C, ops, dev, gate)
        if "fp32" in todo:
            out["fp32"] = fp32_sweep(torch, C, ops, dev, gate)
        if "stack" in todo:
            out["llama2_7b_stack"] = stack_sweep(torch, C, ops, dev, gate)
        if "model" in todo:
            try:
                out["llama2_7b_model"] = model_sweep(torch, dev)
            except Exception as e:              # reported in the line; the other legs stand
                log(f"llama2-7b model sweep failed: {e!r}")
                out["llama2_7b_model"] = {"error": repr(e)[:500]}
                torch.cuda.empty_cache()
        if "producer" in todo:
            out["producer"] = producer_sweep(torch, C, dev)
    out["correctness_checked"] = gate.record()
    if not args.no_cpu:
        log("cpu baseline ...")
        out["cpu_baseline"] = cpu_baseline(torch, dev, base, xs)
    print(json.dumps(out), flush=True)


def trace_summary(trace_csv, bench_json, untraced_json=None, steps=50, warmup=5):
    """Markdown tables of a rocprofv3 kernel trace of a bench run (needs no GPU).  With a
    `batched` sweep in the bench line: per sweep row, its 6 x copies consecutive bstream
    dispatches (eager run, warm replay, 4 timed replays; one kernel, grid and block checked) and
    the kernel durations of the timed replays.  Otherwise: the timed step, the first run of
    (warmup + steps) x 96 decode launches whose (kernel, grid, block) keys repeat with period 3,
    per shape over its last steps x 96 launches, and the kernel time per step against the line."""
    import csv
    import re
    rows = sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Start_Timestamp"]))
    line = json.loads(open(bench_json).read().strip().splitlines()[-1])
    key = lambda r: (r["Kernel_Name"], int(r["Grid_Size_X"]), int(r["Workgroup_Size_X"]))
    dur = lambda r: int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    name = lambda r: re.search(r"(gemv_\w+<[^>]*>)", r["Kernel_Name"]).group(1)
    if "batched" in line:
        b = [r for r in rows if re.search(r"gemv_(bstream|batch|reduce)", r["Kernel_Name"])]
        print("| bits | M | K -> N | kernel | K splits | workgroups x threads | launches | kernel avg ns (trace) "
              "| min ns | us per call (graph replays, traced run) |")
        print("|---|---|---|---|---|---|---|---|---|---|")
        i = 0
        for j in line["batched"]:
            part = b[i:i + 6 * j["copies"]]
            assert len({key(r) for r in part}) == 1 and len(part) == 6 * j["copies"], j
            t = [dur(r) for r in part[-4 * j["copies"]:]]
            print(f"| W{j['bits']} | {j['M']} | {j['K']} -> {j['N']} | `{name(part[0])}` | {j['splits']} | "
                  f"{int(part[0]['Grid_Size_X']) // int(part[0]['Workgroup_Size_X'])} x {part[0]['Workgroup_Size_X']} "
                  f"| {j['launches']} | {statistics.mean(t):.0f} | {min(t)} | {j['us']} |")
            i += 6 * j["copies"]
        assert i == len(b), (i, len(b))
        return
    if "gemm" in line and "gemv_sweep" not in line:
        gemm_trace_tables(rows, line, key, dur)
        return
    # the timed replays: the last run of steps x 96 decode launches whose (kernel, grid, block)
    # keys repeat with period 3 (the eager run and warm-up replays before it have the same keys;
    # the roofline's per-shape graphs after it do not)
    n = steps * 96
    for i in range(len(rows) - n, -1, -1):
        seg = rows[i:i + n]
        if all("gemv_stream_kernel" in r["Kernel_Name"] for r in seg) and \
                all(key(seg[j]) == key(seg[j % 3]) for j in range(n)):
            break
    else:
        raise SystemExit("timed region not found")
    # the roofline's first per-shape graph replays one key 32 times, and its first launches
    # continue the period: the timed run ends before the first two consecutive launches of one
    # key (inside the timed run every launch differs from the next)
    for p in range(i, min(i + n, len(rows) - 1)):
        if key(rows[p]) == key(rows[p + 1]):
            i = p - n
            break
    timed = rows[i:i + n]
    assert all(key(timed[j]) == key(timed[j % 3]) for j in range(n)) and len(timed) == n
    d = [dur(r) for r in timed]
    kms = sum(d) / steps / 1e6
    span = (int(timed[-1]["End_Timestamp"]) - int(timed[0]["Start_Timestamp"])) / steps / 1e6
    step_bytes = line["roofline"]["bytes_per_launch_avg"] * 96
    print(f"traced run: ms_per_step {line['ms_per_step']}, kernel time per step {kms:.4f} ms "
          f"({'<=' if kms <= line['ms_per_step'] else '>'} the traced ms_per_step), dispatch span per step "
          f"{span:.4f} ms, value {line['value']}, frac (events) {line['roofline']['frac']}, frac (trace) "
          f"{step_bytes / (kms * 1e-3) / 1e9 / HBM_PEAK_GBS:.4f}, avg launch us (events) "
          f"{line['roofline']['avg_launch_us']}, (trace) {sum(d) / len(d) / 1e3:.3f}")
    if untraced_json:
        u = json.loads(open(untraced_json).read().strip().splitlines()[-1])
        print(f"untraced run of the same command: ms_per_step {u['ms_per_step']}, frac (events) "
              f"{u['roofline']['frac']}, frac_step {u['roofline'].get('frac_step')}; tracer inflation of the "
              f"step (traced / untraced ms_per_step) {line['ms_per_step'] / u['ms_per_step']:.3f}; trace kernel "
              f"time per step / untraced ms_per_step {kms / u['ms_per_step']:.3f}")
    print("| shape (K -> N) | kernel | grid (threads) | block | launches | avg ns | min ns | max ns |")
    print("|---|---|---|---|---|---|---|---|")
    for sh, (K, N) in enumerate(SHAPES):
        ds = [dur(r) for r in timed[sh::3]]
        r0 = timed[sh]
        print(f"| {K} -> {N} | `{name(r0)}` | {r0['Grid_Size_X']} | {r0['Workgroup_Size_X']} | {len(ds)} | "
              f"{statistics.mean(ds):.0f} | {min(ds)} | {max(ds)} |")


def gemm_trace_tables(rows, line, key, dur):
    """Per row of a `--sweeps gemm` run (gemm_sweep's order), the kernel durations of its timed
    graph replays: a plain row makes 29 launches of one kernel and grid (the gate's call, the
    untimed call, the warm replay, 5 replays of 4), the last 20 timed; a gate-up row makes 22
    gate-up launches (the gate's call, then 3 + 3 + 5 x 3), the last 15 timed, then 42 plain
    GEMM launches for the two-GEMM sequence (6 + 6 + 5 x 6), the last 30 timed."""
    import itertools
    import re
    g = [r for r in rows if "gemm_f16_kernel" in r["Kernel_Name"]]
    runs = [list(v) for _, v in itertools.groupby(g, key=key)]
    tpl = lambda r: re.search(r"gemm_f16_kernel<([^>]*)>", r["Kernel_Name"]).group(1)
    print("| M | K | N | width | kernel | grid (threads) | block | launches timed | avg ns | min ns | max ns "
          "| TFLOP/s | graph-replay us (bench line) |")
    print("|---|---|---|---|---|---|---|---|---|---|---|---|---|")
    i = 0
    for j in line["gemm"]:
        gu = j.get("kind") == "gate_up"
        parts = [(runs[i], 22, 15), (runs[i + 1], 42, 30)] if gu else [(runs[i], 29, 20)]
        i += len(parts)
        for n, (run, total, timed) in enumerate(parts):
            assert len(run) == total, (j, len(run), total)
            t = [dur(r) for r in run[-timed:]]
            flop = 2.0 * j["M"] * j["K"] * (2 * j["N"][0] if gu and n == 0 else (j["N"][0] if gu else j["N"]))
            nn = f"2 x {j['N'][0]}" if gu and n == 0 else (f"{j['N'][0]} (x 2)" if gu else j["N"])
            us = j["us"] if n == 0 else j["two_gemms_and_mul_us"]
            print(f"| {j['M']} | {j['K']} | {nn} | W{j['bits']} | `gemm_f16_kernel<{tpl(run[0])}>` | "
                  f"{run[0]['Grid_Size_X']} | {run[0]['Workgroup_Size_X']} | {timed} | {statistics.mean(t):.0f} | "
                  f"{min(t)} | {max(t)} | {flop / (statistics.mean(t) * 1e-9) / 1e12:.0f} | {us} |")
    assert i == len(runs), (i, len(runs))


def read_traffic():
    """HBM bytes per launch of the timed W3 GEMV, averaged over the step's shapes, from
    the committed counter summary (a `traffic_bytes_per_launch: <int>` line)."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def pmc_workload(torch, ops, dev):
    """Launch sequence of the counter passes: the calibration copy (PMC_COPY_BYTES read and
    written by one device-to-device copy), then 8 copies of each W3 decode shape at M=1 with
    the timed step's defaults.  Dispatch order: copy, 8 x (4096,4096), 8 x (4096,11008),
    8 x (11008,4096)."""
    src = torch.empty(PMC_COPY_BYTES // 2, dtype=torch.float16, device=dev).normal_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    for K, N in SHAPES:
        base = make_weight(torch, N, K, 3, 0, dev)
        ws = [base] + [clone_weight(base) for _ in range(7)]
        x = randx(torch, 1, K, 1, dev)
        torch.cuda.synchronize()
        for w in ws:
            ops.packed_linear(x, w, 1, 1)
        torch.cuda.synchronize()
    log("pmc workload done")


ROTATE_BYTES = 1 << 30          # every GEMV sweep point streams at least this many distinct weight bytes


def copies_for(nbytes, least=8):
    """Weight copies whose total reaches ROTATE_BYTES, so no repeat is served by the 256 MB
    MALL or the 4 MB per-XCD L2."""
    return max(least, math.ceil(ROTATE_BYTES / nbytes))


def weight_bytes(w):
    return w.packed.numel() * 4 + w.scales.numel() * w.scales.element_size() * 2


def pmc_workload_bstream(torch, ops, dev):
    """Launch sequence of the batched decode counter passes: the calibration copy, then 8 copies
    each of the W3 batch-8 decode at 4096 x 4096 and at 11008 -> 4096 (the library's own plans).
    Dispatch order: copy, 8 x (4096, 4096), 8 x (11008, 4096)."""
    src = torch.empty(PMC_COPY_BYTES // 2, dtype=torch.float16, device=dev).normal_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    for K, N in ((4096, 4096), (11008, 4096)):
        base = make_weight(torch, N, K, 3, 0, dev)
        ws = [base] + [clone_weight(base) for _ in range(7)]
        x = randx(torch, 8, K, 1, dev)
        torch.cuda.synchronize()
        for w in ws:
            ops.packed_linear(x, w)
        torch.cuda.synchronize()
    log("pmc bstream workload done")


def pmc_workload_gemm(torch, ops, dev):
    """Launch sequence of the GEMM counter passes: 1 + 5 launches of the M=1024 W4 prefill
    GEMM at 4096 x 4096 (fp16 activations, g=128); the first warms the code and is dropped."""
    w = make_weight(torch, 4096, 4096, 4, 0, dev)
    x = randx(torch, 1024, 4096, 1, dev)
    torch.cuda.synchronize()
    for _ in range(6):
        ops.packed_linear(x, w)
    torch.cuda.synchronize()
    log("pmc gemm workload done")


def gemv_sweep(torch, C, ops, dev, gate):
    """W2/W3/W4 x M in {1,4,8,16} x shapes: µs per call (graph-replayed, a split call counts its
    combine launch) over >= 1 GiB of distinct weight copies per shape; every candidate plan checked
    against the oracle before it is timed."""
    rows = []
    for bits in (4, 3, 2):
        for s, (K, N) in enumerate(SHAPES):
            base = make_weight(torch, N, K, bits, 0, dev)
            ws = [base] + [clone_weight(base) for _ in range(copies_for(weight_bytes(base)) - 1)]
            for M in (1, 4, 8, 16):
                x = randx(torch, M, K, 1, dev)
                best = None
                for sk, rho in [(1, 1), (2, 1), (None, 1)]:
                    gate.gemv(f"gemv sweep W{bits} M={M} {K}->{N} split_k={sk} rho={rho}",
                              ops.packed_linear(x, ws[0], sk, rho), x, base)
                    us = graph_launch_us(torch, lambda: [ops.packed_linear(x, w, sk, rho) for w in ws], len(ws),
                                         replays=4)
                    if best is None or us < best[0]:
                        best = (us, sk, rho)
                us, sk, rho = best
                gbs = gemv_bytes(M, K, N, bits) / (us * 1e-6) / 1e9
                rows.append({"bits": bits, "M": M, "K": K, "N": N, "us": round(us, 3), "GBps": round(gbs, 1),
                             "pct_peak": round(100 * gbs / HBM_PEAK_GBS, 1), "split_k": sk, "rho": rho,
                             "copies": len(ws)})
                log(f"gemv W{bits} M={M} K={K} N={N}: {us:.2f} us {gbs:.0f} GB/s ({len(ws)} copies)")
            del ws, base
            gate.clear()
            torch.cuda.empty_cache()
    return rows


def probe_sweep(torch, C, dev, gemv_rows=None, fused=None):
    """The floor a single launch sets: `C.stream_probe` (one streaming kernel, every 16-byte
    piece read once) over the algorithmic bytes of each M = 1 decode call of the sweeps --
    W2/W3/W4 at the three shapes, fused QKV at the fused sweep's widths, fused gate-up W3 --
    graph-replayed over >= 1 GiB of distinct buffers like the GEMV rows, best of unroll in
    {1, 2, 4, 8, 16} pieces per thread x {256, 1024} threads per workgroup; `probe_us` reads and
    keeps nothing, `probe_store_us` also writes one word per workgroup after a workgroup
    reduction (as a decode workgroup ends).  Each row carries the decode call's own µs from the
    sweeps of the same run when they ran.  The first row is the launch floor: the same kernel
    with one 64-thread workgroup and one 16-byte piece, back to back in the graph, so nearly
    all of its time is the dispatch and the end-of-kernel fences every launch pays."""
    sink = torch.zeros(1024, dtype=torch.int32, device=dev)
    tiny = [torch.zeros(4, dtype=torch.int32, device=dev) for _ in range(64)]
    floor = graph_launch_us(torch, lambda: [C.stream_probe(t, 1, 64, True, sink) for t in tiny], len(tiny),
                            replays=4)
    rows = [{"case": "launch floor: one 64-thread workgroup, 16 bytes", "bits": None, "K": None, "N": None,
             "bytes": 16, "probe_store_us": round(floor, 3), "block": 64, "unroll": 1, "copies": len(tiny)}]
    log(f"probe launch floor: {floor:.2f} us per launch")
    meta = lambda N, K: N * math.ceil(K / GS) * 2 * 2                      # noqa: E731
    packed = lambda N, K, b: N * math.ceil(K / 32) * b * 4                # noqa: E731
    qkv_bits = [int(b) for b in (fused or {}).get("qkv", {}).get("bits", [4, 3, 3])]
    cases = [(f"W{b} {K}->{N}", b, K, N, gemv_bytes(1, K, N, b)) for b in (4, 3, 2) for K, N in SHAPES]
    cases.append(("fused QKV 4096->3x4096", qkv_bits, 4096, 3 * 4096,
                  sum(packed(4096, 4096, b) + meta(4096, 4096) for b in qkv_bits) + 4096 * 2 + 3 * 4096 * 2))
    cases.append(("fused gate-up 4096->2x11008", 3, 4096, 11008,
                  2 * (packed(11008, 4096, 3) + meta(11008, 4096)) + 4096 * 2 + 11008 * 2))
    gemv_us = {(r["bits"], r["K"], r["N"]): r["us"] for r in (gemv_rows or []) if r["M"] == 1}
    for name, b, K, N, nbytes in cases:
        pool = [torch.zeros((nbytes + 15) // 16 * 4, dtype=torch.int32, device=dev)
                for _ in range(copies_for(nbytes))]
        torch.cuda.synchronize()
        best = {}
        for store in (False, True):
            for unroll in (1, 2, 4, 8, 16):
                for block in (256, 1024):
                    us = graph_launch_us(torch, lambda: [C.stream_probe(t, unroll, block, store, sink) for t in pool],
                                         len(pool), replays=4)
                    if store not in best or us < best[store][0]:
                        best[store] = (us, unroll, block)
        us, unroll, block = best[False]
        row = {"case": name, "bits": b, "K": K, "N": N, "bytes": nbytes, "probe_us": round(us, 3),
               "probe_GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
               "probe_pct_peak": round(100 * nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 1),
               "unroll": unroll, "block": block, "probe_store_us": round(best[True][0], 3),
               "store_unroll": best[True][1], "store_block": best[True][2], "copies": len(pool)}
        if name.startswith("fused QKV"):
            call = (fused or {}).get("qkv", {}).get("us")
        elif name.startswith("fused gate-up"):
            call = (fused or {}).get("gate_up", {}).get("us")
        else:
            call = gemv_us.get((b, K, N))
        if call:
            row["call_us"] = call
            row["call_over_probe"] = round(call / us, 3)
        rows.append(row)
        log(f"probe {name}: {us:.2f} us ({row['probe_GBps']:.0f} GB/s, unroll {unroll}, block {block}), "
            f"with stores {best[True][0]:.2f} us"
            + (f"; the call {call:.2f} us" if call else ""))
        del pool
        torch.cuda.empty_cache()
    return rows


def batched_sweep(torch, C, ops, dev, gate):
    """Batched decode at the library's own plan (split_k=None, no candidate search): W3 and W4,
    M in {4, 8, 16} over the three shapes, µs per call graph-replayed over >= 1 GiB of weight
    copies, with the launch the plan makes (kernel family, K splits, workgroups, launches per
    call).  The launch sequence of the batched decode kernel-trace profile."""
    rows = []
    for bits in (3, 4):
        for K, N in SHAPES:
            base = make_weight(torch, N, K, bits, 0, dev)
            ws = [base] + [clone_weight(base) for _ in range(copies_for(weight_bytes(base)) - 1)]
            for M in (4, 8, 16):
                x = randx(torch, M, K, 1, dev)
                fam, splits, grid, threads, lds, launches = C.decode_plan(torch.float16, M, K, GS, N, bits, "gemv",
                                                                          1, 1)
                gate.gemv(f"batched W{bits} M={M} {K}->{N}", ops.packed_linear(x, ws[0]), x, base)
                us = graph_launch_us(torch, lambda: [ops.packed_linear(x, w) for w in ws], len(ws), replays=4)
                gbs = gemv_bytes(M, K, N, bits) / (us * 1e-6) / 1e9
                rows.append({"bits": bits, "M": M, "K": K, "N": N, "us": round(us, 3), "GBps": round(gbs, 1),
                             "pct_peak": round(100 * gbs / HBM_PEAK_GBS, 1), "kernel": fam, "splits": splits,
                             "workgroups": grid, "threads": threads, "launches": launches, "copies": len(ws)})
                log(f"batched W{bits} M={M} K={K} N={N}: {us:.2f} us ({fam}, P={splits}, {grid} workgroups)")
            del ws, base
            gate.clear()
            torch.cuda.empty_cache()
    return rows


def dtype_sweep(torch, C, ops, dev, gate):
    """fp16 against bf16 activations (scales, zeros and outputs of the same dtype, the same codes):
    W3 decode at M = 1 and 8 over the three shapes, graph-replayed over >= 1 GiB of weight copies,
    and the W3 prefill GEMM at M = 1024, with the kernel family each decode plan takes."""
    from dataclasses import replace
    rows = []
    for K, N in SHAPES:
        base = make_weight(torch, N, K, 3, 0, dev)
        n = copies_for(weight_bytes(base))
        for M in (1, 8, 1024):
            r = {"bits": 3, "M": M, "K": K, "N": N}
            for dt, tag in ((torch.float16, "fp16"), (torch.bfloat16, "bf16")):
                k = n if M <= 16 else 4
                ws = [replace(clone_weight(base), scales=base.scales.to(dt), zeros=base.zeros.to(dt)) for _ in range(k)]
                x = randx(torch, M, K, 1, dev).to(dt)
                y = ops.packed_linear(x, ws[0])
                if M <= 16:
                    gate.gemv(f"dtypes {tag} W3 M={M} {K}->{N}", y, x, ws[0])
                else:
                    gate.gemm(f"dtypes {tag} W3 M={M} {K}->{N}", y, x, ws[0])
                del y
                us = graph_launch_us(torch, lambda: [ops.packed_linear(x, w) for w in ws], len(ws), replays=4)
                r[tag + "_us"] = round(us, 3)
                if M <= 16:
                    r[tag + "_kernel"] = C.decode_plan(dt, M, K, GS, N, 3, "gemv", 1, 1)[0]
                    r[tag + "_GBps"] = round(gemv_bytes(M, K, N, 3) / (us * 1e-6) / 1e9, 1)
                else:
                    r[tag + "_TFLOPs"] = round(2 * M * N * K / (us * 1e-6) / 1e12, 1)
                del ws
                gate.clear()
                torch.cuda.empty_cache()
            log(f"dtypes W3 M={M} K={K} N={N}: fp16 {r['fp16_us']:.2f} us, bf16 {r['bf16_us']:.2f} us")
            rows.append(r)
        del base
    return rows


def fused_sweep(torch, C, ops, dev, gate):
    """Config 3 at M = 1: fused QKV (widths by seed) and fused gate-up (W3, 2 x 11008), µs per call
    graph-replayed over >= 1 GiB of weight copies."""
    import numpy as np
    res = {}
    qkv_bits = [int(b) for b in np.random.default_rng(0).choice([2, 3, 4], 3)]
    first = [make_weight(torch, 4096, 4096, b, s + 1, dev) for s, b in enumerate(qkv_bits)]
    n = copies_for(sum(weight_bytes(w) for w in first))
    sets = [first] + [[clone_weight(w) for w in first] for _ in range(n - 1)]
    x = randx(torch, 1, 4096, 1, dev)
    for name, y, w in zip("qkv", ops.fused_qkv(x, *first), first):
        gate.gemv(f"fused QKV ({name}, W{w.bits}) M=1", y, x, w)
    us = graph_launch_us(torch, lambda: [ops.fused_qkv(x, *ws) for ws in sets], len(sets), replays=4)
    nbytes = sum(gemv_bytes(1, 4096, 4096, b) for b in qkv_bits) - 2 * 4096 * 2
    res["qkv"] = {"bits": qkv_bits, "K": 4096, "N": [4096] * 3, "us": round(us, 3),
                  "GBps": round(nbytes / (us * 1e-6) / 1e9, 1), "copies": len(sets)}
    del sets, first
    g0 = make_weight(torch, 11008, 4096, 3, 4, dev)
    u0 = make_weight(torch, 11008, 4096, 3, 5, dev)
    n = copies_for(weight_bytes(g0) + weight_bytes(u0))
    pairs = [(g0, u0)] + [(clone_weight(g0), clone_weight(u0)) for _ in range(n - 1)]
    gate.check("fused gate-up W3 M=1", ops.fused_gate_up(x, g0, u0),
               gate.linear64(x, g0, act="silu") * gate.linear64(x, u0))
    gate.clear()
    us = graph_launch_us(torch, lambda: [ops.fused_gate_up(x, g, u) for g, u in pairs], len(pairs), replays=4)
    nbytes = 2 * gemv_bytes(1, 4096, 11008, 3) - 4096 * 2 - 11008 * 2
    res["gate_up"] = {"bits": 3, "K": 4096, "N": [11008, 11008], "us": round(us, 3),
                      "GBps": round(nbytes / (us * 1e-6) / 1e9, 1), "copies": len(pairs)}
    del pairs
    torch.cuda.empty_cache()
    log(f"fused: {res}")
    return res


# Shapes of the split-K policy sweep (K, N): the Llama-2-7B / 13B, Llama-3-8B and OPT widths,
# and narrow outputs down to 64 rows.
SPLIT_SWEEP_SHAPES = [(4096, 4096), (4096, 11008), (11008, 4096), (2560, 2560), (2560, 10240), (10240, 2560),
                      (2048, 2048), (2048, 8192), (8192, 2048), (5120, 5120), (5120, 13824), (13824, 5120),
                      (4096, 14336), (14336, 4096), (1024, 4096), (4096, 2048), (4096, 1024), (4096, 512),
                      (4096, 256), (4096, 128), (4096, 64), (11008, 256), (11008, 128), (14336, 256),
                      (28672, 512), (28672, 256)]


def split_sweep(torch, C, ops, dev, gate, batches=(1, 8)):
    """The split-K policy against every split request 1, 2, 3, 4, 6, 8 (W3, g = 128, fp16), at
    batch 1 and 8 over SPLIT_SWEEP_SHAPES: µs per call graph-replayed over >= 1 GiB of weight
    copies, the library's K splits for each request, and the policy's pick.  Each request's launch
    is checked against the oracle before it is timed."""
    rows = []
    for K, N in SPLIT_SWEEP_SHAPES:
        base = make_weight(torch, N, K, 3, 0, dev)
        ws = [base] + [clone_weight(base) for _ in range(copies_for(weight_bytes(base), least=4) - 1)]
        for M in batches:
            x = randx(torch, M, K, 1, dev)
            t, P = {}, {}
            for sk in (1, 2, 3, 4, 6, 8):
                gate.gemv(f"split sweep W3 M={M} {K}->{N} split_k={sk}", ops.packed_linear(x, ws[0], sk, 1), x, base)
                P[sk] = C.decode_plan(torch.float16, M, K, GS, N, 3, "gemv", sk, 1)[1]
                t[sk] = round(graph_launch_us(torch, lambda: [ops.packed_linear(x, w, sk, 1) for w in ws], len(ws),
                                              replays=6), 2)
            best = min(t, key=t.get)
            pol = ops._k_splits(None, 1, M, N, K, x)
            rows.append({"K": K, "N": N, "M": M, "us": t, "library_splits": P, "best_request": best,
                         "policy_request": pol, "policy_regret": round(t[pol] / t[best] - 1, 4),
                         "underfill_rule_request": ops.candidate_split_k(-(-M // ops.BATCH_TILE), N, ops.tile_n(),
                                                                         ops.sm_count(), 1)})
            log(f"split sweep W3 M={M} {K}->{N}: {t} best {best} policy {pol}")
        del ws, base
        gate.clear()
        torch.cuda.empty_cache()
    return rows


# The reference ablation's models (Kernel/scripts/_common.py MODELS): hidden, intermediate,
# heads, KV heads, family.
ABLATION_MODELS = {"llama2-7b": (4096, 11008, 32, 32, "llama"), "opt-2.7b": (2560, 10240, 32, 32, "opt")}


def ablation_sweep(torch, C, ops, dev, gate, bits=3):
    """The decode ablation of Kernel/scripts/ablation_decode.py:66-103 at M = 1, W3, for one block of
    Llama-2-7B and of OPT-2.7B: the block's projections unfused (gate and up as two GEMVs and a
    torch SiLU-multiply; fc1 then a torch ReLU), then with the projection fusion (fused QKV, fused
    gate-up, fc1 with the ReLU in the kernel), fixed K splits 2 / 4 / 8, the split-K policy
    (autotune's pick) and the exhaustive-grid oracle, beside dense fp16 (torch F.linear, i.e.
    hipBLASLt) on the same shapes.  The reference's rho rows have no counterpart: no launch here
    depends on rho (the kernels are not persistent), which the library's decode plan shows.  Each
    row is µs per block, graph-replayed over >= 1 GiB of block copies; every configuration is
    checked against the oracle before it is timed."""
    import torch.nn.functional as F
    from dataclasses import replace
    from crispybits_kernels.autotune import tune_gate_up, tune_gemv, tune_qkv
    out = {}
    for model, (H, I, nh, nkv, fam) in ABLATION_MODELS.items():
        opt = fam == "opt"
        hd = H // nh
        shapes = {"q": (nh * hd, H), "k": (nkv * hd, H), "v": (nkv * hd, H), "o": (H, H)}
        shapes.update({"fc1": (I, H), "fc2": (H, I)} if opt else {"gate": (I, H), "up": (I, H), "down": (H, I)})
        base = {}
        for seed, (name, (N, K)) in enumerate(shapes.items(), start=1):
            w = make_weight(torch, N, K, bits, seed, dev)
            if opt:
                g = torch.Generator().manual_seed(100 + seed)
                w = replace(w, bias=(torch.randn(N, generator=g) * 0.02).half().to(dev))
            base[name] = w
        block_bytes = sum(weight_bytes(w) for w in base.values())
        blocks = [base] + [{n: replace(clone_weight(w), bias=w.bias) for n, w in base.items()}
                           for _ in range(copies_for(block_bytes, least=2) - 1)]
        xh, xi = randx(torch, 1, H, 1, dev), randx(torch, 1, I, 2, dev)
        down = "fc2" if opt else "down"
        up_mod = "fc1" if opt else "gu"
        mods = ["qkv", "o", up_mod, down]

        def unfused(b, sk=lambda m: 1):
            outs = [ops.packed_linear(xh, b[n], sk(n), 1) for n in ("q", "k", "v", "o")]
            if opt:
                outs.append(torch.relu(ops.packed_linear(xh, b["fc1"], sk("fc1"), 1)))
            else:
                outs.append(F.silu(ops.packed_linear(xh, b["gate"], sk("gate"), 1)) *
                            ops.packed_linear(xh, b["up"], sk("up"), 1))
            outs.append(ops.packed_linear(xi, b[down], sk(down), 1))
            return outs

        def fused(b, sk=lambda m: 1):
            outs = list(ops.fused_qkv(xh, b["q"], b["k"], b["v"], sk("qkv"), 1))
            outs.append(ops.packed_linear(xh, b["o"], sk("o"), 1))
            if opt:
                outs.append(ops.packed_linear(xh, b["fc1"], sk("fc1"), 1, "relu"))
            else:
                outs.append(ops.fused_gate_up(xh, b["gate"], b["up"], sk("gu"), 1))
            outs.append(ops.packed_linear(xi, b[down], sk(down), 1))
            return outs

        def refs():
            w = base
            r = [gate.linear64(xh, w[n]) for n in ("q", "k", "v", "o")]
            if opt:
                r.append(torch.relu(gate.linear64(xh, w["fc1"]) + w["fc1"].bias.double().cpu()))
            else:
                r.append(gate.linear64(xh, w["gate"], act="silu") * gate.linear64(xh, w["up"]))
            r.append(gate.linear64(xi, w[down]))
            if opt:
                for i, n in enumerate(("q", "k", "v", "o")):
                    r[i] = r[i] + w[n].bias.double().cpu()
                r[5] = r[5] + w["fc2"].bias.double().cpu()
            return r

        ref = refs()
        names = ["q", "k", "v", "o", "fc1" if opt else "gate*up", down]

        def timed(tag, fn):
            for nm, y, r in zip(names, fn(base), ref):
                gate.check(f"ablation {model} W{bits} {tag}: {nm}", y, r)
            return graph_launch_us(torch, lambda: [fn(b) for b in blocks], len(blocks), replays=4)

        rows = [("1 base packed (unfused, P_K = 1)", timed("unfused", unfused)),
                ("2 + projection fusion", timed("fused", fused))]
        for pk in (2, 4, 8):
            rows.append((f"5 fixed split-K P_K = {pk}", timed(f"P_K={pk}", lambda b, pk=pk: fused(b, lambda m: pk))))

        def tune(m):
            it = dict(warmup=5, iters=10, exhaustive=True)
            if m == "qkv":
                return tune_qkv(xh, base["q"], base["k"], base["v"], **it)
            if m == "gu":
                return tune_gate_up(xh, base["gate"], base["up"], **it)
            return tune_gemv(xi if m == down else xh, base[m], act="relu" if m == "fc1" else None, **it)

        reports = {m: tune(m) for m in mods}
        pol = {m: r.best.split_k for m, r in reports.items()}
        orc = {m: r.oracle.split_k for m, r in reports.items()}
        rows.append(("6 split-K policy", timed("policy", lambda b: fused(b, lambda m: pol[m]))))
        rows.append(("7 oracle (exhaustive grid)", timed("oracle", lambda b: fused(b, lambda m: orc[m]))))
        gate.clear()

        dense = [{n: torch.randn(N, K, device=dev, dtype=torch.float16) * 0.02 for n, (N, K) in shapes.items()}
                 for _ in range(max(2, copies_for(sum(2 * N * K for N, K in shapes.values()), least=2)))]
        bias = {n: base[n].bias for n in shapes} if opt else {n: None for n in shapes}

        def fp16_block(d):
            for n in ("q", "k", "v", "o"):
                F.linear(xh, d[n], bias[n])
            if opt:
                torch.relu(F.linear(xh, d["fc1"], bias["fc1"]))
            else:
                F.silu(F.linear(xh, d["gate"])) * F.linear(xh, d["up"])
            F.linear(xi, d[down], bias[down])

        fp = graph_launch_us(torch, lambda: [fp16_block(d) for d in dense], len(dense), replays=4)
        del dense
        b0 = rows[0][1]
        out[model] = {
            "bits": bits, "M": 1, "group_size": GS, "block_copies": len(blocks),
            "rows": [{"step": n, "us": round(us, 2), "x_vs_base": round(b0 / us, 3), "x_vs_fp16": round(fp / us, 3)}
                     for n, us in rows],
            "fp16_dense_us": round(fp, 2),
            "policy_split_k": pol, "oracle_split_k": orc,
            "regret": {m: round(r.regret, 4) for m, r in reports.items()},
            "rho": "no launch depends on rho (non-persistent kernels)"}
        for n, us in rows:
            log(f"ablation {model}: {n:36s} {us:8.2f} us  {b0 / us:5.2f}x vs base  {fp / us:5.2f}x vs fp16")
        log(f"ablation {model}: fp16 dense {fp:.2f} us")
        del blocks, base
        torch.cuda.empty_cache()
    return out


def fp32_sweep(torch, C, ops, dev, gate):
    """fp32 activations (fp32 scales, zeros and outputs; the reference's T = float): the W3 decode
    at M in {1, 2, 4, 8} over the three shapes (the decode plan's kernel: the streaming kernel at
    batch 1, the batched streaming kernel at 2..8), graph-replayed over
    >= 1 GiB of weight copies, and the W4 prefill at M = 1024 (4096 x 4096) on the fp32 matrix-core
    GEMM, beside the fp16 prefill with the 16-bit matrix cores turned off (use_tensor_cores=False,
    the same fp32 kernel).  Every row checked against the oracle before it is timed."""
    from dataclasses import replace
    rows = []
    for K, N in SHAPES:
        base = make_weight(torch, N, K, 3, 0, dev)
        w32 = replace(base, scales=base.scales.float(), zeros=base.zeros.float())
        ws = [w32] + [clone_weight(w32) for _ in range(copies_for(weight_bytes(w32)) - 1)]
        for M in (1, 2, 4, 8):
            x = randx(torch, M, K, 1, dev).float()
            gate.gemv(f"fp32 decode W3 M={M} {K}->{N}", ops.packed_linear(x, ws[0]), x, w32)
            fam = C.decode_plan(torch.float32, M, K, GS, N, 3, "gemv", 1, 1)[0]
            us = graph_launch_us(torch, lambda: [ops.packed_linear(x, w) for w in ws], len(ws), replays=4)
            nbytes = N * math.ceil(K / 32) * 3 * 4 + N * math.ceil(K / GS) * 8 + M * K * 4 + M * N * 4
            gbs = nbytes / (us * 1e-6) / 1e9
            rows.append({"kind": "decode", "bits": 3, "M": M, "K": K, "N": N, "us": round(us, 3),
                         "GBps": round(gbs, 1), "pct_peak": round(100 * gbs / HBM_PEAK_GBS, 1), "kernel": fam})
            log(f"fp32 decode W3 M={M} {K}->{N}: {us:.2f} us {gbs:.0f} GB/s ({fam})")
        del ws, base, w32
        gate.clear()
        torch.cuda.empty_cache()
    w = make_weight(torch, 4096, 4096, 4, 0, dev)
    w32 = replace(w, scales=w.scales.float(), zeros=w.zeros.float())
    for tag, ww, x, tc in (("fp32", w32, randx(torch, 1024, 4096, 1, dev).float(), True),
                           ("fp16, use_tensor_cores=False", w, randx(torch, 1024, 4096, 1, dev), False)):
        y = ops.packed_linear(x, ww, use_tensor_cores=tc)
        rs = gate.rows(1024)
        gate.check(f"prefill {tag} W4 M=1024 4096^2", y, gate.linear64(x, ww, rs), rs)
        ws = [ww] + [clone_weight(ww) for _ in range(3)]
        us = graph_launch_us(torch, lambda: [ops.packed_linear(x, v, use_tensor_cores=tc) for v in ws], len(ws),
                             replays=3)
        tfs = 2.0 * 1024 * 4096 * 4096 / (us * 1e-6) / 1e12
        rows.append({"kind": "prefill", "x": tag, "bits": 4, "M": 1024, "K": 4096, "N": 4096, "us": round(us, 2),
                     "TFLOPs": round(tfs, 1), "pct_fp32_matrix_peak": round(100 * tfs / MFMA_F32_PEAK_TFS, 1)})
        log(f"prefill {tag} W4 M=1024 4096^2: {us:.1f} us {tfs:.1f} TFLOP/s")
        del ws, y
    gate.clear()
    torch.cuda.empty_cache()
    return rows


def producer_sweep(torch, C, dev):
    """The on-device quantizer + packer (cbk_quantize_pack) over the decode shapes' fp16
    weights, W2/W3/W4, g=128: kernel us per weight and its HBM rate counting the weight
    read once plus the packed words and fp16 scales/zeros written."""
    rows = []
    for K, N in SHAPES:
        g = torch.Generator(device=dev).manual_seed(7)
        W = (torch.randn(N, K, generator=g, device=dev) * 0.02).half()
        for bits in (4, 3, 2):
            run = lambda: [C.quantize_pack(W, bits, GS) for _ in range(8)]
            run()
            torch.cuda.synchronize()
            total, _ = timed_kernels(C, run, 8)
            us = total * 1e3 / 8
            nbytes = N * K * 2 + N * math.ceil(K / 32) * bits * 4 + N * math.ceil(K / GS) * 4
            gbs = nbytes / (us * 1e-6) / 1e9
            rows.append({"bits": bits, "K": K, "N": N, "us": round(us, 2), "GBps": round(gbs, 1),
                         "pct_peak": round(100 * gbs / HBM_PEAK_GBS, 1)})
        del W
    log(f"producer: {rows}")
    return rows


def gemm_sweep(torch, C, ops, dev, gate):
    """Config 4: the prefill GEMM at M in {1024, 2048}, µs per call graph-replayed over 4 weight
    copies (the weights are read once per 128-row tile either way; the activations dominate);
    every row checked against the oracle before it is timed."""
    rows = []
    for M in (1024, 2048):
        for K, N in SHAPES:
            x = randx(torch, M, K, 1, dev)
            for bits in (4, 3, 2):
                ws = [make_weight(torch, N, K, bits, 0, dev)]
                ws += [clone_weight(ws[0]) for _ in range(3)]
                gate.gemm(f"gemm W{bits} M={M} {K}->{N}", ops.packed_linear(x, ws[0]), x, ws[0])
                gate.clear()
                us = graph_launch_us(torch, lambda: [ops.packed_linear(x, w) for w in ws], len(ws), replays=5)
                tfs = 2.0 * M * N * K / (us * 1e-6) / 1e12
                rows.append({"M": M, "K": K, "N": N, "bits": bits, "us": round(us, 2), "TFLOPs": round(tfs, 1),
                             "pct_peak": round(100 * tfs / MFMA_F16_PEAK_TFS, 1)})
                log(f"gemm M={M} K={K} N={N} W{bits}: {us:.1f} us {tfs:.1f} TFLOP/s")
                del ws
    # the Llama-2-7B MLP's gate-up at the prefill batches: one launch (ops.fused_gate_up)
    # against the two GEMMs and the product it replaces, over 3 copies of the pair
    K, N = STACK_H, STACK_I
    for M in (1024, 2048):
        x = randx(torch, M, K, 1, dev)
        for bits in (4, 3, 2):
            g0, u0 = make_weight(torch, N, K, bits, 4, dev), make_weight(torch, N, K, bits, 5, dev)
            pairs = [(g0, u0)] + [(clone_weight(g0), clone_weight(u0)) for _ in range(2)]
            r = gate.rows(M)
            ref = gate.linear64(x, g0, r, round_w=x.dtype, act="silu") * gate.linear64(x, u0, r, round_w=x.dtype)
            gate.check(f"gemm gate-up W{bits} M={M}", ops.fused_gate_up(x, g0, u0), ref, r)
            gate.clear()

            def two():
                out = []
                for g, u in pairs:
                    y = C.packed_gemm(x, g.packed, g.scales, g.zeros, None, bits, K, 128, ops.ACT["silu"], True)
                    out.append(y.mul_(C.packed_gemm(x, u.packed, u.scales, u.zeros, None, bits, K, 128,
                                                    ops.ACT["none"], True)))
                return out

            us = graph_launch_us(torch, lambda: [ops.fused_gate_up(x, g, u) for g, u in pairs], len(pairs), replays=5)
            us2 = graph_launch_us(torch, two, len(pairs), replays=5)
            tfs = 2.0 * M * 2 * N * K / (us * 1e-6) / 1e12
            rows.append({"M": M, "K": K, "N": [N, N], "bits": bits, "kind": "gate_up", "us": round(us, 2),
                         "TFLOPs": round(tfs, 1), "pct_peak": round(100 * tfs / MFMA_F16_PEAK_TFS, 1),
                         "two_gemms_and_mul_us": round(us2, 2)})
            log(f"gemm gate-up M={M} W{bits}: {us:.1f} us (two GEMMs + mul {us2:.1f} us)")
            del pairs, g0, u0
    return rows


STACK_H, STACK_I, STACK_BLOCKS = 4096, 11008, 32
STACK_LINEARS = [("q", STACK_H, STACK_H), ("k", STACK_H, STACK_H), ("v", STACK_H, STACK_H), ("o", STACK_H, STACK_H),
                 ("gate", STACK_I, STACK_H), ("up", STACK_I, STACK_H), ("down", STACK_H, STACK_I)]   # (name, N, K)
PREFILL_M = 2048


def stack_energy(torch, gr, gr16, seconds=4.0):
    """Energy per decode step of the graph-captured stack and of its fp16 dense twin, from
    the GPU's energy accumulator over a steady back-to-back run (crispybits_kernels.energy;
    the paper's energy-per-request metric restricted to the linear stack).  None when
    AMD-SMI is not usable on the box."""
    from crispybits_kernels.energy import AMDSMIPowerSampler, steady_energy
    try:
        sampler = AMDSMIPowerSampler(torch.cuda.current_device())
    except RuntimeError as e:
        log(f"energy: skipped ({e})")
        return None
    try:
        out = {}
        for name, g in (("packed", gr), ("fp16_dense", gr16)):
            m = steady_energy(g.replay, sampler, seconds=seconds, synchronize=torch.cuda.synchronize)
            out[name] = {"J_per_step": round(m.joules, 4), "mean_W": round(m.mean_watts, 1),
                         "steps": m.samples, "counter_window_s": round(m.seconds, 3)}
        out["energy_ratio_fp16_over_packed"] = round(out["fp16_dense"]["J_per_step"] / out["packed"]["J_per_step"], 2)
        out["method"] = ("AMD-SMI energy accumulator between two counter updates inside a ~4 s back-to-back "
                         "run of the step graph; J/step = mean W x wall time per step")
        log(f"energy: {out}")
        return out
    except RuntimeError as e:
        log(f"energy: failed ({e})")
        return None
    finally:
        sampler.close()


def stack_check(torch, ops, gate, blocks, bitmap, xh, xi, Xh, Xi):
    """The stack's launch configurations against the oracle: the first block of each bit width
    (every (shape, mode, bits) plan a step makes), at decode and at the prefill rows."""
    firsts = sorted({b: i for i, b in reversed(list(enumerate(bitmap)))}.values())
    for i in firsts:
        b = blocks[i]
        tag = f"stack block {i} (W{bitmap[i]})"
        for nm, y in zip("qkv", ops.fused_qkv(xh, b["q"], b["k"], b["v"])):
            gate.gemv(f"{tag} decode fused QKV {nm}", y, xh, b[nm])
        gate.gemv(f"{tag} decode o", ops.packed_linear(xh, b["o"]), xh, b["o"])
        gate.check(f"{tag} decode fused gate-up", ops.fused_gate_up(xh, b["gate"], b["up"]),
                   gate.linear64(xh, b["gate"], act="silu") * gate.linear64(xh, b["up"]))
        gate.gemv(f"{tag} decode down", ops.packed_linear(xi, b["down"]), xi, b["down"])
        for nm, y in zip("qkv", ops.fused_qkv(Xh, b["q"], b["k"], b["v"])):
            gate.gemm(f"{tag} prefill QKV {nm}", y, Xh, b[nm])
        gate.gemm(f"{tag} prefill o", ops.packed_linear(Xh, b["o"]), Xh, b["o"])
        rows = gate.rows(Xh.shape[0])
        ref = (gate.linear64(Xh, b["gate"], rows, round_w=Xh.dtype, act="silu")
               * gate.linear64(Xh, b["up"], rows, round_w=Xh.dtype))
        gate.check(f"{tag} prefill gate-up", ops.fused_gate_up(Xh, b["gate"], b["up"]), ref, rows)
        gate.gemm(f"{tag} prefill down", ops.packed_linear(Xi, b["down"]), Xi, b["down"])
        gate.clear()
    log(f"correctness gate: stack blocks {firsts} passed")


def stack_sweep(torch, C, ops, dev, gate, steps=20):
    """Config 5: the Llama-2-7B linear stack at decode (M = 1), 32 blocks, bits per block
    from default_rng(0).choice([2, 3, 4], 32); block i, linear j weights from a device
    generator seeded 1000*i + j (quantized and packed on the GPU by the HIP producer).  A step is, per block,
    fused QKV, o, fused gate-up and down (ablation_decode.py:48-56); eager and as one
    captured HIP graph, against the same stack as dense fp16 F.linear (the dequantized
    weights) in a graph.  Inputs are fixed activations; the rest of the model (attention,
    norms) is not part of the path."""
    import numpy as np
    import torch.nn.functional as F
    from crispybits_kernels.ops import PackedLinearWeight
    from crispybits_kernels import _C
    from crispybits_kernels.reference import dequantize, quantize_pack
    bitmap = [int(b) for b in np.random.default_rng(0).choice([2, 3, 4], STACK_BLOCKS)]
    blocks, dense = [], []
    for i, bits in enumerate(bitmap):
        pb, db = {}, {}
        for j, (nm, N, K) in enumerate(STACK_LINEARS):
            g = torch.Generator(device=dev).manual_seed(1000 * i + j)
            W = torch.randn(N, K, generator=g, device=dev) * 0.02
            packed, s, z = quantize_pack(W, bits, GS)
            pb[nm] = PackedLinearWeight(packed, s, z, bits, GS, K, N)
            db[nm] = dequantize(_C.unpack_codes(packed, bits, K), s.float(), z.float(), GS).half()
            del W
        blocks.append(pb)
        dense.append(db)
    torch.cuda.synchronize()
    xh = randx(torch, 1, STACK_H, 1, dev)
    xi = randx(torch, 1, STACK_I, 2, dev)
    stack_check(torch, ops, gate, blocks, bitmap, xh, xi, randx(torch, PREFILL_M, STACK_H, 3, dev),
                randx(torch, PREFILL_M, STACK_I, 4, dev))
    packed_gb = sum(w.packed.numel() * 4 + w.scales.numel() * 4 for b in blocks for w in b.values()) / 1e9
    step_bytes = sum(gemv_bytes(1, K, N, b["q"].bits) for b in blocks for _, N, K in STACK_LINEARS)

    def step():
        for b in blocks:
            ops.fused_qkv(xh, b["q"], b["k"], b["v"])
            ops.packed_linear(xh, b["o"])
            ops.fused_gate_up(xh, b["gate"], b["up"])
            ops.packed_linear(xi, b["down"])

    def step_fp16():
        for d in dense:
            for nm in ("q", "k", "v", "o"):
                F.linear(xh, d[nm])
            F.silu(F.linear(xh, d["gate"])) * F.linear(xh, d["up"])
            F.linear(xi, d["down"])

    def wall(fn, n):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n

    def graphed(fn):
        fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            fn()
        torch.cuda.synchronize()
        return gr

    eager = wall(step, 5)
    gr = graphed(step)
    graph_t = wall(gr.replay, steps)
    kern_ms, durs = timed_kernels(C, step, 4 * STACK_BLOCKS + 64)
    gr16 = graphed(step_fp16)
    fp16_t = wall(gr16.replay, steps)
    energy = stack_energy(torch, gr, gr16)
    del gr, gr16

    # prefill leg: the same 32 blocks at M = 2048 (every linear on the prefill GEMM; fused QKV
    # as three GEMMs, fused gate-up as two GEMMs and their product), one graph per step
    Xh = randx(torch, PREFILL_M, STACK_H, 3, dev)
    Xi = randx(torch, PREFILL_M, STACK_I, 4, dev)

    def prefill():
        for b in blocks:
            ops.fused_qkv(Xh, b["q"], b["k"], b["v"])
            ops.packed_linear(Xh, b["o"])
            ops.fused_gate_up(Xh, b["gate"], b["up"])
            ops.packed_linear(Xi, b["down"])

    def prefill_fp16():
        for d in dense:
            for nm in ("q", "k", "v", "o"):
                F.linear(Xh, d[nm])
            F.silu(F.linear(Xh, d["gate"])) * F.linear(Xh, d["up"])
            F.linear(Xi, d["down"])

    flops = 2.0 * PREFILL_M * sum(N * K for _, N, K in STACK_LINEARS) * len(blocks)
    gp = graphed(prefill)
    pre_t = wall(gp.replay, 3)
    del gp
    gp16 = graphed(prefill_fp16)
    pre16_t = wall(gp16.replay, 3)
    del gp16, Xh, Xi
    prefill_res = {"M": PREFILL_M, "TFLOP_per_step": round(flops / 1e12, 3),
                   "graph_ms_per_step": round(pre_t * 1e3, 3), "TFLOPs": round(flops / pre_t / 1e12, 1),
                   "pct_peak": round(100 * flops / pre_t / 1e12 / MFMA_F16_PEAK_TFS, 1),
                   "fp16_dense_graph_ms_per_step": round(pre16_t * 1e3, 3),
                   "speedup_vs_fp16": round(pre16_t / pre_t, 3)}
    log(f"llama2-7b stack prefill: {prefill_res}")
    dense_gb = sum(t.numel() * 2 for d in dense for t in d.values()) / 1e9
    res = {"workload": "Llama-2-7B linear stack, decode M=1, 32 blocks x (fused QKV, o, fused gate-up, down)",
           "bitmap": bitmap, "mean_bits": round(float(np.mean(bitmap)), 3), "packed_GB": round(packed_gb, 3),
           "launches_per_step": len(durs), "eager_us_per_step": round(eager * 1e6, 1),
           "graph_us_per_step": round(graph_t * 1e6, 1), "kernel_us_per_step": round(kern_ms * 1e3, 1),
           "GBps_graph": round(step_bytes / graph_t / 1e9, 1),
           "fp16_dense_GB": round(dense_gb, 3), "fp16_graph_us_per_step": round(fp16_t * 1e6, 1),
           "speedup_vs_fp16": round(fp16_t / graph_t, 2), "energy": energy, "prefill": prefill_res}
    log(f"llama2-7b stack: {res}")
    del blocks, dense
    torch.cuda.empty_cache()
    return res


def model_sweep(torch, dev, steps=20, prompt_len=32):
    """Config 5 through the integration glue: an HF LlamaForCausalLM with Llama-2-7B dimensions
    (32 blocks, hidden 4096, intermediate 11008, 32 heads, random init), written with the config-5
    bitmap (write_packed_dir(bitmap=...), GPU producer) and installed with
    install_bitmap(fuse=True, fuse_rope=True) (integration.py:201-218 interface).  One decode
    step over a static KV cache is captured as a HIP graph and replayed; the same model with every
    block linear replaced by its dequantized fp16 weight is captured the same way.  Reports µs per
    step of both and the relative difference of their logits."""
    import copy
    import shutil
    import tempfile
    import numpy as np
    import transformers
    from crispybits_kernels import _C
    from crispybits_kernels.integration import _blocks, install_bitmap
    from crispybits_kernels.reference import dequantize, pack_linear_dict, write_packed_dir
    bitmap = [int(b) for b in np.random.default_rng(0).choice([2, 3, 4], STACK_BLOCKS)]
    cfg = transformers.LlamaConfig(hidden_size=STACK_H, intermediate_size=STACK_I, num_hidden_layers=STACK_BLOCKS,
                                   num_attention_heads=32, num_key_value_heads=32, vocab_size=32000,
                                   max_position_embeddings=512)
    torch.manual_seed(0)
    t0 = time.perf_counter()
    with torch.device(dev):
        base = transformers.LlamaForCausalLM(cfg).half().eval()
    tmp = tempfile.mkdtemp(prefix="cbk_model_", dir="/tmp")
    try:
        write_packed_dir(base, tmp, group_size=GS, dtype=torch.float16, bitmap=bitmap)
        ref = copy.deepcopy(base)
        with torch.no_grad():
            for block, bits in zip(_blocks(ref), bitmap):
                for _, m in block.named_modules():
                    if isinstance(m, torch.nn.Linear):
                        d = pack_linear_dict(m.weight.detach(), bits, GS, None, torch.float16)
                        q = _C.unpack_codes(d["packed"].to(dev), bits, m.in_features)
                        m.weight.copy_(dequantize(q, d["scales"].to(dev).float(), d["zeros"].to(dev).float(),
                                                  GS).half())
        t1 = time.perf_counter()
        model = install_bitmap(base, tmp, bitmap, device=dev, dtype=torch.float16, fuse=True, fuse_rope=True)
        install_s = time.perf_counter() - t1
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    prompt = torch.randint(0, 32000, (1, prompt_len), generator=torch.Generator().manual_seed(1)).to(dev)

    def captured(m):
        """Decode steps of m as one captured graph.  HF's StaticLayer writes each update at its
        own device counter and advances it in place (cache_position is not read for the
        write), so the step advances its position buffer the same way: the warm-up and every
        replay decode the next slot, as a generation loop does.  The cache holds the prompt,
        the warm-up and every replay, and each replay is checked to stay inside it."""
        slots = prompt_len + steps + 8
        cache = transformers.StaticCache(config=cfg, max_cache_len=slots)
        with torch.no_grad():
            m(prompt, past_key_values=cache, cache_position=torch.arange(prompt_len, device=dev), use_cache=True)
        tok = prompt[:, -1:].clone()
        pos = torch.tensor([prompt_len], device=dev)

        def step():
            logits = m(tok, past_key_values=cache, cache_position=pos, use_cache=True).logits[:, -1]
            pos.add_(1)
            return logits

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.no_grad(), torch.cuda.stream(side):
            step()                                        # slot prompt_len
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(g):
            logits = step()
        written = prompt_len + 1
        if written + 1 + steps > slots:
            raise RuntimeError("decode replays would run past the static cache")
        g.replay()                                        # slot prompt_len + 1
        torch.cuda.synchronize()
        first = logits.float().clone()
        t = time.perf_counter()
        for _ in range(steps):
            g.replay()
        torch.cuda.synchronize()
        elapsed = (time.perf_counter() - t) / steps
        del g
        return elapsed, first

    packed_t, packed_logits = captured(model)
    fp16_t, fp16_logits = captured(ref)
    diff = ((packed_logits - fp16_logits).abs().max() / fp16_logits.abs().max()).item()
    res = {"workload": "HF LlamaForCausalLM, Llama-2-7B dimensions (32 blocks, random init), config-5 bitmap, "
                       "install_bitmap(fuse=True, fuse_rope=True); one decode step (M=1) over a static KV cache "
                       f"after a {prompt_len}-token prompt, as a HIP graph",
           "bitmap": bitmap, "packed_graph_us_per_step": round(packed_t * 1e6, 1),
           "fp16_dequantized_graph_us_per_step": round(fp16_t * 1e6, 1),
           "speedup_vs_fp16": round(fp16_t / packed_t, 3), "logits_rel_diff_vs_dequantized_fp16": round(diff, 5),
           "build_s": round(t1 - t0, 1), "install_s": round(install_s, 1)}
    log(f"llama2-7b model: {res}")
    del model, ref, base
    torch.cuda.empty_cache()
    return res


if __name__ == "__main__":
    main()
