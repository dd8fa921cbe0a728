"""Host logic of crispybits_kernels (ops / io / autotune / integration) on the CPU,
with the oracle injected as the backend (the ``emu`` fixture).  Mirrors the
reference's emulator-parametrised tests (Kernel/tests/test_correctness.py,
test_integration.py); the GPU parity tests run the same API on the HIP kernels."""
import copy

import pytest
import torch

from crispybits_kernels import (apply_rope_reference, candidate_split_k, fused_gate_up, fused_qkv, new_workspace,
                                packed_linear, permute_for_rope, sm_count, tile_n, ops)
from crispybits_kernels.io import from_packed_dict
from crispybits_kernels.reference import dequantized_weight, pack_linear_dict

TOL = {torch.float16: 3e-3, torch.bfloat16: 2e-2, torch.float32: 1e-4}


def make(n, k, bits, dtype, device, bias=False, seed=0, gs=128):
    g = torch.Generator().manual_seed(seed)
    W = torch.randn(n, k, generator=g) * 0.05
    b = torch.randn(n, generator=g) * 0.1 if bias else None
    d = pack_linear_dict(W, bits, gs, b, dtype)
    return from_packed_dict(d, device, dtype), dequantized_weight(d).to(device), (
        None if b is None else d["bias"].float().to(device))


def ref_linear(x, Wd, bd, act=None):
    y = x.float() @ Wd.T
    if bd is not None:
        y = y + bd
    if act == "relu":
        y = torch.relu(y)
    elif act == "silu":
        y = torch.nn.functional.silu(y)
    return y


def close(y, ref, dtype):
    err = (y.float() - ref).abs().max().item()
    scale = ref.abs().max().item() + 1e-6
    assert err / scale < TOL[dtype], f"rel err {err / scale:.2e}"


@pytest.mark.parametrize("M", [1, 3, 8, 9, 20])
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_packed_linear_routes_and_reshapes(emu, M, bits):
    w, Wd, bd = make(48, 200, bits, torch.float32, emu, bias=True)
    x = torch.randn(M, 200)
    y = packed_linear(x, w, act="relu")
    close(y, ref_linear(x, Wd, bd, "relu"), torch.float32)
    x3 = torch.randn(2, M, 200)
    assert packed_linear(x3, w).shape == (2, M, 48)


def test_decode_threshold_boundary(emu, monkeypatch):
    w, Wd, _ = make(32, 128, 4, torch.float32, emu)
    calls = []
    for name in ("packed_gemv", "packed_gemm"):
        fn = getattr(ops._C, name)
        monkeypatch.setattr(ops._C, name, lambda *a, _fn=fn, _n=name: (calls.append(_n), _fn(*a))[1])
    packed_linear(torch.randn(ops.DECODE_THRESHOLD, 128), w)
    packed_linear(torch.randn(ops.DECODE_THRESHOLD + 1, 128), w)
    assert calls == ["packed_gemv", "packed_gemm"]


def test_fused_gate_up_decode_and_prefill(emu):
    g, Gd, _ = make(96, 256, 3, torch.float32, emu, seed=1)
    u, Ud, _ = make(96, 256, 3, torch.float32, emu, seed=2)
    for M in (1, 12, ops.DECODE_THRESHOLD + 4):
        x = torch.randn(M, 256)
        ref = torch.nn.functional.silu(x @ Gd.T) * (x @ Ud.T)
        close(fused_gate_up(x, g, u, 2, 1), ref, torch.float32)
    g2, _, _ = make(96, 256, 2, torch.float32, emu)
    with pytest.raises(ValueError):
        fused_gate_up(torch.randn(1, 256), g2, u)


def test_fused_gate_up_prefill_on_a_seven_function_backend(emu):
    """A backend with only the reference's seven _C functions (its emulator, say) takes the
    two-GEMM prefill sequence; the result equals the one-call path of this package's oracle."""
    import types
    from oracle import emulator
    g, _, _ = make(96, 256, 4, torch.float16, emu, seed=1)
    u, _, _ = make(96, 256, 4, torch.float16, emu, seed=2)
    x = torch.randn(ops.DECODE_THRESHOLD + 3, 256).half()
    full = fused_gate_up(x, g, u)
    seven = types.SimpleNamespace(**{n: getattr(emulator, n) for n in (
        "packed_gemv", "packed_gemm", "fused_gate_up", "fused_qkv", "sm_count", "tile_n", "max_rho",
        "decode_plan")})
    ops.set_backend(seven)
    try:
        assert torch.equal(fused_gate_up(x, g, u), full)
    finally:
        ops.set_backend(emulator)


def _rope_tables(M, head_dim, device):
    pos = torch.randint(0, 2048, (M,)).float()
    inv = 1.0 / (10000 ** (torch.arange(0, head_dim, 2).float() / head_dim))
    f = pos[:, None] * inv[None]
    emb = torch.cat([f, f], -1)
    return emb.cos().to(device), emb.sin().to(device)


@pytest.mark.parametrize("M", [1, 3, 12])
@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("bits", [(3, 3, 3), (4, 2, 3)])
def test_fused_qkv_gqa(emu, M, rope, bits):
    K, nq, nkv, hd = 256, 4, 2, 64
    q, Qd, qb = make(nq * hd, K, bits[0], torch.float32, emu, True, 1)
    k, Kd, kb = make(nkv * hd, K, bits[1], torch.float32, emu, True, 2)
    v, Vd, vb = make(nkv * hd, K, bits[2], torch.float32, emu, False, 3)
    q, k = permute_for_rope(q, hd), permute_for_rope(k, hd)
    x = torch.randn(M, K)
    rq, rk, rv = ref_linear(x, Qd, qb), ref_linear(x, Kd, kb), ref_linear(x, Vd, vb)
    r = None
    if rope:
        cos, sin = _rope_tables(M, hd, emu)
        rq, rk = apply_rope_reference(rq, cos, sin, hd), apply_rope_reference(rk, cos, sin, hd)
        r = (cos, sin, hd)
    oq, ok, ov = fused_qkv(x, q, k, v, 2, 1, rope=r)
    close(oq, rq, torch.float32); close(ok, rk, torch.float32); close(ov, rv, torch.float32)


def test_rope_requires_permuted_weights(emu):
    q, _, _ = make(256, 256, 3, torch.float32, emu)
    x = torch.randn(1, 256)
    cos, sin = _rope_tables(1, 128, emu)
    with pytest.raises(ValueError):
        fused_qkv(x, q, q, q, rope=(cos, sin, 128))
    with pytest.raises(ValueError):
        packed_linear(x, permute_for_rope(q, 128))
    with pytest.raises(ValueError):
        permute_for_rope(permute_for_rope(q, 128), 64)


def test_policy_rule(emu):
    S, bn = sm_count(), tile_n()
    assert candidate_split_k(1, bn * 4, bn, S, 1) == max(1, -(-S // 4))
    assert candidate_split_k(64, 4096, bn, S, 1) == 1
    assert candidate_split_k(1, 10 ** 6, bn, S, 1) == 1
    assert candidate_split_k(1, bn, bn, S, 2, max_split=8) == 8
    # a requested split clamps to the chunk count; split_k=None takes the policy, which
    # requests no split on this GPU at any shape, rho or batch (and respects max_split)
    x = torch.empty(0)
    assert ops._k_splits(5, 1, 1, 64, 4096, x) == 5
    assert ops._k_splits(99, 1, 1, 64, 100, x) == 4            # ceil(100 / 32) chunks
    for batch, v_rows, k, rho in ((1, 64, 64, 1), (1, 512, 4096, 1), (8, 256, 28672, 2), (16, 11008, 4096, 4)):
        assert ops._k_splits(None, rho, batch, v_rows, k, x) == ops.POLICY_SPLIT_K == 1
    assert ops.policy_split_k(1, 64, 4096, 1, max_split=1) == 1


def test_workspace_contract(emu):
    w, Wd, _ = make(512, 256, 3, torch.float32, emu)
    ws = new_workspace(emu)
    x = torch.randn(1, 256)
    for pk, rho in [(1, 1), (4, 2), (1, 0), (7, 1)]:
        close(packed_linear(x, w, pk, rho, workspace=ws), ref_linear(x, Wd, None), torch.float32)
    assert ws.tolist() == [0, 0]
    ws[0] = 3
    with pytest.raises(AssertionError):
        packed_linear(x, w, 1, 1, workspace=ws)


def test_set_backend_names():
    with pytest.raises(ValueError):
        ops.set_backend("nonsense")
    with pytest.raises(RuntimeError):
        ops.set_backend("emulator")


def test_autotune_report_on_emulator(emu):
    from crispybits_kernels import tune_gemv
    w, _, _ = make(64, 256, 4, torch.float32, emu)
    rep = tune_gemv(torch.randn(1, 256), w, warmup=0, iters=1, exhaustive=True)
    assert rep.best in rep.results and rep.oracle in rep.results
    assert rep.regret >= 0
    assert all(1 <= r.split_k <= 8 for r in rep.results)


# ---------------------------------------------------------------- HF integration (tiny models)

transformers = pytest.importorskip("transformers")

from crispybits_kernels import FusedLlamaMLP, FusedQKV, install_bitmap, tune_model  # noqa: E402
from crispybits_kernels.integration import _blocks  # noqa: E402
from crispybits_kernels.reference import write_packed_dir  # noqa: E402


def _dequantize_model_(model, bitmap):
    for block, bits in zip(_blocks(model), bitmap):
        for _, m in block.named_modules():
            if isinstance(m, torch.nn.Linear):
                d = pack_linear_dict(m.weight.detach().float().cpu(), bits, 128, None, torch.float16)
                m.weight.data.copy_(dequantized_weight(d).to(m.weight))


def _tiny(kind):
    if kind == "llama":
        cfg = transformers.LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=3,
                                       num_attention_heads=4, num_key_value_heads=2, vocab_size=512)
        m = transformers.LlamaForCausalLM(cfg)
        with torch.no_grad():
            for blk in _blocks(m):
                blk.self_attn.q_proj.weight.mul_(8.0)
                blk.self_attn.k_proj.weight.mul_(8.0)
        return m
    cfg = transformers.OPTConfig(hidden_size=256, ffn_dim=512, num_hidden_layers=3, num_attention_heads=4,
                                 vocab_size=512, word_embed_proj_dim=256)
    return transformers.OPTForCausalLM(cfg)


@pytest.mark.parametrize("kind,fuse,fuse_rope", [("llama", False, False), ("llama", True, False),
                                                 ("llama", True, True), ("opt", True, True)])
def test_model_matches_dequantized(emu, tmp_path, kind, fuse, fuse_rope):
    torch.manual_seed(0)
    dtype = torch.float32
    base = _tiny(kind).to(dtype).eval()
    bitmap = [4, 2, 3]
    write_packed_dir(base, tmp_path, bits_options=(2, 3, 4), dtype=dtype)
    ref = copy.deepcopy(base)
    _dequantize_model_(ref, bitmap)
    model = install_bitmap(copy.deepcopy(base), tmp_path, bitmap, device="cpu", dtype=dtype, fuse=fuse,
                           fuse_rope=fuse_rope)
    if fuse and kind == "llama":
        owners = [m for m in model.modules() if isinstance(m, FusedQKV)]
        assert owners and any(isinstance(m, FusedLlamaMLP) for m in model.modules())
        assert all(bool(o.rope_head_dim) == fuse_rope for o in owners)
    if fuse:
        tune_model(model, iters=1, warmup=0, dtype=dtype)
    ids = torch.randint(0, 512, (1, 12))
    with torch.no_grad():
        a, b = ref(ids, use_cache=True), model(ids, use_cache=True)
        la, lb = a.logits[:, -1], b.logits[:, -1]
        assert (la - lb).abs().max() / la.abs().max() < 2e-2
        pa, pb = a.past_key_values, b.past_key_values
        for _ in range(2):
            nxt = la.argmax(-1, keepdim=True)
            a = ref(nxt, past_key_values=pa, use_cache=True)
            b = model(nxt, past_key_values=pb, use_cache=True)
            la, lb, pa, pb = a.logits[:, -1], b.logits[:, -1], a.past_key_values, b.past_key_values
            assert (la - lb).abs().max() / la.abs().max() < 2e-2


def test_proxy_mismatch_raises(emu):
    from crispybits_kernels.ops import PackedLinear
    from crispybits_kernels.integration import _QKVProxy
    ws = [PackedLinear(from_packed_dict(pack_linear_dict(torch.randn(128, 128) * .05, 3, 128, None, torch.float32),
                                        "cpu", torch.float32)) for _ in range(3)]
    ws[0].permute_for_rope_(64)
    ws[1].permute_for_rope_(64)
    owner = FusedQKV(*ws, rope_head_dim=64)
    x = torch.randn(1, 128)
    owner.prime(x, torch.ones(1, 64), torch.zeros(1, 64))
    with pytest.raises(RuntimeError):
        _QKVProxy(owner, 0)(x.clone())


def test_paper_checkpoint_dir_installs(emu, tmp_path):
    """pack_checkpoint.py's layout (block_{i:03d}.pt + manifest.json, continuous bitstream,
    the paper quantizer) installs through install_bitmap with the manifest's bitmap, and the
    model matches the same weights dequantized on the CPU."""
    from crispybits_kernels.reference import write_checkpoint_dir
    from oracle import reference as R
    torch.manual_seed(0)
    dtype = torch.float32
    base = _tiny("llama").to(dtype).eval()
    bitmap = [3, 2, 4]
    write_checkpoint_dir(base, tmp_path, bitmap, group_size=128, model_name="tiny-llama")
    assert sorted(p.name for p in tmp_path.iterdir()) == ["block_000.pt", "block_001.pt", "block_002.pt",
                                                          "manifest.json"]
    ref = copy.deepcopy(base)
    for block, bits in zip(_blocks(ref), bitmap):
        for _, m in block.named_modules():
            if isinstance(m, torch.nn.Linear):
                q, s, z = R.affine_quantize_weight(m.weight.detach().float().numpy(), bits, 128)
                m.weight.data.copy_(torch.from_numpy(R.dequantize(q, s, z, 128)).to(m.weight))
    model = install_bitmap(copy.deepcopy(base), tmp_path, None, device="cpu", dtype=dtype, fuse=True)
    ids = torch.randint(0, 512, (1, 12))
    with torch.no_grad():
        la, lb = ref(ids).logits[:, -1], model(ids).logits[:, -1]
    assert (la - lb).abs().max() / la.abs().max() < 2e-2
    with pytest.raises(ValueError):
        install_bitmap(copy.deepcopy(base), tmp_path, [4, 2, 4], device="cpu", dtype=dtype)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; any other --gpus exits non-zero with a message, before
    touching a device."""
    import subprocess
    import sys
    root = __import__("os").path.dirname(__import__("os").path.dirname(__import__("os").path.abspath(__file__)))
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2", "--steps", "1"], cwd=root,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "--gpus 2 is not supported" in r.stderr


def test_fused_rope_hooks_prime_once_and_keep_the_model_exact(emu, tmp_path, monkeypatch):
    """The attention pre-hook primes each block's owner once per forward, the slots take the
    parked outputs (nothing stays parked), and the identity tables are what keeps the model's
    own rotation from rotating Q/K a second time: without them the block output is far off."""
    torch.manual_seed(0)
    dtype = torch.float32
    base = _tiny("llama").to(dtype).eval()
    write_packed_dir(base, tmp_path, bits_options=(3,), dtype=dtype)
    ref = copy.deepcopy(base)
    _dequantize_model_(ref, [3, 3, 3])
    model = install_bitmap(copy.deepcopy(base), tmp_path, [3, 3, 3], device="cpu", dtype=dtype, fuse_rope=True)
    primes = []
    orig_prime = FusedQKV.prime
    monkeypatch.setattr(FusedQKV, "prime", lambda self, *a: (primes.append(1), orig_prime(self, *a))[1])
    ids = torch.randint(0, 512, (1, 16))

    def block0_update(m):
        h = m(ids, output_hidden_states=True).hidden_states
        return (h[1] - h[0]).float()

    with torch.no_grad():
        la, lb = block0_update(ref), block0_update(model)
    assert len(primes) == 3
    assert (la - lb).abs().max() / la.abs().max() < 2e-2
    assert not any(blk.self_attn.crispybits_qkv.pending for blk in _blocks(model))
    monkeypatch.setattr(FusedQKV, "identity_tables", lambda self, cos, sin: (cos, sin))
    with torch.no_grad():
        lb2 = block0_update(model)
    assert (la - lb2).abs().max() / la.abs().max() > 0.2, "a second rotation went unnoticed"


def test_trace_summary_finds_the_timed_step(tmp_path, capsys):
    """bench.py --trace-summary on a synthetic kernel trace of the default command: the eager
    and warm-up runs and the timed replays share the step's period-3 keys, and the roofline's
    first per-shape graph (32 launches of the first shape) continues that period for one
    launch; the timed region ends before it and each shape gets its own kernel and grid."""
    import csv
    import json
    import os
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    sys.path.insert(0, root)
    import bench
    grids = [(65536, 256, "<0, 3, 1, 8, 0>"), (176128, 256, "<0, 3, 1, 8, 0>"), (393216, 768, "<0, 3, 1, 4, 0>")]
    durs = [4000, 6600, 7300]
    launches = [(s, 10) for _ in range(56) for _ in range(32) for s in range(3)]     # step order: layer, shape
    launches[-50 * 96:] = [(s, 0) for _ in range(50 * 32) for s in range(3)]          # the timed replays
    launches += [(s, 20) for s in range(3) for _ in range(32)]                         # roofline graphs
    path = tmp_path / "trace.csv"
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, ["Kernel_Name", "Grid_Size_X", "Workgroup_Size_X", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        t = 0
        for s, extra in launches:
            g, b, tpl = grids[s]
            w.writerow({"Kernel_Name": f"void cbk::(anonymous namespace)::gemv_stream_kernel{tpl}(cbk::GemvArgs)",
                        "Grid_Size_X": g, "Workgroup_Size_X": b, "Start_Timestamp": t,
                        "End_Timestamp": t + durs[s] + extra})
            t += 10000
    line = {"ms_per_step": 0.6, "value": 1.0, "roofline": {"frac": 0.3, "avg_launch_us": 6.0,
                                                           "bytes_per_launch_avg": 14509056}}
    bj = tmp_path / "b.json"
    bj.write_text(json.dumps(line) + "\n")
    bench.trace_summary(str(path), str(bj))
    out = capsys.readouterr().out.splitlines()
    rows = [r for r in out if r.startswith("| 4096") or r.startswith("| 11008")]
    assert len(rows) == 3
    for (K, N), r, (g, b, _), d in zip(bench.SHAPES, rows, grids, durs):
        cells = [c.strip() for c in r.strip("|").split("|")]
        assert cells[0] == f"{K} -> {N}" and cells[2] == str(g) and cells[3] == str(b)
        assert cells[4] == "1600" and cells[5] == str(d)              # only the timed replays


def test_trace_summary_gemm_rows(tmp_path, capsys):
    """bench.py --trace-summary on a synthetic trace of a `--sweeps gemm` run: each sweep row's
    launches form one run of a kernel and grid (a gate-up row two: its own kernel, then the plain
    GEMMs of the sequence it replaces, with elementwise kernels between them); the timed tail of
    each run is reported."""
    import csv
    import json
    import os
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    sys.path.insert(0, root)
    import bench
    plain = "void cbk::(anonymous namespace)::gemm_f16_kernel<4, false, true, 0, false>(cbk::GemmArgs)"
    gu = "void cbk::(anonymous namespace)::gemm_f16_kernel<4, false, true, 0, true>(cbk::GemmArgs)"
    seq = [(plain, 131072, 50000 if i >= 9 else 60000) for i in range(29)]
    seq += [(gu, 704512, 200000 if i >= 7 else 250000) for i in range(22)]
    for i in range(42):
        seq.append((plain, 352256, 100000 if i >= 12 else 130000))
        seq.append(("void at::native::elementwise_kernel<128, 4>(int, float)", 4096, 9000))
    path = tmp_path / "trace.csv"
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, ["Kernel_Name", "Grid_Size_X", "Workgroup_Size_X", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        t = 0
        for name, grid, d in seq:
            w.writerow({"Kernel_Name": name, "Grid_Size_X": grid, "Workgroup_Size_X": 512, "Start_Timestamp": t,
                        "End_Timestamp": t + d})
            t += 300000
    line = {"ms_per_step": 0.6, "value": 1.0, "roofline": {}, "gemm": [
        {"M": 1024, "K": 4096, "N": 4096, "bits": 4, "us": 51.0},
        {"M": 1024, "K": 4096, "N": [11008, 11008], "bits": 4, "kind": "gate_up", "us": 210.0,
         "two_gemms_and_mul_us": 230.0}]}
    bj = tmp_path / "b.json"
    bj.write_text(json.dumps(line) + "\n")
    bench.trace_summary(str(path), str(bj))
    out = [r for r in capsys.readouterr().out.splitlines() if r.startswith("| 1024")]
    cells = [[c.strip() for c in r.strip("|").split("|")] for r in out]
    assert [c[7:9] for c in cells] == [["20", "50000"], ["15", "200000"], ["30", "100000"]]
    assert cells[1][2] == "2 x 11008" and "true" in cells[1][4] and cells[2][2] == "11008 (x 2)"
    assert cells[1][11] == str(round(2 * 1024 * 4096 * 2 * 11008 / 200e-6 / 1e12))
