"""The callers of the path on the GPU: the HF integration glue (install_bitmap,
FusedQKV, FusedLlamaMLP) on tiny Llama / OPT models through the HIP library, and
blocks of the Llama-2-7B linear stack (config 5) captured in a HIP graph.

Mirrors the reference's Kernel/tests/test_integration.py:41-71 (logits of the
packed model against the dequantized fp16 model, prefill then cached decode) and
the decode step of Kernel/scripts/ablation_decode.py:48-56."""
import copy

import numpy as np
import pytest
import torch

from crispybits_kernels import fused_gate_up, fused_qkv, packed_linear
from crispybits_kernels.ops import PackedLinearWeight
from crispybits_kernels.reference import dequantize, dequantized_weight, pack_codes, pack_linear_dict, quantize_affine

transformers = pytest.importorskip("transformers")

from crispybits_kernels import FusedLlamaMLP, FusedQKV, install_bitmap, tune_model  # noqa: E402
from crispybits_kernels.integration import _blocks  # noqa: E402
from crispybits_kernels.reference import write_packed_dir  # noqa: E402

pytestmark = pytest.mark.gpu


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
        with torch.no_grad():                     # sharper attention, so RoPE errors would show
            for blk in _blocks(m):
                blk.self_attn.q_proj.weight.mul_(8.0)
                blk.self_attn.k_proj.weight.mul_(8.0)
        return m
    cfg = transformers.OPTConfig(hidden_size=256, ffn_dim=512, num_hidden_layers=3, num_attention_heads=4,
                                 vocab_size=512, word_embed_proj_dim=256)
    return transformers.OPTForCausalLM(cfg)


def _rel(a, b):
    return ((a.float() - b.float()).abs().max() / a.float().abs().max()).item()


@pytest.mark.parametrize("kind,fuse,fuse_rope", [("llama", False, False), ("llama", True, False),
                                                 ("llama", True, True), ("opt", False, False), ("opt", True, True)])
def test_model_matches_dequantized(hip, tmp_path, kind, fuse, fuse_rope):
    torch.manual_seed(0)
    dtype = torch.float16
    base = _tiny(kind).to(dtype).to("cuda").eval()
    bitmap = [4, 2, 3]
    # quantized on the CPU, like _dequantize_model_: torch's fp32 arithmetic on the GPU
    # rounds some scales differently, which would change a few codes
    write_packed_dir(copy.deepcopy(base).cpu(), tmp_path, bits_options=(2, 3, 4), dtype=dtype)
    ref = copy.deepcopy(base)
    _dequantize_model_(ref, bitmap)
    model = install_bitmap(copy.deepcopy(base), tmp_path, bitmap, device="cuda", dtype=dtype, fuse=fuse,
                           fuse_rope=fuse_rope)
    if fuse and kind == "llama":
        owners = [m for m in model.modules() if isinstance(m, FusedQKV)]
        assert owners and any(isinstance(m, FusedLlamaMLP) for m in model.modules())
        assert all(bool(o.rope_head_dim) == fuse_rope for o in owners)
    if fuse:
        tune_model(model, iters=2, warmup=1, dtype=dtype)
    ids = torch.randint(0, 512, (1, 12), device="cuda")
    with torch.no_grad():
        a, b = ref(ids, use_cache=True), model(ids, use_cache=True)
        la, lb = a.logits[:, -1], b.logits[:, -1]
        assert _rel(la, lb) < 2e-2, f"prefill logits diverge: {_rel(la, lb):.3e}"
        pa, pb = a.past_key_values, b.past_key_values
        for _ in range(4):
            nxt = la.argmax(-1, keepdim=True)
            a = ref(nxt, past_key_values=pa, use_cache=True)
            b = model(nxt, past_key_values=pb, use_cache=True)
            la, lb, pa, pb = a.logits[:, -1], b.logits[:, -1], a.past_key_values, b.past_key_values
            assert _rel(la, lb) < 2e-2, f"decode logits diverge: {_rel(la, lb):.3e}"


# ---------------------------------------------------------------- Llama-2-7B linear stack (config 5)

H, I = 4096, 11008
LINEARS = [("q", H, H), ("k", H, H), ("v", H, H), ("o", H, H), ("gate", I, H), ("up", I, H), ("down", H, I)]


def _stack_block(i, bits, dev):
    """Block i of config 5: linear j from a device generator seeded 1000 * i + j."""
    pb, db = {}, {}
    for j, (nm, N, K) in enumerate(LINEARS):
        g = torch.Generator(device=dev).manual_seed(1000 * i + j)
        W = torch.randn(N, K, generator=g, device=dev) * 0.02
        q, s, z = quantize_affine(W, bits, 128)
        s, z = s.half(), z.half()
        pb[nm] = PackedLinearWeight(pack_codes(q, bits), s, z, bits, 128, K, N)
        db[nm] = dequantize(q, s.float(), z.float(), 128)
    return pb, db


def _step(blocks, xh, xi):
    outs = []
    for b in blocks:
        outs += list(fused_qkv(xh, b["q"], b["k"], b["v"]))
        outs.append(packed_linear(xh, b["o"]))
        outs.append(fused_gate_up(xh, b["gate"], b["up"]))
        outs.append(packed_linear(xi, b["down"]))
    return outs


def test_llama_stack_blocks_graph_replay(hip):
    """Two blocks of the stack (bits from the config-5 bitmap) at decode: every output
    against fp32 on the dequantized weights, and the captured step replayed three
    times, with eager work and synchronizations between, bit-identical to eager."""
    dev = torch.device("cuda", 0)
    bitmap = [int(b) for b in np.random.default_rng(0).choice([2, 3, 4], 32)][:2]
    built = [_stack_block(i, bits, dev) for i, bits in enumerate(bitmap)]
    blocks = [pb for pb, _ in built]
    xh = (torch.randn(1, H, generator=torch.Generator().manual_seed(1)) * 1.0).half().to(dev)
    xi = (torch.randn(1, I, generator=torch.Generator().manual_seed(2)) * 1.0).half().to(dev)

    eager = [t.clone() for t in _step(blocks, xh, xi)]
    torch.cuda.synchronize()
    k = 0
    for pb, db in built:
        refs = [xh.float() @ db[n].T for n in ("q", "k", "v", "o")]
        refs.append(torch.nn.functional.silu(xh.float() @ db["gate"].T) * (xh.float() @ db["up"].T))
        refs.append(xi.float() @ db["down"].T)
        for r in refs:
            err = _rel(r, eager[k])
            assert err < 1e-2, f"stack output {k}: rel err {err:.2e}"
            k += 1

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = _step(blocks, xh, xi)
    torch.cuda.synchronize()
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for j, (c, e) in enumerate(zip(captured, eager)):
            assert torch.equal(c, e), f"replay {rep}: output {j} differs from eager"
        _step(blocks, xh, xi)                     # eager work between the replays
        torch.cuda.synchronize()


def test_llama_stack_blocks_prefill_graph_replay(hip):
    """The same two blocks at a prefill batch (M = 256: the QKV, o and down GEMMs and the
    one-launch gate-up GEMM) captured as one graph and replayed three times, with eager work
    and synchronizations between, bit-identical to eager every time."""
    dev = torch.device("cuda", 0)
    bitmap = [int(b) for b in np.random.default_rng(0).choice([2, 3, 4], 32)][:2]
    blocks = [_stack_block(i, bits, dev)[0] for i, bits in enumerate(bitmap)]
    g = torch.Generator().manual_seed(3)
    xh = torch.randn(256, H, generator=g).half().to(dev)
    xi = torch.randn(256, I, generator=g).half().to(dev)
    eager = [t.clone() for t in _step(blocks, xh, xi)]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = _step(blocks, xh, xi)
    torch.cuda.synchronize()
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for j, (c, e) in enumerate(zip(captured, eager)):
            assert torch.equal(c.view(torch.int16), e.view(torch.int16)), f"replay {rep}: output {j} differs"
        _step(blocks, xh, xi)
        torch.cuda.synchronize()


def test_llama_stack_blocks_oracle_decode_and_prefill(hip):
    """Three blocks of the stack (config-5 bits, Llama-2-7B widths: blocks 0, 1 and 3, the first
    W4, W3 and W2 blocks of the bitmap) against the CPU oracle, the
    decode leg at M = 1 and the prefill leg at M = 2048: every linear of both blocks (fused QKV,
    o, fused gate-up, down) against the float64 product on the oracle's dequantized weights --
    W-hat for decode, W-hat rounded once to fp16 for the prefill GEMM (oracle/emulator.py).  The
    GPU computes every output; the float64 reference covers 256 sampled output features of each
    linear, and the prefill 64 sampled rows, so the oracle stays small."""
    from oracle import emulator as E

    dev = torch.device("cuda", 0)
    full = [int(b) for b in np.random.default_rng(0).choice([2, 3, 4], 32)]
    picked = [full.index(4), full.index(3), full.index(2)]
    assert picked == [0, 1, 3]
    rng = np.random.default_rng(7)
    rows = np.sort(rng.choice(2048, 64, replace=False))
    gx = torch.Generator().manual_seed(11)
    xh = torch.randn(2048, H, generator=gx).half().to(dev)
    xi = torch.randn(2048, I, generator=gx).half().to(dev)
    for i in picked:
        bits = full[i]
        pb, _ = _stack_block(i, bits, dev)
        cols, W64 = {}, {}
        for nm, N, K in LINEARS:
            c = np.sort(rng.choice(N, 256, replace=False)) if nm != "up" else cols["gate"]
            w = pb[nm]
            cols[nm] = c
            W64[nm] = E.dequant64(w.packed.cpu().numpy()[c], w.scales.double().cpu().numpy()[c],
                                  w.zeros.double().cpu().numpy()[c], bits, K, 128)
        for M in (1, 2048):
            a, b = (xh[:1], xi[:1]) if M == 1 else (xh, xi)
            sel = np.arange(1) if M == 1 else rows
            xa, xb = a[sel].double().cpu().numpy(), b[sel].double().cpu().numpy()
            Wd = W64 if M == 1 else {nm: E.round_to(W, torch.float16) for nm, W in W64.items()}
            oq, ok, ov = fused_qkv(a, pb["q"], pb["k"], pb["v"])
            outs = {"q": oq, "k": ok, "v": ov, "o": packed_linear(a, pb["o"]),
                    "gate": fused_gate_up(a, pb["gate"], pb["up"]), "down": packed_linear(b, pb["down"])}
            refs = {nm: (xb if nm == "down" else xa) @ Wd[nm].T for nm in ("q", "k", "v", "o", "down")}
            gv, uv = xa @ Wd["gate"].T, xa @ Wd["up"].T
            refs["gate"] = E.silu64(gv) * uv
            for nm, ref in refs.items():
                got = outs[nm][torch.from_numpy(sel).to(dev)][:, torch.from_numpy(cols[nm]).to(dev)]
                err = _rel(torch.from_numpy(ref), got.cpu())
                assert err < 3e-3, f"block {i} (W{bits}) M={M} {nm}: rel err {err:.2e}"
