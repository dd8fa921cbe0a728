"""Config 5 through the integration glue at full Llama-2-7B width: an HF LlamaForCausalLM with
hidden 4096, intermediate 11008 and 32 heads (random init; 2 of the 32 blocks here, the bench
runs all 32), quantized on the GPU into block_{i:03d}_w{bits}.pt files with the config-5
bitmap, installed with install_bitmap(fuse=True, fuse_rope=True), then

  * prefill and cached-decode logits against the same model with every linear replaced by its
    dequantized fp16 weight (Kernel/tests/test_integration.py:41-71, tolerance 2e-2), and
  * one decode step captured in a HIP graph over a static KV cache, replayed for successive
    tokens and checked against eager decode of the same tokens.
"""
import copy

import numpy as np
import pytest
import torch

transformers = pytest.importorskip("transformers")

from crispybits_kernels import FusedLlamaMLP, FusedQKV, install_bitmap  # noqa: E402
from crispybits_kernels import _C  # noqa: E402
from crispybits_kernels.integration import _blocks  # noqa: E402
from crispybits_kernels.reference import dequantize, pack_linear_dict, write_packed_dir  # noqa: E402

pytestmark = pytest.mark.gpu

LAYERS = 2


def _model():
    cfg = transformers.LlamaConfig(hidden_size=4096, intermediate_size=11008, num_hidden_layers=LAYERS,
                                   num_attention_heads=32, num_key_value_heads=32, vocab_size=32000,
                                   max_position_embeddings=512)
    torch.manual_seed(0)
    with torch.device("cuda"):
        m = transformers.LlamaForCausalLM(cfg).half().eval()
    return m


def write_bitmap_dir(model, out, bitmap, gs=128):
    """block_{i:03d}_w{bitmap[i]}.pt for each block, its linears quantized and packed on the GPU."""
    write_packed_dir(model, out, group_size=gs, dtype=torch.float16, bitmap=bitmap)


@torch.no_grad()
def dequantize_linears_(model, bitmap, gs=128):
    """Every block linear replaced by RN_fp16((q - z) s) of its own quantization."""
    for block, bits in zip(_blocks(model), bitmap):
        for _, m in block.named_modules():
            if isinstance(m, torch.nn.Linear):
                d = pack_linear_dict(m.weight.detach(), int(bits), gs, None, torch.float16)
                q = _C.unpack_codes(d["packed"].cuda(), int(bits), m.in_features)
                m.weight.copy_(dequantize(q, d["scales"].cuda().float(), d["zeros"].cuda().float(), gs).half())


def _rel(a, b):
    return ((a.float() - b.float()).abs().max() / a.float().abs().max()).item()


def test_llama7b_width_model_through_install_bitmap(hip, tmp_path):
    bitmap = [int(b) for b in np.random.default_rng(0).choice([2, 3, 4], 32)][:LAYERS]
    base = _model()
    write_bitmap_dir(base, tmp_path, bitmap)
    ref = copy.deepcopy(base)
    dequantize_linears_(ref, bitmap)
    model = install_bitmap(base, tmp_path, bitmap, device="cuda", dtype=torch.float16, fuse=True, fuse_rope=True)
    owners = [m for m in model.modules() if isinstance(m, FusedQKV)]
    assert len(owners) == LAYERS and all(o.rope_head_dim == 128 for o in owners)
    assert sum(isinstance(m, FusedLlamaMLP) for m in model.modules()) == LAYERS

    ids = torch.randint(0, 32000, (1, 24), generator=torch.Generator().manual_seed(1)).cuda()
    with torch.no_grad():
        a, b = ref(ids, use_cache=True), model(ids, use_cache=True)
        la, lb = a.logits[:, -1], b.logits[:, -1]
        assert _rel(la, lb) < 2e-2, f"prefill logits diverge: {_rel(la, lb):.3e}"
        pa, pb = a.past_key_values, b.past_key_values
        for _ in range(3):
            nxt = la.argmax(-1, keepdim=True)
            a = ref(nxt, past_key_values=pa, use_cache=True)
            b = model(nxt, past_key_values=pb, use_cache=True)
            la, lb, pa, pb = a.logits[:, -1], b.logits[:, -1], a.past_key_values, b.past_key_values
            assert _rel(la, lb) < 2e-2, f"decode logits diverge: {_rel(la, lb):.3e}"


def test_llama7b_width_decode_step_graph(hip, tmp_path):
    """A decode step over a static KV cache, captured once and replayed for successive tokens,
    equals eager decode of the same tokens on a second cache.

    HF's StaticLayer writes each update at its own device counter and advances it in place (it
    does not read cache_position), so the captured step advances its position buffer the same
    way and every call -- the warm-up, then each replay -- decodes the next slot; the replays
    stay inside the cache (checked before each one)."""
    bitmap = [int(b) for b in np.random.default_rng(0).choice([2, 3, 4], 32)][:LAYERS]
    base = _model()
    write_bitmap_dir(base, tmp_path, bitmap)
    model = install_bitmap(base, tmp_path, bitmap, device="cuda", dtype=torch.float16, fuse=True, fuse_rope=True)
    cfg = model.config
    P, CACHE = 12, 64
    prompt = torch.randint(0, 32000, (1, P), generator=torch.Generator().manual_seed(2)).cuda()
    tokens = torch.randint(0, 32000, (4,), generator=torch.Generator().manual_seed(3)).tolist()

    def prefilled_cache():
        cache = transformers.StaticCache(config=cfg, max_cache_len=CACHE)
        with torch.no_grad():
            model(prompt, past_key_values=cache, cache_position=torch.arange(P, device="cuda"), use_cache=True)
        return cache

    # eager reference: tokens[t] decoded at position P + t
    cache_e = prefilled_cache()
    eager = []
    with torch.no_grad():
        for t, tok in enumerate(tokens):
            out = model(torch.tensor([[tok]], device="cuda"), past_key_values=cache_e,
                        cache_position=torch.tensor([P + t], device="cuda"), use_cache=True)
            eager.append(out.logits[:, -1].clone())
    # captured step: decodes tok_buf at pos_buf, then advances pos_buf (the cache's own counter
    # advances inside the update)
    cache_g = prefilled_cache()
    tok_buf = torch.tensor([[tokens[0]]], device="cuda")
    pos_buf = torch.tensor([P], device="cuda")

    def step():
        logits = model(tok_buf, past_key_values=cache_g, cache_position=pos_buf, use_cache=True).logits[:, -1]
        pos_buf.add_(1)
        return logits

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.no_grad(), torch.cuda.stream(side):
        warm = step().clone()                 # tokens[0] at position P
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert _rel(eager[0], warm) < 1e-3
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.graph(graph):
        logits = step()
    for t in range(1, len(tokens)):
        assert P + t < CACHE and int(pos_buf) == P + t     # the slot this replay writes
        tok_buf.fill_(tokens[t])
        graph.replay()
        torch.cuda.synchronize()
        assert _rel(eager[t], logits) < 1e-3, f"token {t}: replay differs from eager ({_rel(eager[t], logits):.2e})"
