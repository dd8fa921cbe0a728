"""The product's torch quantizer/packer (crispybits_kernels.reference) produces
bit-identical packed words, scales and zeros to the pinned CPU oracle."""
import numpy as np
import pytest
import torch

from crispybits_kernels import reference as P
from oracle import reference as R


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("N,K,gs", [(7, 32, 32), (5, 200, 64), (33, 4128, 128), (300, 640, 128), (3, 96, 256)])
def test_quantize_pack_bit_exact(bits, N, K, gs):
    g = torch.Generator().manual_seed(bits * 7 + K)
    w = torch.randn(N, K, generator=g) * 0.02
    q, s, z = P.quantize_affine(w, bits, gs)
    qo, so, zo = R.quantize_affine(w.numpy(), bits, gs)
    assert np.array_equal(q.numpy(), qo) and np.array_equal(s.numpy(), so) and np.array_equal(z.numpy(), zo)
    p = P.pack_codes(q, bits)
    assert np.array_equal(p.numpy(), R.pack_codes(qo, bits))
    assert torch.equal(P.unpack_codes(p, bits, K), q)


def test_pack_linear_dict_and_dequant():
    w = torch.randn(17, 300) * 0.02
    b = torch.randn(17)
    d = P.pack_linear_dict(w, 3, 128, b)
    do = R.pack_linear_dict(w.numpy(), 3, 128, b.numpy())
    for key in ("packed", "scales", "zeros", "bias"):
        assert np.array_equal(d[key].numpy(), do[key])
    assert d["bits"] == 3 and d["in_features"] == 300 and d["out_features"] == 17
    assert np.array_equal(P.dequantized_weight(d).numpy(), R.dequantized_weight(do))


# ---------------------------------------------------------------- the paper quantizer's format

@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("N,K,gs", [(5, 257, 128), (33, 4096, 128), (7, 96, 32), (300, 200, 64)])
def test_affine_quantizer_and_continuous_packer_bit_exact(bits, N, K, gs):
    g = torch.Generator().manual_seed(bits * 11 + K)
    w = torch.randn(N, K, generator=g) * 0.02
    w[0] = 0.37                                      # constant positive row: min clamps to 0
    w[1] = 0.0                                       # all-zero row: scale below eps -> 1
    w[2, : min(K, 100)] = -2.0
    q, s, z = P.affine_quantize_weight(w, bits, gs)
    qo, so, zo = R.affine_quantize_weight(w.numpy(), bits, gs)
    assert np.array_equal(q.numpy(), qo) and np.array_equal(s.numpy(), so) and np.array_equal(z.numpy(), zo)
    assert np.all(so[1] == 1.0)
    pc = P.pack_codes_continuous(q, bits)
    assert np.array_equal(pc.numpy(), R.pack_codes_continuous(qo, bits))
    assert torch.equal(P.unpack_codes_continuous(pc, K, bits), q)
    assert torch.equal(P.continuous_to_chunked(pc, bits, K), P.pack_codes(q, bits))


def test_quantize_pack_schemes_on_cpu():
    w = torch.randn(9, 200) * 0.02
    p0, s0, z0 = P.quantize_pack(w, 3, 64, torch.float32, scheme="kernel")
    p1, s1, z1 = P.quantize_pack(w, 3, 64, torch.float32, scheme="affine")
    q, s, z = R.affine_quantize_weight(w.numpy(), 3, 64)
    assert np.array_equal(p1.numpy(), R.pack_codes(q, 3)) and np.array_equal(s1.numpy(), s)
    assert np.array_equal(p0.numpy(), R.pack_codes(R.quantize_affine(w.numpy(), 3, 64)[0], 3))
    with pytest.raises(ValueError):
        P.quantize_pack(w, 3, 64, scheme="gptq")


def test_pack_block_and_chunked_loading():
    """pack_block writes the paper's continuous layout (K = 200: 19 words per W3 row, not 21);
    io.from_packed_dict re-packs it into the kernels' chunked layout and rejects other lengths."""
    from crispybits_kernels.io import chunked_packed, from_packed_dict
    blk = torch.nn.Sequential(torch.nn.Linear(200, 16), torch.nn.Linear(256, 8, bias=False)).half()
    d = P.pack_block(blk, 3, 64)
    assert set(d) == {"0", "1"} and d["0"]["packed"].shape == (16, 19) and d["1"]["packed"].shape == (8, 24)
    assert d["0"]["scales"].dtype == torch.float16 and d["0"]["bias"] is not None and d["1"]["bias"] is None
    q, s, z = R.affine_quantize_weight(blk[0].weight.detach().float().numpy(), 3, 64)
    assert np.array_equal(d["0"]["packed"].numpy(), R.pack_codes_continuous(q, 3))
    w = from_packed_dict(d["0"], "cpu", torch.float32)
    assert np.array_equal(w.packed.numpy(), R.pack_codes(q, 3))
    with pytest.raises(ValueError):
        chunked_packed(d["0"]["packed"][:, :18], 3, 200)
