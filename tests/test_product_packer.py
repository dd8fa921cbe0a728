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
