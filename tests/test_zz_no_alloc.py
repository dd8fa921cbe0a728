"""The allocation-free decode entry point (cbk_packed_gemv_noalloc) through the C ABI:
its output equals cbk_packed_gemv's (same kernels, split-K partials in the library's
device scratch instead of a caller buffer) bit for bit, on two calls in a row, the
second with a smaller input; sizes above the scratch are rejected on the host."""
import numpy as np
import pytest
import torch

import cabi
from crispybits_kernels import _C
from crispybits_kernels.io import from_packed_dict
from crispybits_kernels.reference import pack_linear_dict
from oracle import emulator as E

pytestmark = pytest.mark.gpu


def _weight(n, k, bits, seed):
    g = torch.Generator().manual_seed(seed)
    d = pack_linear_dict(torch.randn(n, k, generator=g) * 0.02, bits, 128, None, torch.float16)
    W64 = E.dequant64(d["packed"].numpy(), d["scales"].double().numpy(), d["zeros"].double().numpy(), bits, k, 128)
    return from_packed_dict(d, "cuda", torch.float16), W64


def _noalloc(x, w, split_k, rho=1, act=0):
    out = torch.empty((x.size(0), w.out_features), dtype=x.dtype, device=x.device)
    dev = x.get_device()
    rc = cabi.lib.cbk_packed_gemv_noalloc(x.data_ptr(), 0, x.size(0), x.size(1), w.packed.data_ptr(),
                                         w.scales.data_ptr(), w.zeros.data_ptr(), None, w.out_features, w.bits,
                                         w.group_size, split_k, rho, act, out.data_ptr(), dev,
                                         torch.cuda.current_stream(dev).cuda_stream)
    assert rc == 0, cabi.lib.cbk_last_error().decode()
    return out


@pytest.mark.parametrize("split_k", [1, 4])
def test_noalloc_matches_allocating_entry_point(split_k):
    cases = [(2, 4096, 4096, 3, 11), (1, 1024, 2048, 4, 12)]     # the second call is smaller
    for M, N, K, bits, seed in cases:
        print(f"noalloc case M={M} N={N} K={K} W{bits} split_k={split_k}", flush=True)
        w, W64 = _weight(N, K, bits, seed)
        g = torch.Generator().manual_seed(seed + 100)
        x = torch.randn(M, K, generator=g).half().cuda()
        y = _noalloc(x, w, split_k)
        ref = _C.packed_gemv(x, w.packed, w.scales, w.zeros, None, w.bits, K, 128, split_k, 1, 0, None)
        torch.cuda.synchronize()
        assert torch.equal(y, ref)
        r64 = x.double().cpu().numpy() @ W64.T
        err = np.abs(y.double().cpu().numpy() - r64).max() / np.abs(r64).max()
        assert err < 3e-3, err


def test_noalloc_rejects_oversized_partials():
    # 16 batch rows x 4096 rows x 64 splits of fp32 partials exceed the scratch; the check
    # runs on the host before any device work (fake, never dereferenced addresses)
    a = 1 << 20
    rc = cabi.lib.cbk_packed_gemv_noalloc(a, 0, 16, 4096, a, a, a, None, 4096, 4, 128, 64, 1, 0, a, 0, None)
    assert rc == 1
    assert "device scratch" in cabi.lib.cbk_last_error().decode()
    limit = 1 << 21
    need = cabi.lib.cbk_gemv_partial_floats(0, 16, 4096, 4096, 128, 64)
    assert need > limit
