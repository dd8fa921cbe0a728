"""GPU parity of the on-device quantizer + packer (quant.hip, through the C-ABI entry
cbk_quantize_pack) against the CPU oracle's quantize_affine + pack_codes
(Kernel/crispybits_kernels/reference.py:10-55).

Bar: bit-exact -- packed words, and scales/zeros after the same rounding to the
metadata dtype -- for every width, group size, ragged K, input dtype and metadata
dtype below, including rows whose codes land exactly on rounding ties and
constant groups (scale clamped to 1e-8).
"""
import numpy as np
import pytest
import torch

from crispybits_kernels import _C
from crispybits_kernels import reference as P
from oracle import reference as R

pytestmark = pytest.mark.gpu

# vector path: group size 32..512 dividing 512, K % 8 == 0; the rest take the general path
CASES = [(7, 32, 32), (5, 200, 64), (33, 4128, 128), (300, 640, 128), (3, 96, 256), (2, 250, 256), (64, 11008, 128),
         (9, 1000, 512), (4, 2080, 1024), (6, 544, 96), (1, 8, 32)]


def _oracle(w32, bits, gs, mdt):
    q, s, z = R.quantize_affine(w32, bits, gs)
    st = torch.from_numpy(s).to(mdt).float().numpy()
    zt = torch.from_numpy(z).to(mdt).float().numpy()
    return R.pack_codes(q, bits), st, zt


def _check(w, bits, gs, mdt):
    wd = w.cuda()
    packed, s, z = _C.quantize_pack(wd, bits, gs, mdt)
    torch.cuda.synchronize()
    po, so, zo = _oracle(w.float().numpy(), bits, gs, mdt)
    assert packed.dtype == torch.int32 and s.dtype == mdt and z.dtype == mdt
    assert np.array_equal(packed.cpu().numpy(), po)
    assert np.array_equal(s.float().cpu().numpy(), so)
    assert np.array_equal(z.float().cpu().numpy(), zo)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("N,K,gs", CASES)
def test_quantize_pack_bit_exact(hip, bits, N, K, gs):
    g = torch.Generator().manual_seed(bits * 13 + K + gs)
    w = torch.randn(N, K, generator=g) * 0.02
    _check(w, bits, gs, torch.float16)


@pytest.mark.parametrize("wdt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("mdt", [torch.float16, torch.bfloat16, torch.float32])
def test_quantize_pack_dtypes(hip, wdt, mdt):
    g = torch.Generator().manual_seed(5)
    w = (torch.randn(40, 300, generator=g) * 0.05).to(wdt)
    _check(w, 3, 128, mdt)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_rounding_ties_and_constant_groups(hip, bits):
    """Integer weights over [0, 2*qmax] give scale 2, so every odd weight sits on a
    .5 tie (round half to even); a constant group clamps its scale to 1e-8."""
    qmax = (1 << bits) - 1
    rng = np.random.default_rng(bits)
    w = rng.integers(0, 2 * qmax + 1, size=(16, 256)).astype(np.float32)
    w[:, ::32] = 0
    w[:, 1::32] = 2 * qmax
    w[3] = 0.7
    w[4, 128:] = -2.5
    _check(torch.from_numpy(w), bits, 32, torch.float32)
    _check(torch.from_numpy(w), bits, 128, torch.float16)


def test_unaligned_weight_takes_the_general_path(hip):
    g = torch.Generator().manual_seed(3)
    buf = (torch.randn(24 * 256 + 1, generator=g) * 0.02).half().cuda()
    w = buf[1:].view(24, 256)                       # contiguous, 2 bytes past a 16-byte boundary
    packed, s, z = _C.quantize_pack(w, 3, 128)
    torch.cuda.synchronize()
    po, so, zo = _oracle(w.float().cpu().numpy(), 3, 128, torch.float16)
    assert np.array_equal(packed.cpu().numpy(), po)
    assert np.array_equal(s.float().cpu().numpy(), so) and np.array_equal(z.float().cpu().numpy(), zo)


def test_full_size_weight_matches_cpu_producer(hip):
    """A Llama-7B MLP weight [11008, 4096]: the torch CPU producer (itself pinned to
    the oracle) against the device path, and pack_linear_dict routes CUDA weights
    through the device producer."""
    g = torch.Generator().manual_seed(11)
    w = torch.randn(11008, 4096, generator=g) * 0.02
    q, s, z = P.quantize_affine(w, 3, 128)
    pc = P.pack_codes(q, 3)
    packed, sd, zd = _C.quantize_pack(w.cuda(), 3, 128, torch.float16)
    assert torch.equal(packed.cpu(), pc)
    assert torch.equal(sd.cpu(), s.half()) and torch.equal(zd.cpu(), z.half())
    d = P.pack_linear_dict(w[:64].cuda(), 3, 128)
    assert torch.equal(d["packed"], pc[:64]) and d["packed"].device.type == "cpu"


def test_empty_weight_is_a_no_op(hip):
    packed, s, z = _C.quantize_pack(torch.empty(0, 256, device="cuda"), 4, 128)
    torch.cuda.synchronize()
    assert packed.shape == (0, 32) and s.shape == (0, 2)


# ---------------------------------------------------------------- scheme 1: the paper quantizer

def _check_affine(w, bits, gs, mdt):
    packed, s, z = _C.quantize_pack(w.cuda(), bits, gs, mdt, scheme=1)
    torch.cuda.synchronize()
    q, so, zo = R.affine_quantize_weight(w.float().numpy(), bits, gs)
    assert np.array_equal(packed.cpu().numpy(), R.pack_codes(q, bits))
    assert np.array_equal(s.float().cpu().numpy(), torch.from_numpy(so).to(mdt).float().numpy())
    assert np.array_equal(z.float().cpu().numpy(), torch.from_numpy(zo).to(mdt).float().numpy())


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("N,K,gs", [(7, 32, 32), (5, 257, 128), (33, 4128, 128), (300, 640, 64), (6, 544, 96),
                                    (64, 11008, 128)])
def test_affine_scheme_bit_exact(hip, bits, N, K, gs):
    g = torch.Generator().manual_seed(bits * 17 + K)
    w = torch.randn(N, K, generator=g) * 0.02
    w[0] = 0.37                                   # positive row: min clamps to 0
    w[1] = 0.0                                    # zero row: scale 1
    w[2, : min(K, 100)] = -2.0
    _check_affine(w, bits, gs, torch.float16)


@pytest.mark.parametrize("wdt", [torch.float16, torch.bfloat16, torch.float32])
def test_affine_scheme_dtypes_and_ties(hip, wdt):
    g = torch.Generator().manual_seed(9)
    _check_affine((torch.randn(40, 300, generator=g) * 0.05).to(wdt), 3, 128, wdt)
    tie = torch.zeros(4, 64)
    tie[:, :4] = torch.tensor([-1.0, 0.5, 2.0, 1.5])     # scale 1, zero 1: round(0.5 + 1) = 2
    _check_affine(tie, 2, 32, torch.float32)


def test_pack_block_on_the_device_matches_cpu(hip):
    from crispybits_kernels.reference import pack_block
    blk = torch.nn.Sequential(torch.nn.Linear(200, 48), torch.nn.Linear(256, 16)).half()
    cpu = pack_block(blk, 3, 64)
    dev = pack_block(blk.cuda(), 3, 64)
    for name in cpu:
        for key in ("packed", "scales", "zeros", "bias"):
            assert torch.equal(cpu[name][key], dev[name][key]), (name, key)
