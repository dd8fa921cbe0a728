"""GPU parity of the one-launch prefill gate-up GEMM (cbk_packed_gemm_gate_up).

Bars:
  * bit-exact (every bit, signed zeros included) against the sequence it replaces -- the gate GEMM with SiLU and
    the up GEMM through cbk_packed_gemm, multiplied in the activation dtype (the reference's
    ops.py:216-220): the same dequantized weights, MFMA order and roundings;
  * against the CPU oracle (float64 products of W-hat rounded once to the dtype, each factor
    rounded to the dtype, product rounded once): max|y - ref| / max|ref| below the fp16 bar
    3e-3 (bf16 2e-2), inside the brief's 1e-2.
Shapes cover partial tiles in M, N and K, group sizes 32..256, fractional zero points on one
projection only, W2/W3/W4, fp16 and bf16, and the BASELINE stack shape M = 2048, 4096 -> 11008.
"""
import numpy as np
import pytest
import torch

from crispybits_kernels import _C, fused_gate_up, ops
from crispybits_kernels.io import from_packed_dict
from crispybits_kernels.reference import pack_linear_dict
from oracle import emulator as E

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 3e-3, torch.bfloat16: 2e-2}


def _dict(n, k, bits, dtype, seed, gs=128, scale=0.05):
    g = torch.Generator().manual_seed(seed)
    W = torch.randn(n, k, generator=g) * scale
    return pack_linear_dict(W, bits, gs, None, dtype)


def _x(M, K, dtype, seed=3):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(M, K, generator=g).to(dtype).cuda()


def _two_gemms(x, g, u):
    a = _C.packed_gemm(x, g.packed, g.scales, g.zeros, None, g.bits, g.in_features, g.group_size, ops.ACT["silu"],
                       True)
    b = _C.packed_gemm(x, u.packed, u.scales, u.zeros, None, u.bits, u.in_features, u.group_size, ops.ACT["none"],
                       True)
    return a * b


def _oracle(x, dg, du, bits, K, gs, dtype):
    Wg = E.gemm_weight64(dg["packed"].numpy(), dg["scales"].to(dtype).double().numpy(),
                         dg["zeros"].to(dtype).double().numpy(), bits, K, gs, dtype, True)
    Wu = E.gemm_weight64(du["packed"].numpy(), du["scales"].to(dtype).double().numpy(),
                         du["zeros"].to(dtype).double().numpy(), bits, K, gs, dtype, True)
    xd = x.cpu().double().numpy()
    gv = E.round_to(E.silu64(xd @ Wg.T), dtype)
    uv = E.round_to(xd @ Wu.T, dtype)
    return gv * uv


def _check(y, ref, dtype):
    yd = y.float().cpu().double().numpy()
    e = np.abs(yd - ref).max() / (np.abs(ref).max() + 1e-6)
    assert e < TOL[dtype], f"rel err {e:.2e}"
    assert e < 1e-2


def _same_bits(a, b):
    """Bitwise equality (torch.equal takes -0.0 == +0.0)."""
    iv = {2: torch.int16, 4: torch.int32}[a.element_size()]
    return a.shape == b.shape and a.dtype == b.dtype and torch.equal(a.view(iv), b.view(iv))


def _gate_up(x, g, u):
    return _C.packed_gemm_gate_up(x, g.packed, g.scales, g.zeros, u.packed, u.scales, u.zeros, g.bits,
                                  g.in_features, g.group_size)


def _timed_launches(fn):
    _C.timer_start(64)
    try:
        y = fn()
        torch.cuda.synchronize()
    finally:
        _, d = _C.timer_stop()
    return y, len(d)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("M,K,N,gs", [(17, 256, 384, 128), (130, 400, 300, 128), (257, 640, 100, 64),
                                      (64, 1024, 130, 32), (200, 768, 256, 256)])
def test_gate_up_gemm(hip, dtype, bits, M, K, N, gs):
    dg, du = _dict(N, K, bits, dtype, 1, gs), _dict(N, K, bits, dtype, 2, gs)
    g, u = from_packed_dict(dg, "cuda", dtype), from_packed_dict(du, "cuda", dtype)
    x = _x(M, K, dtype)
    y, launches = _timed_launches(lambda: _gate_up(x, g, u))
    assert launches == 1
    assert _same_bits(y, _two_gemms(x, g, u))
    _check(y, _oracle(x, dg, du, bits, K, gs, dtype), dtype)
    assert _same_bits(fused_gate_up(x, g, u), y)          # the ops path past the decode threshold


@pytest.mark.parametrize("which", ["gate", "up"])
@pytest.mark.parametrize("bits", [3, 4])
def test_gate_up_gemm_fractional_zeros(hip, which, bits):
    """Zero points that are not integers on the first 40 columns of one projection: those
    column slabs take the fp32 dequant, the others the packed-fp16 one."""
    K, N, M = 512, 200, 150
    dg, du = _dict(N, K, bits, torch.float16, 1), _dict(N, K, bits, torch.float16, 2)
    d = dict(dg if which == "gate" else du)
    z = d["zeros"].clone()
    z[:40] = z[:40] + 0.375
    d["zeros"] = z
    if which == "gate":
        dg = d
    else:
        du = d
    g, u = from_packed_dict(dg, "cuda", torch.float16), from_packed_dict(du, "cuda", torch.float16)
    x = _x(M, K, torch.float16)
    y = _gate_up(x, g, u)
    assert _same_bits(y, _two_gemms(x, g, u))
    _check(y, _oracle(x, dg, du, bits, K, 128, torch.float16), torch.float16)


def test_gate_up_gemm_fallbacks(hip):
    """Calls the one-launch kernel cannot take run the two GEMMs and the product: fp32
    activations, and x at an address that is not 16-byte aligned."""
    K, N, M = 256, 96, 40
    dg, du = _dict(N, K, 4, torch.float16, 1), _dict(N, K, 4, torch.float16, 2)
    g, u = from_packed_dict(dg, "cuda", torch.float16), from_packed_dict(du, "cuda", torch.float16)
    x = _x(M, K, torch.float16)
    xs = torch.empty(M * K + 1, dtype=torch.float16, device="cuda")[1:].view(M, K)
    xs.copy_(x)
    assert xs.data_ptr() % 16 != 0
    y, launches = _timed_launches(lambda: _gate_up(xs, g, u))
    assert launches == 2                                   # two GEMM launches (the product is torch's)
    assert _same_bits(y, _two_gemms(xs, g, u))
    _check(y, _oracle(x, dg, du, 4, K, 128, torch.float16), torch.float16)   # another GEMM kernel's k order
    d32g, d32u = _dict(N, K, 4, torch.float32, 1), _dict(N, K, 4, torch.float32, 2)
    g32, u32 = from_packed_dict(d32g, "cuda", torch.float32), from_packed_dict(d32u, "cuda", torch.float32)
    x32 = x.float()
    assert _same_bits(_gate_up(x32, g32, u32), _two_gemms(x32, g32, u32))


def test_gate_up_gemm_empty_batch(hip):
    dg = _dict(64, 256, 4, torch.float16, 1)
    g = from_packed_dict(dg, "cuda", torch.float16)
    assert _gate_up(torch.empty(0, 256, dtype=torch.float16, device="cuda"), g, g).shape == (0, 64)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_gate_up_gemm_baseline_stack_shape(hip, bits):
    """The Llama-2-7B MLP at the stack's prefill batch (M = 2048, 4096 -> 2 x 11008, weights
    N(0, 0.02)): bit-exact against the two GEMMs; oracle check on a row sample."""
    K, N, M = 4096, 11008, 2048
    dg, du = _dict(N, K, bits, torch.float16, 11, scale=0.02), _dict(N, K, bits, torch.float16, 12, scale=0.02)
    g, u = from_packed_dict(dg, "cuda", torch.float16), from_packed_dict(du, "cuda", torch.float16)
    x = _x(M, K, torch.float16)
    y = _gate_up(x, g, u)
    assert _same_bits(y, _two_gemms(x, g, u))
    rows = torch.tensor([0, 1, 127, 128, 1000, 2047])
    _check(y[rows.cuda()], _oracle(x[rows.cuda()], dg, du, bits, K, 128, torch.float16), torch.float16)


def test_gate_up_gemm_signed_zero(hip):
    """Regression: bench.py's gate-up inputs at M = 2048 (W3, weights from the device
    producer) hold an output whose up factor is a signed zero; the one-launch epilogue must
    form it as the up GEMM stores it (act(sum + 0) rounded), so every bit matches."""
    import os
    import sys
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench
    dev = torch.device("cuda", 0)
    x = bench.randx(torch, 2048, 4096, 1, dev)
    g, u = bench.make_weight(torch, 11008, 4096, 3, 4, dev), bench.make_weight(torch, 11008, 4096, 3, 5, dev)
    y = _gate_up(x, g, u)
    assert _same_bits(y, _two_gemms(x, g, u))
    assert bool((y == 0).any())


def test_gate_up_gemm_through_the_c_abi(hip):
    """cbk_packed_gemm_gate_up called through ctypes (device pointers, a non-default stream)
    writes the same bits as the op binding, and M = 0 launches nothing."""
    import os
    import sys
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import cabi
    K, N, M = 768, 200, 96
    dg, du = _dict(N, K, 3, torch.float16, 1), _dict(N, K, 3, torch.float16, 2)
    g, u = from_packed_dict(dg, "cuda", torch.float16), from_packed_dict(du, "cuda", torch.float16)
    x = _x(M, K, torch.float16)
    ref = _gate_up(x, g, u)
    out = torch.full_like(ref, float("nan"))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    rc = cabi.lib.cbk_packed_gemm_gate_up(x.data_ptr(), 0, M, K, g.packed.data_ptr(), g.scales.data_ptr(),
                                          g.zeros.data_ptr(), u.packed.data_ptr(), u.scales.data_ptr(),
                                          u.zeros.data_ptr(), N, 3, 128, out.data_ptr(), 0, s.cuda_stream)
    assert rc == 0, cabi.last_error()
    s.synchronize()
    assert _same_bits(out, ref)
    rc = cabi.lib.cbk_packed_gemm_gate_up(x.data_ptr(), 0, 0, K, g.packed.data_ptr(), g.scales.data_ptr(),
                                          g.zeros.data_ptr(), u.packed.data_ptr(), u.scales.data_ptr(),
                                          u.zeros.data_ptr(), N, 3, 128, out.data_ptr(), 0, s.cuda_stream)
    assert rc == 0
    s.synchronize()
    assert _same_bits(out, ref)


@pytest.mark.parametrize("bits", [3, 4])
def test_gate_up_gemm_bf16_stack_shape(hip, bits):
    """bf16 activations (bf16 scales and zeros) at the stack's prefill shape: bit-exact against
    the two bf16 GEMMs and their bf16 product; oracle check on a row sample."""
    K, N, M = 4096, 11008, 2048
    dt = torch.bfloat16
    dg, du = _dict(N, K, bits, dt, 21, scale=0.02), _dict(N, K, bits, dt, 22, scale=0.02)
    g, u = from_packed_dict(dg, "cuda", dt), from_packed_dict(du, "cuda", dt)
    x = _x(M, K, dt)
    y = _gate_up(x, g, u)
    assert _same_bits(y, _two_gemms(x, g, u))
    rows = torch.tensor([0, 77, 1024, 2047])
    _check(y[rows.cuda()], _oracle(x[rows.cuda()], dg, du, bits, K, 128, dt), dt)
