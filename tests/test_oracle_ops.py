"""Pins the oracle's operator semantics (oracle/emulator.py) against independent
derivations: the reference's per-chunk formula s*(sum x q - z sum x) evaluated
with Python loops on tiny inputs (Kernel/csrc/packed_gemv.cu:113-138), split-K
invariance, the gate-up identity (Kernel/tests/test_correctness.py:105), Q/K/V as
three linears plus rotate-half RoPE (test_correctness.py:125-146), and the GEMM's
once-rounded W-hat (packed_gemm.cu:56)."""
import math

import numpy as np
import pytest
import torch

from oracle import emulator as E
from oracle import reference as R


def _make(n, k, bits, gs=128, seed=0, bias=False):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    d = R.pack_linear_dict(w, bits, gs, (rng.standard_normal(n) * 0.1).astype(np.float32) if bias else None)
    t = dict(packed=torch.from_numpy(d["packed"]), scales=torch.from_numpy(d["scales"]),
             zeros=torch.from_numpy(d["zeros"]), bias=None if d["bias"] is None else torch.from_numpy(d["bias"]))
    return d, t


def _loop_gemv(x, d):
    """Reference per-chunk formula with Python floats."""
    q = R.unpack_codes(d["packed"], d["bits"], d["in_features"])
    s, z = d["scales"].astype(np.float64), d["zeros"].astype(np.float64)
    N, K = q.shape
    C = math.ceil(K / 32)
    out = np.zeros((x.shape[0], N))
    for b in range(x.shape[0]):
        for n in range(N):
            acc = 0.0
            for c in range(C):
                ks = range(c * 32, min(K, c * 32 + 32))
                dot = sum(float(x[b, k]) * q[n, k] for k in ks)
                xs = sum(float(x[b, k]) for k in ks)
                g = c * 32 // d["group_size"]
                acc += s[n, g] * (dot - z[n, g] * xs)
            out[b, n] = acc
    return out


@pytest.mark.parametrize("bits,K,gs", [(2, 96, 32), (3, 200, 64), (4, 256, 128)])
def test_gemv_matches_per_chunk_formula(bits, K, gs):
    d, t = _make(9, K, bits, gs, seed=bits)
    x = torch.randn(2, K, dtype=torch.float32, generator=torch.Generator().manual_seed(3))
    y = E.packed_gemv(x, t["packed"], t["scales"].float(), t["zeros"].float(), torch.empty(0), bits, K, gs,
                      1, 1, 0, None)
    ref = _loop_gemv(x.numpy(), d)
    assert np.allclose(y.numpy(), ref, rtol=1e-5, atol=1e-6)


def test_gemv_split_k_invariance_and_partials():
    d, t = _make(40, 1000, 3, seed=1)
    x = torch.randn(3, 1000, dtype=torch.float32)
    C = math.ceil(1000 / 32)
    full = E.gemv_partials64(x.double().numpy(), d["packed"], d["scales"], d["zeros"], 3, 1000, 128, 1)[0]
    for P in (2, 7, C, C + 5):
        parts = E.gemv_partials64(x.double().numpy(), d["packed"], d["scales"], d["zeros"], 3, 1000, 128, P)
        assert parts.shape[0] == min(P, C)
        assert np.allclose(parts.sum(0), full, rtol=1e-12, atol=1e-12)


def test_gemv_bias_and_activations():
    d, t = _make(30, 128, 4, seed=2, bias=True)
    x = torch.randn(2, 128)
    base = _loop_gemv(x.numpy(), d) + d["bias"].astype(np.float64)[None]
    for act, fn in ((0, lambda v: v), (1, lambda v: np.maximum(v, 0)), (2, lambda v: v / (1 + np.exp(-v)))):
        y = E.packed_gemv(x, t["packed"], t["scales"].float(), t["zeros"].float(), t["bias"].float(), 4, 128,
                          128, 1, 1, act, None)
        assert np.allclose(y.numpy(), fn(base), rtol=1e-5, atol=1e-6)


def test_fused_gate_up_identity():
    dg, g = _make(64, 256, 3, seed=4)
    du, u = _make(64, 256, 3, seed=5)
    x = torch.randn(2, 256)
    y = E.fused_gate_up(x, g["packed"], g["scales"].float(), g["zeros"].float(), u["packed"], u["scales"].float(),
                        u["zeros"].float(), 3, 256, 128, 2, 1, None)
    gv, uv = _loop_gemv(x.numpy(), dg), _loop_gemv(x.numpy(), du)
    assert np.allclose(y.numpy(), gv / (1 + np.exp(-gv)) * uv, rtol=1e-5, atol=1e-6)


def _rope_np(t, cos, sin, hd):
    M, W = t.shape
    th = t.reshape(M, W // hd, hd)
    h = hd // 2
    rot = np.concatenate([-th[..., h:], th[..., :h]], -1)
    return (th * cos[:, None] + rot * sin[:, None]).reshape(M, W)


def test_fused_qkv_is_three_linears_plus_rope():
    hd, K = 16, 128
    dq, q = _make(4 * hd, K, 4, seed=6, bias=True)
    dk, k = _make(2 * hd, K, 4, seed=7, bias=True)
    dv, v = _make(2 * hd, K, 4, seed=8)
    x = torch.randn(3, K)
    # store Q/K pair-interleaved (stored row p <- original row order[p])
    order = lambda n: (np.arange(n) // hd) * hd + (np.arange(hd) // 2 + (np.arange(hd) % 2) * (hd // 2))[np.arange(n) % hd]
    qp = {key: (val[order(4 * hd)] if val is not None else None) for key, val in q.items()}
    kp = {key: (val[order(2 * hd)] if val is not None else None) for key, val in k.items()}
    pos = np.array([3.0, 17.0, 100.0])
    inv = 1.0 / (10000 ** (np.arange(0, hd, 2) / hd))
    emb = np.concatenate([pos[:, None] * inv, pos[:, None] * inv], 1)
    cos, sin = np.cos(emb), np.sin(emb)
    oq, ok, ov = E.fused_qkv(x, qp["packed"], qp["scales"].float(), qp["zeros"].float(), qp["bias"].float(),
                             kp["packed"], kp["scales"].float(), kp["zeros"].float(), kp["bias"].float(),
                             v["packed"], v["scales"].float(), v["zeros"].float(), torch.empty(0),
                             torch.from_numpy(cos).float(), torch.from_numpy(sin).float(), hd, hd, 4, K, 128, 3, 1,
                             None)
    rq = _rope_np(_loop_gemv(x.numpy(), dq) + dq["bias"].astype(np.float64), cos, sin, hd)
    rk = _rope_np(_loop_gemv(x.numpy(), dk) + dk["bias"].astype(np.float64), cos, sin, hd)
    rv = _loop_gemv(x.numpy(), dv)
    for o, r in ((oq, rq), (ok, rk), (ov, rv)):
        assert np.allclose(o.numpy(), r, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gemm_weight_rounded_once(dtype):
    d, t = _make(20, 96, 3, gs=32, seed=9)
    s = t["scales"].to(dtype)
    z = t["zeros"].to(dtype)
    W = E.gemm_weight64(d["packed"], s.double().numpy(), z.double().numpy(), 3, 96, 32, dtype, True)
    q = R.unpack_codes(d["packed"], 3, 96)
    for n in range(20):
        for k in range(0, 96, 5):
            g = k // 32
            exact = (float(q[n, k]) - float(z[n, g])) * float(s[n, g])
            assert W[n, k] == torch.tensor(exact, dtype=torch.float32).to(dtype).double().item()


def test_rope64_is_a_complex_rotation():
    """rotate-half RoPE on the pair (d, d + h) is the complex product
    (y_d + i y_{d+h}) * e^{i theta_d} with HF's tables cos/sin = cat(f, f)."""
    rng = np.random.default_rng(5)
    M, heads, hd = 3, 4, 64
    h = hd // 2
    y = rng.standard_normal((M, heads * hd))
    theta = rng.uniform(-7, 7, (M, h))
    cos, sin = np.cos(np.concatenate([theta, theta], -1)), np.sin(np.concatenate([theta, theta], -1))
    out = E.rope64(y, cos, sin, hd).reshape(M, heads, hd)
    t = y.reshape(M, heads, hd)
    z = (t[..., :h] + 1j * t[..., h:]) * np.exp(1j * theta)[:, None, :]
    assert np.allclose(out[..., :h], z.real, atol=1e-12) and np.allclose(out[..., h:], z.imag, atol=1e-12)
    # angle zero is the identity; norms of each pair are kept
    assert np.array_equal(E.rope64(y, np.ones((M, hd)), np.zeros((M, hd)), hd), y)


def test_silu64_is_overflow_free_and_exact():
    """SiLU v sigmoid(v): equals v / (1 + e^-v) wherever that form does not overflow, satisfies
    silu(v) - silu(-v) = v (sigmoid(v) + sigmoid(-v) = 1), tends to 0 for large negative v
    without overflow (exp(-|v|) may underflow to 0, which is exact here), and to v for large
    positive v."""
    v = np.linspace(-30.0, 30.0, 2001)
    np.testing.assert_allclose(E.silu64(v), v / (1.0 + np.exp(-v)), rtol=1e-14, atol=1e-300)
    np.testing.assert_allclose(E.silu64(v) - E.silu64(-v), v, rtol=1e-13, atol=1e-13)
    with np.errstate(over="raise", invalid="raise", divide="raise"):
        big = np.array([-1e4, -800.0, 800.0, 1e4])
        out = E.silu64(big)
    assert out[0] == 0.0 and out[1] == 0.0 and out[2] == 800.0 and out[3] == 1e4
