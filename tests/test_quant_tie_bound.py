"""The producer's fast path (quant.hip: quant_piece) replaces rint(w / scale) by
rint(fma(w, inv, zero)) and redoes a lane with the IEEE division when some code lies within
tol = (max|w| inv + qmax + 1) 2^-21 of a half-integer.  This checks that bound on the CPU,
against the exact results of both quantizers (Kernel/crispybits_kernels/reference.py:24-26:
rint(w/s) + z; quantization/crispybits_quant/affine.py:57-58: rint(w/s + z)), on inputs
packed next to rounding ties, with the reciprocal off by up to one ulp either way (the
hardware reciprocal's error before the Newton step).

fma is emulated in float64: w * inv is exact there (24 + 24 bits), and adding the integer
zero rounds at most once more, far inside the bound's margin."""
import numpy as np
import pytest

f32 = np.float32


def _fast(w, scale, zero, qmax, ulp_shift):
    inv0 = (f32(1) / scale).astype(f32)
    inv0 = np.nextafter(inv0, np.where(ulp_shift > 0, np.inf, -np.inf).astype(f32)) if ulp_shift else inv0
    e = (f32(1) - scale.astype(np.float64) * inv0.astype(np.float64)).astype(f32)          # fma(-s, inv, 1)
    inv = (e.astype(np.float64) * inv0 + inv0).astype(f32)                                # fma(e, inv, inv)
    y = (w.astype(np.float64) * inv.astype(np.float64) + zero).astype(f32)               # fma(w, inv, zero)
    r = np.rint(y)
    lim = f32(0.5) - (np.abs(w) * inv + (qmax + 1)).astype(f32) * f32(2.0 ** -21)
    return r, np.abs(y - r) < lim


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("ulp_shift", [-1, 0, 1])
def test_fast_path_never_disagrees_when_taken(bits, ulp_shift):
    rng = np.random.default_rng(bits * 10 + ulp_shift + 1)
    qmax = f32((1 << bits) - 1)
    n = 1_000_000
    scale = (rng.random(n) * 0.01 + 1e-5).astype(f32)
    zero = rng.integers(0, int(qmax) + 1, n).astype(f32)
    # quotients at k + 1/2 plus a few ulps either way, and uniformly spread ones
    k = rng.integers(-int(qmax) - 2, 2 * int(qmax) + 2, n).astype(np.float64)
    frac = np.where(rng.random(n) < 0.7, 0.5 + rng.integers(-64, 65, n) * 2.0 ** -23, rng.random(n))
    w = ((k + frac) * scale.astype(np.float64)).astype(f32)
    r_fast, taken = _fast(w, scale, zero, qmax, ulp_shift)
    kernel_ref = np.rint((w / scale).astype(f32)) + zero                   # rint(w/s) + z
    paper_ref = np.rint(((w / scale).astype(f32) + zero).astype(f32))    # rint(w/s + z)
    assert taken.mean() > 0.25                      # 70 % of the inputs sit within 64 ulps of a tie
    assert np.array_equal(r_fast[taken], kernel_ref[taken])
    assert np.array_equal(r_fast[taken], paper_ref[taken])
    # the exact ties themselves are never taken on the fast path
    tie = (w / scale).astype(f32) - np.floor((w / scale).astype(f32)) == f32(0.5)
    assert not np.any(taken & tie)
