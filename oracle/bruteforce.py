"""Pure-Python scalar restatements used to pin the numpy oracle -- TEST INFRASTRUCTURE ONLY.

Each function re-derives a closed form of the packed format or the quantizer one
element at a time, with Python integers (arbitrary-width bitstreams) and numpy
float32 *scalars* (IEEE fp32 rounding at every step).  They share no code with
``oracle.reference``; a mistake in either (a wrong shift, a dropped straddle bit,
a different rounding rule) makes the golden-fixture tests fail.
"""
from __future__ import annotations

import numpy as np


def pack_row(codes, bits: int) -> list:
    """One row -> list of uint32 words: a single LSB-first Python-int bitstream,
    padded to whole 32-code chunks (Kernel/crispybits_kernels/reference.py:37-55)."""
    stream = 0
    for k, c in enumerate(codes):
        stream |= (int(c) & ((1 << bits) - 1)) << (k * bits)
    nchunks = -(-len(codes) // 32)
    nwords = nchunks * bits
    return [(stream >> (32 * i)) & 0xFFFFFFFF for i in range(nwords)]


def unpack_row(words, bits: int, K: int) -> list:
    """Inverse of pack_row: rebuild the bitstream and cut it into codes."""
    stream = 0
    for i, w in enumerate(words):
        stream |= (int(w) & 0xFFFFFFFF) << (32 * i)
    return [(stream >> (k * bits)) & ((1 << bits) - 1) for k in range(K)]


def quantize_row(row, bits: int, group_size: int):
    """Scalar fp32 min/max affine quantization of one row (reference.py:10-27).

    scale = max((max - min) / qmax, 1e-8); zero = clamp(rne(-min / scale), 0, qmax);
    q = clamp(rne(w / scale) + zero, 0, qmax); the last group is padded by
    repeating the last element.  Every operation rounds to fp32.
    """
    f32 = np.float32
    K = len(row)
    G = -(-K // group_size)
    padded = [f32(v) for v in row] + [f32(row[-1])] * (G * group_size - K)
    qmax = f32((1 << bits) - 1)
    qs, ss, zs = [], [], []
    for g in range(G):
        grp = padded[g * group_size:(g + 1) * group_size]
        mn, mx = min(grp), max(grp)
        scale = f32(mx - mn) / qmax
        scale = scale if scale > f32(1e-8) else f32(1e-8)
        zero = f32(np.rint(f32(-mn) / scale))
        zero = min(max(zero, f32(0)), qmax)
        for v in grp:
            q = f32(np.rint(f32(v) / scale)) + zero
            qs.append(int(min(max(q, f32(0)), qmax)))
        ss.append(float(scale))
        zs.append(float(zero))
    return qs[:K], ss, zs


def pack_row_continuous(codes, bits: int) -> list:
    """One row -> ceil(K*bits/32) uint32 words of the unpadded LSB-first bitstream
    (quantization/crispybits_quant/packing.py:24-25,45-54)."""
    stream = 0
    for k, c in enumerate(codes):
        stream |= (int(c) & ((1 << bits) - 1)) << (k * bits)
    nwords = (len(codes) * bits + 31) // 32
    return [(stream >> (32 * i)) & 0xFFFFFFFF for i in range(nwords)]


def affine_quantize_row(row, bits: int, group_size: int, eps: float = 1e-8):
    """Scalar fp32 zero-inclusive quantization of one row (crispybits_quant/affine.py:28-71):
    per group of real columns, min <= 0 <= max, scale = (max - min) / qmax (1 if below eps),
    zero = clamp(rne(-min / scale), 0, qmax), q = clamp(rne(w / scale + zero), 0, qmax)."""
    f32 = np.float32
    K = len(row)
    qmax = f32((1 << bits) - 1)
    qs, ss, zs = [], [], []
    for s in range(0, K, group_size):
        grp = [f32(v) for v in row[s:s + group_size]]
        mn = min(min(grp), f32(0))
        mx = max(max(grp), f32(0))
        scale = f32(mx - mn) / qmax
        if scale < f32(eps):
            scale = f32(1)
        zero = min(max(f32(np.rint(f32(-mn) / scale)), f32(0)), qmax)
        for v in grp:
            y = f32(f32(v / scale) + zero)
            qs.append(int(min(max(f32(np.rint(y)), f32(0)), qmax)))
        ss.append(float(scale))
        zs.append(float(zero))
    return qs, ss, zs

