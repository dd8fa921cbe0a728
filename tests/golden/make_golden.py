"""Writes the small golden fixtures under tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

The expected values come from ``oracle.bruteforce`` -- pure-Python bitstream
and scalar-fp32 restatements of the reference's closed forms
(Kernel/crispybits_kernels/reference.py:10-67, and the paper quantizer's
quantization/crispybits_quant/affine.py:28-71, packing.py:24-54) -- so the vectorised numpy
oracle and the HIP kernels are both checked against an independent derivation.
Floats are stored as the hex of their IEEE fp32 bit pattern so the fixtures
are exact.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import bruteforce  # noqa: E402


def f32hex(v) -> str:
    return "%08x" % int(np.array([v], dtype=np.float32).view(np.uint32)[0])


def packing_cases():
    rng = np.random.default_rng(1234)
    cases = []
    for bits in (2, 3, 4):
        for K in (32, 45, 96, 200):
            q = rng.integers(0, 1 << bits, size=(3, K))
            cases.append(dict(bits=bits, K=K, codes=q.tolist(),
                              words=[bruteforce.pack_row(r, bits) for r in q]))
    # structured rows: all-max codes, a single straddling code, ascending codes
    for bits in (2, 3, 4):
        qmax = (1 << bits) - 1
        rows = [[qmax] * 64, [0] * 64, [k % (qmax + 1) for k in range(64)]]
        if bits == 3:
            rows[1][10] = 0b101    # straddles words 0|1 of chunk 0
            rows[1][21] = 0b110    # straddles words 1|2 of chunk 0
            rows[1][42] = 0b011    # code 10 of chunk 1
        cases.append(dict(bits=bits, K=64, codes=rows, words=[bruteforce.pack_row(r, bits) for r in rows]))
    return cases


def quant_cases():
    rng = np.random.default_rng(99)
    cases = []
    for bits in (2, 3, 4):
        for K, gs in ((64, 32), (96, 64), (200, 128), (256, 128)):
            w = (rng.standard_normal((2, K)) * 0.02).astype(np.float32)
            rows = []
            for r in w:
                q, s, z = bruteforce.quantize_row(r.tolist(), bits, gs)
                rows.append(dict(q=q, scale=[f32hex(v) for v in s], zero=[f32hex(v) for v in z]))
            cases.append(dict(bits=bits, K=K, group_size=gs, w=[[f32hex(v) for v in r] for r in w], rows=rows))
    # constant group (scale clamps to 1e-8) and a group that does not span zero
    for bits in (2, 3, 4):
        w = np.stack([np.full(128, 0.37, np.float32), np.linspace(1.0, 2.0, 128, dtype=np.float32)])
        rows = []
        for r in w:
            q, s, z = bruteforce.quantize_row(r.tolist(), bits, 128)
            rows.append(dict(q=q, scale=[f32hex(v) for v in s], zero=[f32hex(v) for v in z]))
        cases.append(dict(bits=bits, K=128, group_size=128, w=[[f32hex(v) for v in r] for r in w], rows=rows))
    return cases


def continuous_cases():
    """The unpadded bitstream of quantization/crispybits_quant/packing.py:45-54."""
    rng = np.random.default_rng(4321)
    cases = []
    for bits in (2, 3, 4):
        for K in (32, 45, 259):
            q = rng.integers(0, 1 << bits, size=(2, K))
            cases.append(dict(bits=bits, K=K, codes=q.tolist(),
                              words=[bruteforce.pack_row_continuous(r, bits) for r in q]))
    return cases


def affine_cases():
    """crispybits_quant/affine.py:28-71: zero-spanning random rows, groups that do not span
    zero, constant and all-zero groups, a ragged last group, and a rounding tie where the
    zero is odd (w/s = 0.5, z = 1: round(w/s + z) = 2, round(w/s) + z = 1)."""
    rng = np.random.default_rng(77)
    f = np.float32
    cases = []

    def case(bits, gs, w):
        rows = []
        for r in w:
            q, sc, z = bruteforce.affine_quantize_row(r.tolist(), bits, gs)
            rows.append(dict(q=q, scale=[f32hex(v) for v in sc], zero=[f32hex(v) for v in z]))
        return dict(bits=bits, K=w.shape[1], group_size=gs, w=[[f32hex(v) for v in r] for r in w], rows=rows)

    for bits in (2, 3, 4):
        for K, gs in ((64, 32), (257, 128), (256, 128)):
            cases.append(case(bits, gs, (rng.standard_normal((2, K)) * 0.02).astype(f)))
        special = np.stack([np.linspace(1.0, 2.0, 128, dtype=f), -np.linspace(1.0, 2.0, 128, dtype=f),
                            np.full(128, 0.37, f), np.full(128, -0.37, f), np.zeros(128, f)])
        cases.append(case(bits, 128, special))
    tie = np.zeros((1, 32), f)
    tie[0, :4] = [-1.0, 0.5, 2.0, 1.5]
    cases.append(case(2, 32, tie))
    return cases


def main():
    with open(os.path.join(HERE, "packing.json"), "w") as f:
        json.dump(packing_cases(), f, separators=(",", ":"))
    with open(os.path.join(HERE, "quantize.json"), "w") as f:
        json.dump(quant_cases(), f, separators=(",", ":"))
    with open(os.path.join(HERE, "packing_continuous.json"), "w") as f:
        json.dump(continuous_cases(), f, separators=(",", ":"))
    with open(os.path.join(HERE, "affine_quantize.json"), "w") as f:
        json.dump(affine_cases(), f, separators=(",", ":"))


if __name__ == "__main__":
    main()
