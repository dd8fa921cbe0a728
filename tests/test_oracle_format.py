"""Pins the CPU oracle's format functions (oracle/reference.py) and the kernels'
decode order on the CPU.

Sources of truth, none of them a retyped oracle formula:
  * committed golden fixtures from the pure-Python bitstream / scalar-fp32
    restatements (tests/golden/make_golden.py, oracle/bruteforce.py);
  * the reference's inline known-answer tests (Kernel/tests/test_packing.py:19-36,
    test_device_logic.py:32-56, 84-88);
  * closed-form invariants (round trips, error bounds, exact magic conversion).
"""
import json
import math
import os

import numpy as np
import pytest

from oracle import bruteforce
from oracle import reference as R

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _h2f(hexes):
    return np.array([int(h, 16) for h in hexes], dtype=np.uint32).view(np.float32)


def _words(rows):
    return np.array(rows, dtype=np.uint64).astype(np.uint32).view(np.int32)


@pytest.mark.parametrize("case", json.load(open(os.path.join(GOLDEN, "packing.json"))),
                         ids=lambda c: f"W{c['bits']}-K{c['K']}")
def test_pack_matches_golden(case):
    q = np.array(case["codes"])
    p = R.pack_codes(q, case["bits"])
    assert np.array_equal(p, _words(case["words"]))
    assert np.array_equal(R.unpack_codes(p, case["bits"], case["K"]), q)
    assert np.array_equal(R.unpack_codes_by_slot(p, case["bits"], case["K"]), q)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("K", [32, 200, 4096, 4128])
def test_unpack_by_slot_equals_random_access(bits, K):
    """The slot-wise unpack (and the float64 dequant built on it) against the random-access
    unpack on arbitrary words -- every bit pattern, including the words past K."""
    rng = np.random.default_rng(bits * 7 + K)
    C = math.ceil(K / 32)
    p = rng.integers(0, 1 << 32, size=(9, C * bits), dtype=np.uint64).astype(np.uint32).view(np.int32)
    q = R.unpack_codes(p, bits, K)
    assert np.array_equal(R.unpack_codes_by_slot(p, bits, K), q)
    from oracle import emulator as E
    for gs in (32, 128):
        G = math.ceil(K / gs)
        sc = rng.standard_normal((9, G)).astype(np.float16)
        ze = rng.integers(0, 1 << bits, size=(9, G)).astype(np.float16)
        assert np.array_equal(E.dequant64_fast(p, sc, ze, bits, K, gs), E.dequant64(p, sc, ze, bits, K, gs))


@pytest.mark.parametrize("case", json.load(open(os.path.join(GOLDEN, "quantize.json"))),
                         ids=lambda c: f"W{c['bits']}-K{c['K']}-g{c['group_size']}")
def test_quantize_matches_golden(case):
    w = np.stack([_h2f(r) for r in case["w"]])
    q, s, z = R.quantize_affine(w, case["bits"], case["group_size"])
    for i, row in enumerate(case["rows"]):
        assert np.array_equal(q[i], row["q"])
        assert np.array_equal(s[i], _h2f(row["scale"]))
        assert np.array_equal(z[i], _h2f(row["zero"]))


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("K", [32, 128, 200, 4096, 5120])
def test_pack_roundtrip(bits, K):
    rng = np.random.default_rng(bits * 1000 + K)
    q = rng.integers(0, 1 << bits, size=(7, K)).astype(np.int32)
    p = R.pack_codes(q, bits)
    assert p.dtype == np.int32 and p.shape[1] == math.ceil(K / 32) * bits
    assert np.array_equal(R.unpack_codes(p, bits, K), q)


@pytest.mark.parametrize("bits,per_word", [(2, 16), (4, 8)])
def test_codes_per_word(bits, per_word):
    # Kernel/tests/test_packing.py:19-25
    q = np.concatenate([np.arange(per_word) % (1 << bits), np.zeros(32 - per_word, int)])[None]
    w0 = int(R.pack_codes(q, bits)[0, 0]) & 0xFFFFFFFF
    assert [(w0 >> (bits * i)) & ((1 << bits) - 1) for i in range(per_word)] == q[0, :per_word].tolist()


def test_w3_three_words_per_chunk_and_straddle():
    # Kernel/tests/test_packing.py:28-36
    p = R.pack_codes(np.full((1, 32), 7), 3)
    assert p.shape == (1, 3) and all((int(v) & 0xFFFFFFFF) == 0xFFFFFFFF for v in p[0])
    q = np.zeros((1, 32), int)
    q[0, 10] = 0b101
    p = R.pack_codes(q, 3)
    assert (int(p[0, 0]) & 0xFFFFFFFF) >> 30 == 0b01 and (int(p[0, 1]) & 1) == 0b1


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_quantize_error_bounded(bits):
    # Kernel/tests/test_packing.py:39-46: |W-hat - W| <= 1.5 steps
    rng = np.random.default_rng(0)
    w = rng.standard_normal((16, 384)).astype(np.float32)
    q, s, z = R.quantize_affine(w, bits, 128)
    wd = R.dequantize(q, s, z, 128)
    step = np.repeat(s, 128, axis=1)
    assert np.all(np.abs(wd - w) <= step * 1.5 + 1e-5)
    # zero-point is an integer in [0, qmax]; codes in range
    assert np.all((z >= 0) & (z <= (1 << bits) - 1) & (z == np.rint(z)))
    assert q.min() >= 0 and q.max() <= (1 << bits) - 1


def test_quantize_constant_group_and_padding():
    # a constant group has scale clamped to 1e-8; K padding repeats the last column
    w = np.full((1, 128), 0.37, np.float32)
    q, s, z = R.quantize_affine(w, 4, 128)
    assert s[0, 0] == np.float32(1e-8)
    w = np.concatenate([np.linspace(-1, 1, 100, dtype=np.float32)[None]], 1)
    q, s, z = R.quantize_affine(w, 3, 64)
    wp = np.concatenate([w[:, 64:], np.repeat(w[:, -1:], 28, 1)], 1)
    q2, s2, z2 = R.quantize_affine(wp, 3, 64)
    assert s[0, 1] == s2[0, 0] and z[0, 1] == z2[0, 0]


def test_dequantize_elementwise_matches_python_floats():
    case = json.load(open(os.path.join(GOLDEN, "quantize.json")))[5]
    q = np.array([r["q"] for r in case["rows"]])
    s = np.stack([_h2f(r["scale"]) for r in case["rows"]]).astype(np.float16)
    z = np.stack([_h2f(r["zero"]) for r in case["rows"]]).astype(np.float16)
    wd = R.dequantize(q, s, z, case["group_size"])
    for i in range(q.shape[0]):
        for k in range(0, q.shape[1], 7):
            g = k // case["group_size"]
            expect = (float(q[i, k]) - float(z[i, g])) * float(s[i, g])     # exact in fp64, rounds once
            assert wd[i, k] == np.float32(expect)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_chunk_code_matches_layout(bits):
    # Kernel/tests/test_device_logic.py:32-41 (scalar chunk extraction)
    rng = np.random.default_rng(bits)
    q = rng.integers(0, 1 << bits, size=(16, 160))
    p = R.pack_codes(q, bits)
    for r in range(q.shape[0]):
        for c in range(5):
            w = p[r, c * bits:(c + 1) * bits]
            assert [R.chunk_code(w, j, bits) for j in range(32)] == q[r, c * 32:(c + 1) * 32].tolist()


def test_magic_float_conversion_exact():
    # Kernel/tests/test_device_logic.py:44-45
    assert all(R.code_to_float(q) == float(q) for q in range(16))


# ---- static check of the MFMA kernels' packed-fp16 decode (csrc/cbk_decode.hpp) ------------

def _perm_b32(s0, s1, sel):
    """v_perm_b32: byte i of the result = byte sel[i] of (s0:s1), bytes 0-3 from s1."""
    src = (s0 << 32) | s1
    out = 0
    for i in range(4):
        b = (sel >> (8 * i)) & 0xFF
        out |= ((src >> (8 * b)) & 0xFF) << (8 * i)
    return out


def _alignbit(hi, lo, sh):
    return (((hi << 32) | lo) >> sh) & 0xFFFFFFFF


def _decode(words, bits):
    """Python restatement of Decode<BITS>::run: 16 packed pairs of fp16 bit patterns."""
    M = 0x64006400
    w = [int(v) & 0xFFFFFFFF for v in words]
    h = []
    if bits == 4:
        for t in range(4):
            for s in range(4):
                h.append(((w[t] >> (4 * s)) & 0x000F000F) | M)
    elif bits == 2:
        for t in range(2):
            for s in range(8):
                h.append(((w[t] >> (2 * s)) & 0x00030003) | M)
    else:
        v0 = (w[0] & 0xFFFF) | ((w[0] << 1) & 0xFFFF0000)
        v1 = ((w[1] >> 1) & 0xFFFF) | (w[1] & 0xFFFF0000)
        v2 = ((w[2] >> 2) & 0xFFFF) | ((w[2] >> 1) & 0xFFFF0000)
        h = [0] * 16
        for k in range(5):
            h[k] = ((v0 >> (3 * k)) & 0x00070007) | M
            h[5 + k] = ((v1 >> (3 * k)) & 0x00070007) | M
            h[10 + k] = ((v2 >> (3 * k)) & 0x00070007) | M
        c10 = _alignbit(w[1], w[0], 30)
        c21 = _alignbit(w[2], w[1], 31)
        h[15] = (_perm_b32(c21, c10, 0x05040100) & 0x00070007) | M
    return h


def _kappa(bits, p):
    if bits == 4:
        return 8 * (p >> 3) + ((p >> 1) & 3) + 4 * (p & 1)
    if bits == 2:
        return 16 * (p >> 4) + ((p >> 1) & 7) + 8 * (p & 1)
    P = p >> 1
    return (21 if p & 1 else 10) if P == 15 else 11 * (P // 5) + P % 5 + 5 * (p & 1)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_kappa_is_a_permutation(bits):
    assert sorted(_kappa(bits, p) for p in range(32)) == list(range(32))


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_packed_fp16_decode_recovers_every_code(bits):
    """Every half of the decode is fp16(1024 + q) of the code kappa(slot) names."""
    rng = np.random.default_rng(10 + bits)
    q = rng.integers(0, 1 << bits, size=(64, 32))
    q[0] = (1 << bits) - 1                         # all-ones chunk: every straddle bit set
    q[1] = 0
    p = R.pack_codes(q, bits)
    for r in range(q.shape[0]):
        h = _decode(p[r], bits)
        for slot in range(32):
            half = (h[slot >> 1] >> (16 * (slot & 1))) & 0xFFFF
            val = float(np.array([half], dtype=np.uint16).view(np.float16)[0])
            assert val == 1024.0 + q[r, _kappa(bits, slot)]


def test_rope_unperm_inverts_row_order():
    # Kernel/tests/test_device_logic.py:48-56 with the emulator's un-permutation
    import torch
    import sys
    from oracle.emulator import unperm_index
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(__file__)), "llm_quantization-kernel_amd"))
    from crispybits_kernels.ops import rope_row_order
    for hd in (64, 128):
        n = 4 * hd
        assert unperm_index(n, hd).tolist() == rope_row_order(n, hd).tolist()
        u = unperm_index(n, hd)
        for p in range(0, n, 2):
            assert u[p + 1] - u[p] == hd // 2 and u[p] // hd == u[p + 1] // hd


def test_split_boundaries_cover_all_chunks():
    # Kernel/tests/test_device_logic.py:84-88
    from oracle.emulator import split_bounds
    for C in (1, 7, 128, 161):
        for P in range(1, min(C, 40) + 1):
            b = split_bounds(C, P)
            assert b[0][0] == 0 and b[-1][1] == C
            assert all(b[i][1] == b[i + 1][0] and b[i][0] < b[i][1] for i in range(len(b) - 1))


def test_bruteforce_and_numpy_packers_agree_on_random_rows():
    rng = np.random.default_rng(7)
    for bits in (2, 3, 4):
        q = rng.integers(0, 1 << bits, size=(5, 77))
        p = R.pack_codes(q, bits)
        for r in range(5):
            assert (p[r].view(np.uint32).tolist() == bruteforce.pack_row(q[r].tolist(), bits))
            assert bruteforce.unpack_row(p[r].view(np.uint32).tolist(), bits, 77) == q[r].tolist()


# ---------------------------------------------------------------- the paper quantizer's format
# quantization/crispybits_quant/affine.py and packing.py: pinned by the brute-force fixtures
# and the inline checks of quantization/tests/test_affine_pack.py.

@pytest.mark.parametrize("case", json.load(open(os.path.join(GOLDEN, "packing_continuous.json"))),
                         ids=lambda c: f"W{c['bits']}-K{c['K']}")
def test_continuous_pack_matches_golden(case):
    q = np.array(case["codes"])
    p = R.pack_codes_continuous(q, case["bits"])
    assert p.shape[1] == (case["K"] * case["bits"] + 31) // 32          # packing.py:24-25
    assert np.array_equal(p, _words(case["words"]))
    assert np.array_equal(R.unpack_codes_continuous(p, case["K"], case["bits"]), q)


@pytest.mark.parametrize("case", json.load(open(os.path.join(GOLDEN, "affine_quantize.json"))),
                         ids=lambda c: f"W{c['bits']}-K{c['K']}-g{c['group_size']}")
def test_affine_quantize_matches_golden(case):
    w = np.stack([_h2f(r) for r in case["w"]])
    q, s, z = R.affine_quantize_weight(w, case["bits"], case["group_size"])
    for i, row in enumerate(case["rows"]):
        assert np.array_equal(q[i], row["q"])
        assert np.array_equal(s[i], _h2f(row["scale"]))
        assert np.array_equal(z[i], _h2f(row["zero"]))


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_continuous_roundtrip_and_chunked_equivalence(bits):
    # quantization/tests/test_affine_pack.py:6-12 (K = 259), and the two formats agree iff K % 32 == 0
    rng = np.random.default_rng(bits)
    q = rng.integers(0, 1 << bits, size=(7, 259)).astype(np.int32)
    p = R.pack_codes_continuous(q, bits)
    assert np.array_equal(R.unpack_codes_continuous(p, 259, bits), q)
    assert np.array_equal(R.continuous_to_chunked(p, bits, 259), R.pack_codes(q, bits))
    q32 = q[:, :256]
    assert np.array_equal(R.pack_codes_continuous(q32, bits), R.pack_codes(q32, bits))


def test_affine_shapes():
    # quantization/tests/test_affine_pack.py:15-20
    q, s, z = R.affine_quantize_weight(np.random.default_rng(0).standard_normal((5, 257)).astype(np.float32), 3, 128)
    assert q.shape == (5, 257) and s.shape == (5, 3) and z.shape == (5, 3)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_affine_groups_not_spanning_zero(bits):
    # quantization/tests/test_affine_pack.py:23-38: error <= half a step of the zero-inclusive range
    rng = np.random.default_rng(0)
    qmax = (1 << bits) - 1
    for w in (rng.random((3, 128), dtype=np.float32) + 1.0, -(rng.random((3, 128), dtype=np.float32) + 1.0),
              np.full((3, 128), 0.37, np.float32), np.full((3, 128), -0.37, np.float32),
              np.zeros((3, 128), np.float32)):
        q, s, z = R.affine_quantize_weight(w, bits, 128)
        wh = R.dequantize(q, s, z, 128)
        step = (np.maximum(w, 0).max(1) - np.minimum(w, 0).min(1)) / qmax
        assert np.all(np.abs(wh - w).max(1) <= step / 2 + 1e-5)
        assert np.all((z >= 0) & (z <= qmax))
        # zero-inclusive: an exact 0 weight maps to the zero code and dequantizes to 0 exactly
        q0, s0, z0 = R.affine_quantize_weight(np.concatenate([w[:, :127], np.zeros((3, 1), np.float32)], 1), bits, 128)
        assert np.all(R.dequantize(q0, s0, z0, 128)[:, 127] == 0)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_affine_zero_spanning_groups_match_plain_minmax(bits):
    # quantization/tests/test_affine_pack.py:41-55: where each group spans zero, the clamps
    # are inactive and the codes are round(w/s + z) of the plain min/max scale
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((4, 256)) * 0.02).astype(np.float32)
    w[:, 0], w[:, 128], w[:, 1], w[:, 129] = -0.05, 0.05, 0.05, -0.05
    q, _, _ = R.affine_quantize_weight(w, bits, 128)
    qmax = np.float32((1 << bits) - 1)
    for g in range(2):
        wg = w[:, g * 128:(g + 1) * 128]
        s = ((wg.max(1) - wg.min(1)) / qmax).astype(np.float32)
        z = np.clip(np.rint(-wg.min(1) / s), 0, qmax).astype(np.float32)
        ref = np.clip(np.rint((wg / s[:, None]).astype(np.float32) + z[:, None]), 0, qmax)
        assert np.array_equal(q[:, g * 128:(g + 1) * 128], ref.astype(np.int32))


def test_affine_tie_differs_from_kernel_quantizer():
    # the two quantizers differ on ties when the zero is odd: round(w/s + z) vs round(w/s) + z
    w = np.zeros((1, 32), np.float32)
    w[0, :4] = [-1.0, 0.5, 2.0, 1.5]
    qa, sa, za = R.affine_quantize_weight(w, 2, 32)
    qk, sk, zk = R.quantize_affine(w, 2, 32)
    assert sa[0, 0] == sk[0, 0] == 1.0 and za[0, 0] == zk[0, 0] == 1.0
    assert qa[0, 1] == 2 and qk[0, 1] == 1
