"""numpy restatement of the reference quantizer / packer -- TEST INFRASTRUCTURE ONLY.

Follows /root/reference/Crispybits/Kernel/crispybits_kernels/reference.py.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline use this.
"""
from __future__ import annotations

import math

import numpy as np

__all__ = ["quantize_affine", "dequantize", "pack_codes", "unpack_codes", "unpack_codes_by_slot", "pack_linear_dict",
           "dequantized_weight", "chunk_code", "code_to_float", "words_per_row",
           "affine_quantize_weight", "pack_codes_continuous", "unpack_codes_continuous",
           "continuous_to_chunked"]


def words_per_row(K: int, bits: int) -> int:
    """ceil(K/32) * bits int32 words per row (reference.py:41,53; host_utils.h:63-64)."""
    return math.ceil(K / 32) * bits


def quantize_affine(w: np.ndarray, bits: int, group_size: int = 128):
    """Group-wise asymmetric min/max quantization (reference.py:10-27).

    All arithmetic in IEEE fp32, round-half-to-even (``np.rint`` == ``torch.round``).
    K is padded up to a multiple of ``group_size`` by repeating the last column
    (reference.py:18-19).  Returns (q int32 [N,K], scale fp32 [N,G], zero fp32 [N,G]).
    """
    assert bits in (2, 3, 4)
    w = np.asarray(w, dtype=np.float32)
    N, K = w.shape
    G = math.ceil(K / group_size)
    Kp = G * group_size
    wf = np.zeros((N, Kp), dtype=np.float32)
    wf[:, :K] = w
    if Kp != K:
        wf[:, K:] = wf[:, K - 1:K]
    g = wf.reshape(N, G, group_size)
    qmax = np.float32((1 << bits) - 1)
    mn = g.min(-1)
    mx = g.max(-1)
    scale = np.maximum((mx - mn) / qmax, np.float32(1e-8)).astype(np.float32)
    zero = np.clip(np.rint(-mn / scale), 0, qmax).astype(np.float32)
    q = np.clip(np.rint(g / scale[..., None]) + zero[..., None], 0, qmax)
    q = q.reshape(N, Kp)[:, :K].astype(np.int32)
    return q, scale, zero


def dequantize(q: np.ndarray, scales: np.ndarray, zeros: np.ndarray, group_size: int) -> np.ndarray:
    """(q - z) * s in fp32 with the per-group metadata repeated along K (reference.py:30-34)."""
    K = q.shape[1]
    s = np.repeat(np.asarray(scales, dtype=np.float32), group_size, axis=1)[:, :K]
    z = np.repeat(np.asarray(zeros, dtype=np.float32), group_size, axis=1)[:, :K]
    return ((q.astype(np.float32) - z) * s).astype(np.float32)


def pack_codes(q: np.ndarray, bits: int) -> np.ndarray:
    """LSB-first bitstream per row, rows padded to 32-code chunks (reference.py:37-55).

    Code k of a row occupies bits [k*bits, (k+1)*bits) of the row's bitstream; each
    32-code chunk takes exactly ``bits`` words, so chunks start on word boundaries.
    Returned as int32 (two's complement view of the uint32 words).
    """
    assert bits in (2, 3, 4)
    q = np.asarray(q)
    N, K = q.shape
    C = math.ceil(K / 32)
    qq = np.zeros((N, C * 32), dtype=np.uint64)
    qq[:, :K] = q.astype(np.uint64) & np.uint64((1 << bits) - 1)
    qq = qq.reshape(N, C, 32)
    words = np.zeros((N, C, bits + 1), dtype=np.uint64)
    for j in range(32):
        pos = j * bits
        wi, off = pos // 32, pos % 32
        v = qq[:, :, j] << np.uint64(off)
        words[:, :, wi] |= v & np.uint64(0xFFFFFFFF)
        words[:, :, wi + 1] |= v >> np.uint64(32)
    assert not words[:, :, bits].any()
    w = words[:, :, :bits].reshape(N, C * bits).astype(np.uint32)
    return w.view(np.int32).copy()


def unpack_codes(packed: np.ndarray, bits: int, K: int) -> np.ndarray:
    """Random-access inverse of pack_codes (reference.py:58-67): int32 [N, K]."""
    w = np.asarray(packed).astype(np.int64) & 0xFFFFFFFF
    k = np.arange(K)
    pos = k * bits
    wi, off = pos // 32, pos % 32
    lo = w[:, wi] >> off
    nxt = np.minimum(wi + 1, w.shape[1] - 1)
    hi = np.where(off + bits > 32, w[:, nxt] << (32 - off), 0)
    return ((lo | hi) & ((1 << bits) - 1)).astype(np.int32)


def unpack_codes_by_slot(packed: np.ndarray, bits: int, K: int) -> np.ndarray:
    """unpack_codes computed one code slot of the 32-code chunk at a time: slot j of every
    chunk of every row sits at the same word and bit offset (word (j bits) >> 5 of the
    chunk, offset (j bits) & 31, joined with the next word when it straddles), so each slot
    is one shift / or / mask over an [N, C] array of words (int64 torch tensors on the host
    cores).  Same result as unpack_codes (checked in tests/test_oracle_format.py), an order
    of magnitude faster on Llama-sized rows; used where the checker runs at the bench's full
    sizes."""
    import torch
    w = torch.from_numpy(np.ascontiguousarray(packed).view(np.uint32).astype(np.int64))
    N = w.shape[0]
    C = w.shape[1] // bits
    w = w.view(N, C, bits)
    q = torch.empty((N, C, 32), dtype=torch.int32)
    mask = (1 << bits) - 1
    for j in range(32):
        pos = j * bits
        wi, off = pos >> 5, pos & 31
        v = w[:, :, wi] >> off
        if off + bits > 32:
            v = v | (w[:, :, wi + 1] << (32 - off))
        q[:, :, j] = (v & mask).to(torch.int32)
    return q.view(N, C * 32)[:, :K].numpy()


def chunk_code(words, j: int, bits: int) -> int:
    """Code j of one 32-code chunk held in ``bits`` words (bitpack.cuh:35-41 semantics)."""
    pos = j * bits
    wi, off = pos >> 5, pos & 31
    v = (int(words[wi]) & 0xFFFFFFFF) >> off
    if off + bits > 32:
        v |= (int(words[wi + 1]) & 0xFFFFFFFF) << (32 - off)
    return v & ((1 << bits) - 1)


def code_to_float(q: int) -> float:
    """u32 -> fp32 via the 2^23 magic constant (bitpack.cuh:44-46)."""
    f = np.array([q | 0x4B000000], dtype=np.uint32).view(np.float32)[0]
    return float(f - np.float32(8388608.0))


def pack_linear_dict(weight: np.ndarray, bits: int, group_size: int = 128, bias=None,
                     meta_dtype=np.float16) -> dict:
    """Quantize + pack one linear, metadata cast to ``meta_dtype`` (reference.py:70-76)."""
    q, s, z = quantize_affine(weight, bits, group_size)
    return dict(packed=pack_codes(q, bits), scales=s.astype(meta_dtype), zeros=z.astype(meta_dtype),
                bits=bits, group_size=group_size, in_features=weight.shape[1],
                out_features=weight.shape[0],
                bias=None if bias is None else np.asarray(bias).astype(meta_dtype))


def dequantized_weight(d: dict) -> np.ndarray:
    """fp32 W-hat of a packed dict (reference.py:79-82)."""
    q = unpack_codes(d["packed"], d["bits"], d["in_features"])
    return dequantize(q, np.asarray(d["scales"], np.float32), np.asarray(d["zeros"], np.float32),
                      d["group_size"])


# ---------------------------------------------------------------- the second producer
# quantization/crispybits_quant (the paper's offline quantizer, used by
# quantization/scripts/pack_checkpoint.py): a zero-inclusive affine quantizer and a
# continuous bitstream packer.  The kernels consume the chunked format above; these two
# restatements let the product's converter and device producer be checked against them.

def affine_quantize_weight(w: np.ndarray, bits: int, group_size: int = 128, eps: float = 1e-8):
    """Zero-inclusive affine quantization (crispybits_quant/affine.py:28-71).

    Per row and group [s, e) of the real columns (no padding): min clamped to <= 0 and
    max to >= 0 (affine.py:51-52), scale = (max - min) / qmax replaced by 1 where it is
    below eps (affine.py:53-55), zero = clamp(round(-min / scale), 0, qmax), and
    q = clamp(round(w / scale + zero), 0, qmax) -- the zero is added before rounding
    (affine.py:57-58).  All fp32.  Returns (q int32 [N, K], scale fp32 [N, G], zero fp32 [N, G]).
    """
    assert bits in (2, 3, 4)
    w = np.asarray(w, dtype=np.float32)
    N, K = w.shape
    G = math.ceil(K / group_size)
    qmax = np.float32((1 << bits) - 1)
    q = np.empty((N, K), dtype=np.int32)
    scale = np.empty((N, G), dtype=np.float32)
    zero = np.empty((N, G), dtype=np.float32)
    for g in range(G):
        s, e = g * group_size, min(K, (g + 1) * group_size)
        wg = w[:, s:e]
        mn = np.minimum(wg.min(1), np.float32(0))
        mx = np.maximum(wg.max(1), np.float32(0))
        sc = ((mx - mn) / qmax).astype(np.float32)
        sc = np.where(sc < np.float32(eps), np.float32(1), sc).astype(np.float32)
        zr = np.clip(np.rint(-mn / sc), 0, qmax).astype(np.float32)
        y = (wg / sc[:, None]).astype(np.float32) + zr[:, None]
        q[:, s:e] = np.clip(np.rint(y), 0, qmax).astype(np.int32)
        scale[:, g], zero[:, g] = sc, zr
    return q, scale, zero


def pack_codes_continuous(q: np.ndarray, bits: int) -> np.ndarray:
    """One LSB-first bitstream per row with no chunk padding: ceil(K * bits / 32) words
    (crispybits_quant/packing.py:24-25,45-54).  Equal to pack_codes when K % 32 == 0."""
    assert bits in (2, 3, 4)
    q = np.asarray(q)
    N, K = q.shape
    W = (K * bits + 31) // 32
    words = np.zeros((N, W + 1), dtype=np.uint64)
    for k in range(K):
        pos = k * bits
        wi, off = pos // 32, pos % 32
        v = (q[:, k].astype(np.uint64) & np.uint64((1 << bits) - 1)) << np.uint64(off)
        words[:, wi] |= v & np.uint64(0xFFFFFFFF)
        words[:, wi + 1] |= v >> np.uint64(32)
    assert not words[:, W].any()
    return words[:, :W].astype(np.uint32).view(np.int32).copy()


def unpack_codes_continuous(packed: np.ndarray, K: int, bits: int) -> np.ndarray:
    """Inverse of pack_codes_continuous (packing.py:62-80): int32 [N, K].  The bit
    arithmetic is the same random access as unpack_codes -- in both formats code k sits
    at bit k*bits of the row -- only the row length in words differs."""
    return unpack_codes(packed, bits, K)


def continuous_to_chunked(packed: np.ndarray, bits: int, K: int) -> np.ndarray:
    """Re-pack a continuous-bitstream row set into the kernels' chunked format."""
    return pack_codes(unpack_codes_continuous(packed, K, bits), bits)

