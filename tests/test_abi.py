"""The C-ABI library loads and exports every entry point include/crispybits_hip.h
declares, and rejects invalid arguments before touching a device (no GPU needed)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "crispybits_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cbk_\w+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = _declared()
    for n in ("cbk_packed_gemv", "cbk_packed_gemm", "cbk_fused_gate_up", "cbk_fused_qkv", "cbk_sm_count",
              "cbk_tile_n", "cbk_max_rho", "cbk_unpack_codes", "cbk_quantize_pack"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from crispybits_kernels import _C
    import cabi
    lib = ctypes.CDLL(_C.LIB_PATH)
    for name in _declared():
        assert hasattr(lib, name), name
    assert set(_declared()) == set(cabi.SIGS)          # every entry point is callable from the tests
    assert _C.ABI_VERSION == 1
    assert _C.tile_n() == 16


def test_op_module_binds_the_reference_functions():
    """The compiled op module exports the reference's seven _C functions (bindings.cpp:32-40)
    plus the additive ones, and its checks raise RuntimeError without touching a device."""
    import torch
    from crispybits_kernels import _C
    for name in ("packed_gemv", "packed_gemm", "fused_gate_up", "fused_qkv", "sm_count", "tile_n", "max_rho",
                 "packed_gemm_gate_up", "unpack_codes", "quantize_pack", "decode_plan", "timer_start",
                 "timer_stop", "stream_probe"):
        assert callable(getattr(_C, name)), name
    x = torch.zeros(1, 256)
    w = torch.zeros(4, 32, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="x must be CUDA"):
        _C.packed_gemv(x, w, torch.zeros(4, 2), torch.zeros(4, 2), None, 4, 256, 128, 1, 1, 0, None)
    with pytest.raises(RuntimeError, match="kind must be"):
        _C.max_rho(3, "nope")


def _lib():
    import cabi
    return cabi.lib


def _err():
    return _lib().cbk_last_error().decode()


ALIGNED = 1 << 20          # a fake, 16-byte aligned "device" address: never dereferenced


def _gemv(**kw):
    a = dict(x=ALIGNED, dtype=0, M=1, K=256, packed=ALIGNED, scales=ALIGNED, zeros=ALIGNED, bias=None, N=64, bits=4,
             gs=128, split_k=1, rho=1, act=0, ws=None, partial=None, out=ALIGNED, device=0, stream=None)
    a.update(kw)
    return _lib().cbk_packed_gemv(*a.values())


@pytest.mark.parametrize("kw,msg", [
    (dict(bits=5), "bits must be 2/3/4"),
    (dict(gs=48), "group_size must be a positive multiple of 32"),
    (dict(gs=0), "group_size must be a positive multiple of 32"),
    (dict(dtype=7), "x must be fp16/bf16/fp32"),
    (dict(split_k=0), "split_k must be >= 1"),
    (dict(act=3), "act must be 0 (none), 1 (relu) or 2 (silu)"),
    (dict(packed=ALIGNED + 4), "16-byte aligned"),
    (dict(bits=2, packed=ALIGNED + 4), "8-byte aligned"),
    (dict(K=0), "in_features"),
    (dict(out=None), "out must be non-null"),
    (dict(scales=None), "non-null"),
])
def test_gemv_argument_errors(kw, msg):
    assert _gemv(**kw) == 1
    assert msg in _err()


def test_w3_only_needs_word_alignment_and_empty_batch_is_a_no_op():
    assert _gemv(bits=3, packed=ALIGNED + 4, M=0) == 0       # validated, nothing launched


def test_gemm_and_unpack_argument_errors():
    lib = _lib()
    assert lib.cbk_packed_gemm(ALIGNED, 0, 4, 256, ALIGNED, ALIGNED, ALIGNED, None, 64, 4, 100, 0, 1, ALIGNED, 0,
                               None) == 1
    assert "group_size" in _err()
    assert lib.cbk_unpack_codes(ALIGNED, 4, 64, 1, ALIGNED, 0, None) == 1
    assert "bits" in _err()


def _gate_up(**kw):
    a = dict(x=ALIGNED, dtype=0, M=4, K=256, pg=ALIGNED, sg=ALIGNED, zg=ALIGNED, pu=ALIGNED, su=ALIGNED,
             zu=ALIGNED, N=64, bits=4, gs=128, out=ALIGNED, device=0, stream=None)
    a.update(kw)
    return _lib().cbk_packed_gemm_gate_up(*a.values())


@pytest.mark.parametrize("kw,rc,msg", [
    (dict(bits=5), 1, "bits must be 2/3/4"),
    (dict(pu=None), 1, "packed_gemm_gate_up(up): packed/scales/zeros must be non-null"),
    (dict(gs=48), 1, "group_size must be a positive multiple of 32"),
    (dict(out=None), 1, "out must be non-null"),
    (dict(dtype=2), 3, "x must be fp16 or bf16"),
    (dict(K=260), 3, "K % 8 == 0"),
    (dict(x=ALIGNED + 8), 3, "16-byte aligned"),
    (dict(bits=2, zu=ALIGNED + 2), 3, "16-byte aligned"),
])
def test_gemm_gate_up_argument_errors(kw, rc, msg):
    """Invalid arguments are CBK_EINVAL; calls the one-launch kernel cannot take are
    CBK_ENOTSUP (the op binding then runs two GEMMs and a product); neither launches."""
    assert _gate_up(**kw) == rc
    assert msg in _err()


def test_gemm_gate_up_empty_batch_is_a_no_op():
    assert _gate_up(M=0) == 0


@pytest.mark.parametrize("kw,msg", [
    (dict(dtype=5), "weights must be fp16/bf16/fp32"),
    (dict(mdt=9), "scales/zeros must be fp16/bf16/fp32"),
    (dict(bits=1), "bits must be 2/3/4"),
    (dict(gs=100), "positive multiple of 32"),
    (dict(K=0), "bad shape"),
    (dict(zeros=None), "non-null"),
    (dict(scheme=2), "scheme must be 0"),
])
def test_quantize_pack_argument_errors(kw, msg):
    a = dict(w=ALIGNED, dtype=0, N=8, K=256, bits=3, gs=128, scheme=0, packed=ALIGNED, scales=ALIGNED, zeros=ALIGNED,
             mdt=0, device=0, stream=None)
    a.update(kw)
    assert _lib().cbk_quantize_pack(*a.values()) == 1
    assert msg in _err()


def test_quantize_pack_empty_weight_is_a_no_op():
    assert _lib().cbk_quantize_pack(None, 0, 0, 256, 4, 128, 0, None, None, None, 0, 0, None) == 0


def test_fused_qkv_rope_checks():
    lib = _lib()
    args = [ALIGNED, 0, 1, 256] + [ALIGNED, ALIGNED, ALIGNED, None, 256] * 3
    # RoPE tables without pair-interleaved Q/K
    rc = lib.cbk_fused_qkv(*args, ALIGNED, ALIGNED, 128, 0, 4, 128, 1, 1, None, None, ALIGNED, ALIGNED, ALIGNED,
                           0, None)
    assert rc == 1 and "pair-interleaved" in _err()
    rc = lib.cbk_fused_qkv(*args, None, None, 0, 6, 4, 128, 1, 1, None, None, ALIGNED, ALIGNED, ALIGNED, 0, None)
    assert rc == 1 and "multiples of head_dim" in _err()


def test_partial_query():
    lib = _lib()
    assert lib.cbk_gemv_partial_floats(0, 1, 4096, 4096, 128, 1) == 0
    assert lib.cbk_gemv_partial_floats(0, 2, 4096, 4096, 128, 4) == 4 * 2 * 4096
    # fp16 batch 16 x K 16384 needs more LDS than one workgroup holds -> forced split
    assert lib.cbk_gemv_partial_floats(0, 16, 64, 16384, 128, 1) > 0
    # fp32 batch 8 stages 16 operand rows: K 11008 needs at least 3 splits for the LDS
    assert lib.cbk_gemv_partial_floats(2, 8, 4096, 11008, 128, 1) >= 3 * 8 * 4096
