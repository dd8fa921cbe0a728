"""GPU parity of the fp32 matrix-core decode (csrc/gemv_any.hip), the row-pair finish stage
in every mode, the split-K combine launch and counter windows, and the fp32 prefill GEMM
(csrc/gemm_f32.hip), against the oracle's float64 dequant-matmul on the same seeded inputs.

Bars, as in test_gpu_parity: max|y - ref| / max|ref| below the reference's tolerances
(fp16 3e-3, bf16 2e-2, fp32 1e-4; Kernel/tests/test_correctness.py:10).  Each case that
targets a kernel family first asserts that the library's plan takes it (_C.decode_plan,
which plans for 256-byte aligned tensors as torch allocates them).
"""
import numpy as np
import pytest
import torch

from crispybits_kernels import _C, fused_gate_up, fused_qkv, ops, packed_linear, permute_for_rope
from oracle import emulator as E
from test_gpu_parity import _rope64, _rope_tables, close, gemm_ref, make, randx, ref_linear

pytestmark = pytest.mark.gpu

BASELINE = [(4096, 4096), (4096, 11008), (11008, 4096)]


def plan(dtype, M, K, gs, out, bits, kind="gemv", split_k=1):
    fam, splits, grid, threads, lds, launches = _C.decode_plan(dtype, M, K, gs, out, bits, kind, split_k, 1)
    return fam, splits, threads, launches


def fp32_family(M, K, gs=128):
    """Decode family of an fp32 call: streaming at batch 1, the batched streaming kernel at
    batch 2..8 (two operand rows per batch row, 16 at most; groups of whole 128-code units), the
    fp32 matrix-core kernel otherwise."""
    if M == 1:
        return "stream"
    return "bstream" if 2 <= M <= 8 and gs % 128 == 0 else "generic"


# ------------------------------------------------------------------ fp32 activations

@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("K,N", BASELINE)
@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_fp32_decode_baseline_shapes(hip, bits, K, N, M):
    """fp32 x at the BASELINE decode shapes: the streaming kernel at batch 1 (two fp16 operand
    rows per chunk) and the batched streaming kernel at batch 2, 4 and 8 (two operand rows per
    batch row; K splits combined in the dispatch where the staged rows need them); one launch,
    within the fp32 bar."""
    fam, splits, threads, launches = plan(torch.float32, M, K, 128, N, bits)
    assert (fam, launches) == (fp32_family(M, K), 1), (fam, splits, launches)
    assert splits == 1 or fam == "bstream", (fam, splits)
    assert threads % 64 == 0 and 64 <= threads <= 1024
    w, W64, _, _ = make(N, K, bits, torch.float32, scale=0.02)
    x = randx(M, K, torch.float32, seed=10 + M)
    close(packed_linear(x, w, decode_threshold=16), ref_linear(x, W64), torch.float32)


@pytest.mark.parametrize("split_k", [2, 5, 64])
@pytest.mark.parametrize("M", [1, 2, 3, 8, 16, 20])
def test_fp32_decode_splits(hip, split_k, M):
    """K splits of the fp32 decode (the streaming kernel at batch 1, the batched streaming
    kernel at 2-8, the fp32 matrix-core kernel above) combine inside the dispatch (the last
    split of each block adds the partials); the result matches the unsplit call within the bar
    and repeats bit for bit.  The batched kernel may add up to 3 splits to fill the CUs."""
    w, W64, b64, _ = make(600, 4128, 3, torch.float32, bias=True)
    x = randx(M, 4128, torch.float32, seed=M)
    fam, splits, _, launches = plan(torch.float32, M, 4128, 128, 600, 3, split_k=split_k)
    assert fam == fp32_family(M, 4128) and launches == 1, (fam, splits, launches)
    units = -(-4128 // 128)
    if fam == "bstream":
        assert min(split_k, units) <= splits <= split_k + 3, splits
    else:
        assert splits == split_k, splits
    y = packed_linear(x, w, split_k, 1, "silu", decode_threshold=32)
    close(y, ref_linear(x, W64, b64, "silu"), torch.float32)
    assert torch.equal(packed_linear(x, w, split_k, 1, "silu", decode_threshold=32), y)


@pytest.mark.parametrize("dist", ["normal", "wide", "tiny", "outlier"])
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("K,N", BASELINE)
def test_fp32_streaming_activation_ranges(hip, dist, bits, K, N):
    """fp32 x at batch 1 on the streaming kernel: each 32-code chunk is prescaled by its own
    power of two and split into two fp16 operands (hi, lo), so fp32 activations of any range
    keep fp32 accuracy -- N(0,1), values spread over 2^-40..2^40 ("wide"), all below 1e-30
    ("tiny") and a few channels 1e4 times the rest ("outlier") -- within the fp32 bar."""
    assert plan(torch.float32, 1, K, 128, N, bits)[0] == "stream"
    w, W64, _, _ = make(N, K, bits, torch.float32, scale=0.02)
    g = torch.Generator().manual_seed(bits + K)
    x = torch.randn(1, K, generator=g, dtype=torch.float64)
    if dist == "wide":
        x = x * torch.exp2(torch.randint(-40, 41, (1, K), generator=g).double())
    elif dist == "tiny":
        x = x * 1e-32
    elif dist == "outlier":
        x[0, torch.randperm(K, generator=g)[:4]] *= 1e4
    x = x.float().cuda()
    close(packed_linear(x, w), ref_linear(x, W64), torch.float32)


@pytest.mark.parametrize("gs", [32, 64, 256])
@pytest.mark.parametrize("K", [200, 1000, 4128])
@pytest.mark.parametrize("M", [1, 2])
def test_fp32_streaming_groups_and_ragged_k(hip, gs, K, M):
    """Batch-1 and -2 fp32 with group sizes 32..256 and K not a multiple of 32 (the last
    chunk's pieces past K read as zero), bias and SiLU, against the oracle: the streaming kernel
    at batch 1; at batch 2 the batched kernel for groups of 256, the fp32 matrix-core kernel for
    groups of 32 and 64."""
    w, W64, b64, _ = make(300, K, 3, torch.float32, bias=True, gs=gs)
    x = randx(M, K, torch.float32, seed=K + M)
    assert plan(torch.float32, M, K, gs, 300, 3)[0] == fp32_family(M, K, gs)
    close(packed_linear(x, w, act="silu"), ref_linear(x, W64, b64, "silu"), torch.float32)


@pytest.mark.parametrize("dist", ["normal", "wide", "tiny", "outlier"])
@pytest.mark.parametrize("K,N", BASELINE)
@pytest.mark.parametrize("M", [2, 3, 5, 8])
def test_fp32_batched_activation_ranges(hip, dist, K, N, M):
    """fp32 x at batch 2..8 on the batched streaming kernel: each batch row is staged as two fp16
    operand rows (hi, lo) behind one power-of-two prescale per 128-code unit, so fp32 activations
    of any range keep fp32 accuracy (the activation ranges of the batch-1 test; batch rows of
    different magnitude), within the fp32 bar."""
    assert plan(torch.float32, M, K, 128, N, 3)[0] == "bstream"
    w, W64, _, _ = make(N, K, 3, torch.float32, scale=0.02)
    g = torch.Generator().manual_seed(K + M)
    x = torch.randn(M, K, generator=g, dtype=torch.float64)
    if dist == "wide":
        x = x * torch.exp2(torch.randint(-40, 41, (M, K), generator=g).double())
    elif dist == "tiny":
        x = x * 1e-32
    elif dist == "outlier":
        x[:, torch.randperm(K, generator=g)[:4]] *= 1e4
        x[M - 1] *= 1e-3
    x = x.float().cuda()
    close(packed_linear(x, w, decode_threshold=16), ref_linear(x, W64), torch.float32)


@pytest.mark.parametrize("gs", [128, 256])
@pytest.mark.parametrize("K", [1000, 4128, 11008])
@pytest.mark.parametrize("M", [3, 4, 7, 8])
def test_fp32_batched_groups_and_ragged_k(hip, gs, K, M):
    """Batch 3..8 fp32 on the batched streaming kernel with groups of 128 and 256 and K not a
    multiple of 32 or 128 (pieces past K read as zero), bias and SiLU, against the oracle."""
    w, W64, b64, _ = make(300, K, 4, torch.float32, bias=True, gs=gs)
    x = randx(M, K, torch.float32, seed=K + M)
    assert plan(torch.float32, M, K, gs, 300, 4)[0] == "bstream"
    y = packed_linear(x, w, act="silu", decode_threshold=16)
    close(y, ref_linear(x, W64, b64, "silu"), torch.float32)


@pytest.mark.parametrize("B", [1, 2, 5, 8, 16])
@pytest.mark.parametrize("split_k", [1, 3])
def test_fp32_fused_gate_up(hip, B, split_k):
    """Fused gate-up with fp32 x -- the streaming kernel at batch 1, the batched streaming kernel
    at 2..8, the fp32 matrix-core kernel at 16 -- with and without K splits, against the oracle."""
    g, G64, _, _ = make(11008 // 8, 4096, 3, torch.float32, seed=4)
    u, U64, _, _ = make(11008 // 8, 4096, 3, torch.float32, seed=5)
    x = randx(B, 4096, torch.float32, seed=B)
    gv, uv = ref_linear(x, G64), ref_linear(x, U64)
    ref = E.silu64(gv) * uv
    close(fused_gate_up(x, g, u, split_k), ref, torch.float32)


@pytest.mark.parametrize("bits", [3, (4, 2, 3)])
@pytest.mark.parametrize("B", [1, 2, 4, 8, 17])
@pytest.mark.parametrize("rope,head_dim", [(False, 0), (False, 64), (True, 64)])
def test_fp32_fused_qkv(hip, bits, B, rope, head_dim):
    """Fused QKV (GQA widths, bias, mixed widths, RoPE on pair-interleaved Q/K) through the
    fp32 kernel: each stored pair is finished by one thread, both rotated outputs at once."""
    bq, bk, bv = bits if isinstance(bits, tuple) else (bits,) * 3
    K, hd = 512, (head_dim or 64)
    q, Q64, qb, _ = make(6 * hd, K, bq, torch.float32, True, 1)
    k, K64, kb, _ = make(2 * hd, K, bk, torch.float32, True, 2)
    v, V64, vb, _ = make(2 * hd, K, bv, torch.float32, True, 3)
    if head_dim:
        q, k = permute_for_rope(q, head_dim), permute_for_rope(k, head_dim)
    x = randx(B, K, torch.float32, seed=B)
    rq, rk, rv = ref_linear(x, Q64, qb), ref_linear(x, K64, kb), ref_linear(x, V64, vb)
    r = None
    if rope:
        cos, sin = _rope_tables(B, head_dim)
        rq, rk = _rope64(rq, cos, sin, head_dim), _rope64(rk, cos, sin, head_dim)
        r = (cos.cuda(), sin.cuda(), head_dim)
    oq, ok, ov = fused_qkv(x, q, k, v, 1, 1, rope=r, decode_threshold=32)
    for o, ref in ((oq, rq), (ok, rk), (ov, rv)):
        close(o, ref, torch.float32)


# ------------------------------------------------------------------ 16-bit shapes the streaming kernels do not take

@pytest.mark.parametrize("gs", [32, 64])
@pytest.mark.parametrize("M", [3, 8, 16])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_small_groups_batched(hip, gs, M, dtype):
    """Group sizes 32 and 64 at batch 3..16 go to the fp32 matrix-core kernel."""
    fam, *_ = plan(dtype, M, 2048, gs, 1000, 3)
    assert fam == "generic", fam
    w, W64, _, _ = make(1000, 2048, 3, dtype, gs=gs)
    x = randx(M, 2048, dtype, seed=M)
    close(packed_linear(x, w, 2, 1), ref_linear(x, W64), dtype)


@pytest.mark.parametrize("M", [17, 40])
@pytest.mark.parametrize("bits", [2, 4])
def test_batches_past_16(hip, M, bits):
    """Past 16 rows (a raised decode threshold) the decode takes 16-row batch tiles."""
    fam, *_ = plan(torch.float16, M, 768, 128, 1000, bits)
    assert fam == "generic", fam
    w, W64, _, _ = make(1000, 768, bits, torch.float16)
    x = randx(M, 768, torch.float16, seed=M)
    close(packed_linear(x, w, 1, 1, decode_threshold=64), ref_linear(x, W64), torch.float16)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M", [1, 2, 6])
def test_unaligned_activations(hip, dtype, M):
    """A contiguous x whose rows do not start on 16-byte boundaries (a view one element into
    its buffer): the streaming kernels refuse it and the fp32 matrix-core kernel takes
    element loads."""
    w, W64, _, _ = make(300, 1000, 3, dtype)
    flat = randx(1, M * 1000 + 1, dtype, seed=50 + M)[0]
    xu = flat[1:].view(M, 1000)
    assert xu.is_contiguous() and xu.data_ptr() % 16 != 0
    y = _C.packed_gemv(xu, w.packed, w.scales, w.zeros, None, 3, 1000, 128, 1, 1, 0, None)
    close(y, ref_linear(xu, W64), dtype)
    y2 = _C.packed_gemv(xu, w.packed, w.scales, w.zeros, None, 3, 1000, 128, 3, 1, 0, None)
    close(y2, ref_linear(xu, W64), dtype)


def test_qkv_odd_widths(hip):
    """Q/K/V widths that are not multiples of 16 (and an odd Q width): tiles and finish
    pairs that straddle projections."""
    K = 256
    q, Q64, qb, _ = make(101, K, 4, torch.float16, True, 1)
    k, K64, kb, _ = make(40, K, 2, torch.float16, True, 2)
    v, V64, vb, _ = make(27, K, 3, torch.float16, True, 3)
    for B in (1, 5):
        x = randx(B, K, torch.float16, seed=B)
        oq, ok, ov = fused_qkv(x, q, k, v)
        close(oq, ref_linear(x, Q64, qb), torch.float16)
        close(ok, ref_linear(x, K64, kb), torch.float16)
        close(ov, ref_linear(x, V64, vb), torch.float16)


@pytest.mark.parametrize("widths,fam", [((102, 40, 26), "generic"), ((104, 40, 28), "stream"),
                                        ((100, 36, 30), "stream")])
def test_qkv_widths_per_wave(hip, widths, fam):
    """Batch-1 fused QKV with one width: the streaming kernel resolves a wave's 4 rows to
    one projection, so it takes Q and K widths that are multiples of 4 (any V width); other
    widths go to the fp32 matrix-core kernel.  Both within the fp16 bar, with biases."""
    K = 512
    assert plan(torch.float16, 1, K, 128, widths, 3, "qkv")[0] == fam
    ws = [make(n, K, 3, torch.float16, True, s + 1) for s, n in enumerate(widths)]
    x = randx(1, K, torch.float16, seed=7)
    for o, (w, W64, b64, _) in zip(fused_qkv(x, *(t[0] for t in ws)), ws):
        close(o, ref_linear(x, W64, b64), torch.float16)


# ------------------------------------------------------------------ split counters and the combine launch

def _hip_runtime():
    """The HIP runtime torch loaded (by its soname, so the same instance)."""
    import ctypes
    return ctypes.CDLL("libamdhip64.so.7")


def test_split_windows_exhausted_take_the_combine_launch(hip):
    """More streams than counter windows (300 distinct HIP streams > 256 windows), each with
    split calls in flight at once: streams past the last free window take the combine launch
    instead of sharing a window.  Both paths add the splits in the same order, so every
    result equals the single-stream result bit for bit.  (torch.cuda.Stream() hands out
    pooled streams, so the streams here are created with hipStreamCreate and wrapped.)"""
    import ctypes
    w, W64, _, _ = make(4096, 11008, 3, torch.float16, scale=0.02)
    x = randx(8, 11008, torch.float16, seed=3)
    fam, splits, _, launches = plan(torch.float16, 8, 11008, 128, 4096, 3)
    assert fam == "bstream" and splits > 1 and launches == 1
    y = packed_linear(x, w)
    close(y, ref_linear(x, W64), torch.float16)
    torch.cuda.synchronize()
    rt = _hip_runtime()
    handles = []
    try:
        for _ in range(300):
            h = ctypes.c_void_p()
            assert rt.hipStreamCreate(ctypes.byref(h)) == 0
            handles.append(h)
        outs = []
        for h in handles:
            st = torch.cuda.ExternalStream(h.value)
            st.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(st):
                outs.append([packed_linear(x, w) for _ in range(2)])
        torch.cuda.synchronize()
        for o in outs:
            for t in o:
                assert torch.equal(t, y)
    finally:
        torch.cuda.synchronize()
        for h in handles:
            rt.hipStreamDestroy(h)


def test_captured_split_window_is_not_shared_with_eager_calls(hip):
    """A graph captured with split calls keeps a window of its own: replays on a second
    stream while the capturing stream runs eager split calls give the eager results."""
    w, W64, _, _ = make(4096, 11008, 3, torch.float16, scale=0.02)
    x = randx(8, 11008, torch.float16, seed=4)
    y0 = packed_linear(x, w)
    torch.cuda.synchronize()
    cap = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        packed_linear(x, w)                                 # warm-up on the capture stream
        cap.synchronize()
        with torch.cuda.graph(g, stream=cap):
            yg = packed_linear(x, w)
    torch.cuda.synchronize()
    other = torch.cuda.Stream()
    for i in range(3):
        other.wait_stream(torch.cuda.current_stream())
        cap.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(other):
            g.replay()
        with torch.cuda.stream(cap):
            eager = [packed_linear(x, w) for _ in range(4)]
        torch.cuda.synchronize()
        assert torch.equal(yg, y0)
        for t in eager:
            assert torch.equal(t, y0)


# ------------------------------------------------------------------ fp32 prefill GEMM

@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("M,K,N", [(1, 400, 260), (70, 640, 300), (130, 4096, 512), (1024, 4096, 1024)])
def test_prefill_fp32(hip, bits, M, K, N):
    """fp32 x: W-hat kept in fp32 and fp32 accumulation, within the fp32 bar."""
    w, W64, b64, d = make(N, K, bits, torch.float32, bias=True)
    x = randx(M, K, torch.float32, seed=M)
    for act in (None, "relu"):
        y = _C.packed_gemm(x, w.packed, w.scales, w.zeros, w.bias, bits, K, 128, ops.ACT[act], True)
        close(y, ref_linear(x, W64, b64, act), torch.float32)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("gs", [32, 128])
def test_prefill_without_matrix_cores_16bit(hip, dtype, gs):
    """use_tensor_cores=False with 16-bit x: the fp32 kernel, W-hat not rounded to T; the
    only rounding is the output's, so the error stays far inside the dtype's bar."""
    w, W64, _, d = make(300, 1000, 3, dtype, gs=gs)
    x = randx(90, 1000, dtype)
    y = _C.packed_gemm(x, w.packed, w.scales, w.zeros, None, 3, 1000, gs, 0, False)
    ref = ref_linear(x, W64)
    close(y, ref, dtype)
    err = np.abs(y.double().cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err < (4.5e-3 if dtype == torch.bfloat16 else 6e-4), err
    # rows of K % 8 != 0 codes (no vector activation loads) through the same kernel
    w2, W2, _, _ = make(64, 999, 2, dtype, gs=gs)
    x2 = randx(33, 999, dtype)
    y2 = _C.packed_gemm(x2, w2.packed, w2.scales, w2.zeros, None, 2, 999, gs, 0, False)
    close(y2, ref_linear(x2, W2), dtype)
