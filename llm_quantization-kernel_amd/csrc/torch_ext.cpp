// torch_ext.cpp -- the torch-facing op module (crispybits_kernels._ext), a thin PyTorch-ROCm C++
// extension over the C ABI of libcrispybits_hip.so (include/crispybits_hip.h).
//
// Replaces the reference's pybind11 module (Kernel/csrc/bindings.cpp:32-40): the same seven
// functions with the same argument order -- packed_gemv, packed_gemm, fused_gate_up, fused_qkv,
// sm_count, tile_n, max_rho -- tensors in and tensors out, plus the additive entries of this build
// (unpack_codes, quantize_pack, decode_plan, timer_start / timer_stop, stream_probe).  Tensor checks restate
// host_utils.h:38-87 and fail through TORCH_CHECK (RuntimeError in Python); "no bias / no RoPE /
// no workspace" may be None or an empty tensor (ops.py:74-83).  Outputs and split-K partials come
// from torch's caching allocator on x's device; the kernels run on torch's current HIP stream of
// that device.  No device code here and no hipify: the launches are the C ABI's.
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <mutex>
#include <string>
#include <tuple>
#include <unordered_map>
#include <vector>

#include "crispybits_hip.h"

namespace {

using at::Tensor;
using OptT = c10::optional<Tensor>;

void ok(int rc) { TORCH_CHECK(rc == CBK_OK, cbk_last_error()); }

int dtype_of(at::ScalarType t) {
    switch (t) {
        case at::kHalf: return CBK_F16;
        case at::kBFloat16: return CBK_BF16;
        case at::kFloat: return CBK_F32;
        default: return -1;
    }
}

void* stream_of(int device) { return c10::hip::getCurrentHIPStream(device).stream(); }

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

void check_x(const Tensor& x, int64_t K) {
    TORCH_CHECK(x.is_cuda(), "x must be CUDA");
    TORCH_CHECK(x.dim() == 2, "x must be [B,K]");
    TORCH_CHECK(x.is_contiguous(), "x must be contiguous");
    TORCH_CHECK(x.size(1) == K, "x K != in_features");
    TORCH_CHECK(dtype_of(x.scalar_type()) >= 0, "x must be fp16/bf16/fp32");
}

void check_weight(const Tensor& x, const Tensor& packed, const Tensor& scales, const Tensor& zeros, int64_t bits,
                  int64_t K, int64_t gs, const char* name) {
    TORCH_CHECK(packed.is_cuda() && scales.is_cuda() && zeros.is_cuda(), name, ": tensors must be CUDA");
    TORCH_CHECK(packed.device() == x.device() && scales.device() == x.device() && zeros.device() == x.device(),
                name, ": weight and activation on different devices");
    TORCH_CHECK(packed.scalar_type() == at::kInt, name, ": packed must be torch.int32");
    TORCH_CHECK(packed.dim() == 2 && scales.dim() == 2, name, ": packed/scales must be 2-D");
    TORCH_CHECK(packed.is_contiguous() && scales.is_contiguous() && zeros.is_contiguous(), name,
                ": weight tensors must be contiguous");
    TORCH_CHECK(scales.sizes() == zeros.sizes(), name, ": scale/zero shape mismatch");
    TORCH_CHECK(scales.size(0) == packed.size(0), name, ": metadata rows != output rows");
    TORCH_CHECK(scales.scalar_type() == x.scalar_type() && zeros.scalar_type() == x.scalar_type(), name,
                ": metadata dtype must match x");
    TORCH_CHECK(bits == 2 || bits == 3 || bits == 4, name, ": bits must be 2/3/4");
    TORCH_CHECK(gs > 0 && gs % 32 == 0, name, ": group_size must be a positive multiple of 32");
    TORCH_CHECK(packed.size(1) == cdiv(K, 32) * bits, name,
                ": packed row must hold exactly ceil(K/32)*bits words (rows padded to 32 codes)");
    TORCH_CHECK(scales.size(1) == cdiv(K, gs), name, ": expected ceil(K/group_size) groups");
}

// A present, non-empty optional tensor, or nullptr.
const void* opt_ptr(const OptT& t) { return t.has_value() && t->numel() > 0 ? t->data_ptr() : nullptr; }

const void* bias_ptr(const OptT& bias, const Tensor& x, int64_t N) {
    if (!bias.has_value() || bias->numel() == 0) return nullptr;
    TORCH_CHECK(bias->is_cuda() && bias->device() == x.device(), "bias must be on x's device");
    TORCH_CHECK(bias->numel() == N, "bias length must equal out_features");
    TORCH_CHECK(bias->scalar_type() == x.scalar_type(), "bias dtype must match x");
    TORCH_CHECK(bias->is_contiguous(), "bias must be contiguous");
    return bias->data_ptr();
}

int32_t* workspace_ptr(const OptT& ws, const Tensor& x) {
    if (!ws.has_value() || ws->numel() < 2) return nullptr;
    TORCH_CHECK(ws->is_cuda() && ws->device() == x.device(), "workspace must be on x's device");
    TORCH_CHECK(ws->scalar_type() == at::kInt && ws->is_contiguous(), "workspace must be contiguous int32");
    return ws->data_ptr<int32_t>();
}

// fp32 split-K partial buffer of a decode call (nullptr when the plan has one split); the
// library's element count is memoised per call shape.
struct PartialKey {
    int64_t dt, M, V, K, gs, split;
    bool operator==(const PartialKey& o) const {
        return dt == o.dt && M == o.M && V == o.V && K == o.K && gs == o.gs && split == o.split;
    }
};
struct PartialHash {
    size_t operator()(const PartialKey& k) const {
        size_t h = 1469598103934665603ull;
        for (int64_t v : {k.dt, k.M, k.V, k.K, k.gs, k.split}) h = (h ^ (size_t)v) * 1099511628211ull;
        return h;
    }
};
std::mutex g_partial_mu;
std::unordered_map<PartialKey, int64_t, PartialHash> g_partial;

Tensor partial_for(const Tensor& x, int64_t M, int64_t V, int64_t K, int64_t gs, int64_t split) {
    const PartialKey key{dtype_of(x.scalar_type()), M, V, K, gs, split};
    int64_t n;
    {
        std::lock_guard<std::mutex> lk(g_partial_mu);
        auto it = g_partial.find(key);
        if (it == g_partial.end()) {
            n = cbk_gemv_partial_floats((int)key.dt, M, V, K, (int)gs, (int)split);
            g_partial.emplace(key, n);
        } else {
            n = it->second;
        }
    }
    return n > 0 ? at::empty({n}, x.options().dtype(at::kFloat)) : Tensor();
}

void* tensor_ptr(const Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

// ------------------------------------------------------------------------------------- ops

Tensor packed_gemv(const Tensor& x, const Tensor& packed, const Tensor& scales, const Tensor& zeros, const OptT& bias,
                   int64_t bits, int64_t in_features, int64_t group_size, int64_t split_k, int64_t rho, int64_t act,
                   const OptT& workspace) {
    check_x(x, in_features);
    check_weight(x, packed, scales, zeros, bits, in_features, group_size, "packed_gemv");
    TORCH_CHECK(split_k >= 1, "split_k must be >= 1");
    TORCH_CHECK(act >= 0 && act <= 2, "act must be 0 (none), 1 (relu) or 2 (silu)");
    const int64_t N = packed.size(0), M = x.size(0);
    const void* b = bias_ptr(bias, x, N);
    int32_t* ws = workspace_ptr(workspace, x);
    Tensor out = at::empty({M, N}, x.options());
    if (M == 0) return out;
    const Tensor part = partial_for(x, M, N, in_features, group_size, split_k);
    const int dev = x.get_device();
    ok(cbk_packed_gemv(x.data_ptr(), dtype_of(x.scalar_type()), M, in_features, packed.data_ptr<int32_t>(),
                       scales.data_ptr(), zeros.data_ptr(), b, N, (int)bits, (int)group_size, (int)split_k, (int)rho,
                       (int)act, ws, static_cast<float*>(tensor_ptr(part)), out.data_ptr(), dev, stream_of(dev)));
    return out;
}

Tensor packed_gemm(const Tensor& x, const Tensor& packed, const Tensor& scales, const Tensor& zeros, const OptT& bias,
                   int64_t bits, int64_t in_features, int64_t group_size, int64_t act, bool use_tensor_cores) {
    check_x(x, in_features);
    check_weight(x, packed, scales, zeros, bits, in_features, group_size, "packed_gemm");
    TORCH_CHECK(act >= 0 && act <= 2, "act must be 0 (none), 1 (relu) or 2 (silu)");
    const int64_t N = packed.size(0), M = x.size(0);
    const void* b = bias_ptr(bias, x, N);
    Tensor out = at::empty({M, N}, x.options());
    if (M == 0) return out;
    const int dev = x.get_device();
    ok(cbk_packed_gemm(x.data_ptr(), dtype_of(x.scalar_type()), M, in_features, packed.data_ptr<int32_t>(),
                       scales.data_ptr(), zeros.data_ptr(), b, N, (int)bits, (int)group_size, (int)act,
                       use_tensor_cores ? 1 : 0, out.data_ptr(), dev, stream_of(dev)));
    return out;
}

Tensor fused_gate_up(const Tensor& x, const Tensor& wg, const Tensor& sg, const Tensor& zg, const Tensor& wu,
                     const Tensor& su, const Tensor& zu, int64_t bits, int64_t in_features, int64_t group_size,
                     int64_t split_k, int64_t rho, const OptT& workspace) {
    check_x(x, in_features);
    check_weight(x, wg, sg, zg, bits, in_features, group_size, "fused_gate_up(gate)");
    check_weight(x, wu, su, zu, bits, in_features, group_size, "fused_gate_up(up)");
    TORCH_CHECK(wg.sizes() == wu.sizes(), "gate/up packed shapes must match");
    TORCH_CHECK(split_k >= 1, "split_k must be >= 1");
    int32_t* ws = workspace_ptr(workspace, x);
    const int64_t N = wg.size(0), M = x.size(0);
    Tensor out = at::empty({M, N}, x.options());
    if (M == 0) return out;
    const Tensor part = partial_for(x, M, 2 * N, in_features, group_size, split_k);
    const int dev = x.get_device();
    ok(cbk_fused_gate_up(x.data_ptr(), dtype_of(x.scalar_type()), M, in_features, wg.data_ptr<int32_t>(),
                         sg.data_ptr(), zg.data_ptr(), wu.data_ptr<int32_t>(), su.data_ptr(), zu.data_ptr(), N,
                         (int)bits, (int)group_size, (int)split_k, (int)rho, ws, static_cast<float*>(tensor_ptr(part)),
                         out.data_ptr(), dev, stream_of(dev)));
    return out;
}

// Prefill gate-up: silu(x G^T) * (x U^T) with each factor rounded to x's dtype, in one
// launch where the 16-bit matrix-core GEMM takes the call, else two GEMMs and a product.
Tensor packed_gemm_gate_up(const Tensor& x, const Tensor& wg, const Tensor& sg, const Tensor& zg, const Tensor& wu,
                           const Tensor& su, const Tensor& zu, int64_t bits, int64_t in_features,
                           int64_t group_size) {
    check_x(x, in_features);
    check_weight(x, wg, sg, zg, bits, in_features, group_size, "packed_gemm_gate_up(gate)");
    check_weight(x, wu, su, zu, bits, in_features, group_size, "packed_gemm_gate_up(up)");
    TORCH_CHECK(wg.sizes() == wu.sizes(), "gate/up packed shapes must match");
    const int64_t N = wg.size(0), M = x.size(0);
    Tensor out = at::empty({M, N}, x.options());
    if (M == 0) return out;
    const int dev = x.get_device();
    const int rc = cbk_packed_gemm_gate_up(x.data_ptr(), dtype_of(x.scalar_type()), M, in_features,
                                           wg.data_ptr<int32_t>(), sg.data_ptr(), zg.data_ptr(),
                                           wu.data_ptr<int32_t>(), su.data_ptr(), zu.data_ptr(), N, (int)bits,
                                           (int)group_size, out.data_ptr(), dev, stream_of(dev));
    if (rc != CBK_ENOTSUP) {
        ok(rc);
        return out;
    }
    ok(cbk_packed_gemm(x.data_ptr(), dtype_of(x.scalar_type()), M, in_features, wg.data_ptr<int32_t>(),
                       sg.data_ptr(), zg.data_ptr(), nullptr, N, (int)bits, (int)group_size, CBK_ACT_SILU, 1,
                       out.data_ptr(), dev, stream_of(dev)));
    Tensor u = at::empty({M, N}, x.options());
    ok(cbk_packed_gemm(x.data_ptr(), dtype_of(x.scalar_type()), M, in_features, wu.data_ptr<int32_t>(),
                       su.data_ptr(), zu.data_ptr(), nullptr, N, (int)bits, (int)group_size, CBK_ACT_NONE, 1,
                       u.data_ptr(), dev, stream_of(dev)));
    out.mul_(u);
    return out;
}

// ``bits`` is one width (the reference's signature) or a (q, k, v) sequence of widths.
std::vector<Tensor> fused_qkv(const Tensor& x, const Tensor& wq, const Tensor& sq, const Tensor& zq, const OptT& bq,
                              const Tensor& wk, const Tensor& sk, const Tensor& zk, const OptT& bk, const Tensor& wv,
                              const Tensor& sv, const Tensor& zv, const OptT& bv, const OptT& rope_cos,
                              const OptT& rope_sin, int64_t head_dim, int64_t perm_hd, const py::object& bits,
                              int64_t in_features, int64_t group_size, int64_t split_k, int64_t rho,
                              const OptT& workspace) {
    int64_t b3[3];
    const bool mixed = !py::isinstance<py::int_>(bits);
    if (mixed) {
        const auto seq = bits.cast<std::vector<int64_t>>();
        TORCH_CHECK(seq.size() == 3, "bits must be one width or a (q, k, v) triple");
        for (int i = 0; i < 3; ++i) b3[i] = seq[i];
    } else {
        b3[0] = b3[1] = b3[2] = bits.cast<int64_t>();
    }
    check_x(x, in_features);
    check_weight(x, wq, sq, zq, b3[0], in_features, group_size, "fused_qkv(q)");
    check_weight(x, wk, sk, zk, b3[1], in_features, group_size, "fused_qkv(k)");
    check_weight(x, wv, sv, zv, b3[2], in_features, group_size, "fused_qkv(v)");
    TORCH_CHECK(split_k >= 1, "split_k must be >= 1");
    const int64_t B = x.size(0);
    if (perm_hd > 0) {
        TORCH_CHECK(perm_hd % 2 == 0, "perm head_dim must be even");
        TORCH_CHECK(wq.size(0) % perm_hd == 0 && wk.size(0) % perm_hd == 0, "Q/K widths must be multiples of head_dim");
    }
    const bool rope = rope_cos.has_value() && rope_cos->numel() > 0;
    Tensor rc, rs;
    if (rope) {
        TORCH_CHECK(perm_hd > 0 && perm_hd == head_dim,
                    "fused RoPE needs Q/K weights stored pair-interleaved with the same head_dim "
                    "(ops.permute_for_rope / install_bitmap(fuse_rope=True))");
        TORCH_CHECK(rope_sin.has_value() && rope_cos->sizes() == rope_sin->sizes(), "cos/sin shape mismatch");
        TORCH_CHECK(rope_cos->numel() == B * head_dim, "cos/sin must be [B, head_dim] (one row per x row)");
        rc = rope_cos->to(x.device(), at::kFloat).contiguous();
        rs = rope_sin->to(x.device(), at::kFloat).contiguous();
    }
    const int64_t nq = wq.size(0), nk = wk.size(0), nv = wv.size(0);
    const void* pq = bias_ptr(bq, x, nq);
    const void* pk = bias_ptr(bk, x, nk);
    const void* pv = bias_ptr(bv, x, nv);
    int32_t* ws = workspace_ptr(workspace, x);
    // one allocation carved into three contiguous [B, n] outputs (each its own block of it)
    const Tensor flat = at::empty({B * (nq + nk + nv)}, x.options());
    std::vector<Tensor> outs = {flat.narrow(0, 0, B * nq).view({B, nq}), flat.narrow(0, B * nq, B * nk).view({B, nk}),
                                flat.narrow(0, B * (nq + nk), B * nv).view({B, nv})};
    if (B == 0) return outs;
    const Tensor part = partial_for(x, B, nq + nk + nv, in_features, group_size, split_k);
    const int dev = x.get_device();
    const float* c = rope ? rc.data_ptr<float>() : nullptr;
    const float* s = rope ? rs.data_ptr<float>() : nullptr;
    const int hd = rope ? (int)head_dim : 0;
    float* p = static_cast<float*>(tensor_ptr(part));
    if (b3[0] == b3[1] && b3[1] == b3[2]) {
        ok(cbk_fused_qkv(x.data_ptr(), dtype_of(x.scalar_type()), B, in_features, wq.data_ptr<int32_t>(),
                         sq.data_ptr(), zq.data_ptr(), pq, nq, wk.data_ptr<int32_t>(), sk.data_ptr(), zk.data_ptr(),
                         pk, nk, wv.data_ptr<int32_t>(), sv.data_ptr(), zv.data_ptr(), pv, nv, c, s, hd,
                         (int)perm_hd, (int)b3[0], (int)group_size, (int)split_k, (int)rho, ws, p,
                         outs[0].data_ptr(), outs[1].data_ptr(), outs[2].data_ptr(), dev, stream_of(dev)));
    } else {
        ok(cbk_fused_qkv_mixed(x.data_ptr(), dtype_of(x.scalar_type()), B, in_features, wq.data_ptr<int32_t>(),
                               sq.data_ptr(), zq.data_ptr(), pq, nq, wk.data_ptr<int32_t>(), sk.data_ptr(),
                               zk.data_ptr(), pk, nk, wv.data_ptr<int32_t>(), sv.data_ptr(), zv.data_ptr(), pv, nv,
                               c, s, hd, (int)perm_hd, (int)b3[0], (int)b3[1], (int)b3[2], (int)group_size,
                               (int)split_k, (int)rho, ws, p, outs[0].data_ptr(), outs[1].data_ptr(),
                               outs[2].data_ptr(), dev, stream_of(dev)));
    }
    return outs;
}

int current_device() { return c10::hip::current_device(); }

int64_t sm_count() {
    int v = 0;
    ok(cbk_sm_count(current_device(), &v));
    return v;
}

int64_t tile_n() { return cbk_tile_n(); }

int kind_code(const std::string& kind) {
    if (kind == "gemv") return CBK_MODE_GEMV;
    if (kind == "qkv") return CBK_MODE_QKV;
    if (kind == "gate_up") return CBK_MODE_GATEUP;
    TORCH_CHECK(false, "kind must be 'gemv', 'qkv' or 'gate_up'");
}

int64_t max_rho(int64_t bits, const std::string& kind) {
    int v = 0;
    ok(cbk_max_rho(current_device(), (int)bits, kind_code(kind), &v));
    return v;
}

// ------------------------------------------------------------------------------ additive entries

Tensor unpack_codes(const Tensor& packed, int64_t bits, int64_t in_features) {
    TORCH_CHECK(packed.is_cuda() && packed.scalar_type() == at::kInt && packed.is_contiguous() && packed.dim() == 2,
                "packed must be a contiguous 2-D CUDA int32 tensor");
    TORCH_CHECK(packed.size(1) == cdiv(in_features, 32) * bits, "packed row must hold exactly ceil(K/32)*bits words");
    Tensor out = at::empty({packed.size(0), in_features}, packed.options());
    const int dev = packed.get_device();
    ok(cbk_unpack_codes(packed.data_ptr<int32_t>(), packed.size(0), in_features, (int)bits, out.data_ptr<int32_t>(),
                        dev, stream_of(dev)));
    return out;
}

// (packed int32 [N, ceil(K/32)*bits], scales, zeros [N, ceil(K/g)] in ``dtype``) of a CUDA weight
// [N, K]: scheme 0 reference.py:10-55, scheme 1 crispybits_quant/affine.py:28-71, bit for bit.
std::tuple<Tensor, Tensor, Tensor> quantize_pack(const Tensor& weight, int64_t bits, int64_t group_size,
                                                 py::object dtype, int64_t scheme) {
    TORCH_CHECK(weight.is_cuda() && weight.dim() == 2, "weight must be a 2-D CUDA tensor");
    TORCH_CHECK(dtype_of(weight.scalar_type()) >= 0, "weight must be fp16/bf16/fp32");
    const at::ScalarType mdt = dtype.is_none() ? at::kHalf : torch::python::detail::py_object_to_dtype(dtype);
    TORCH_CHECK(dtype_of(mdt) >= 0, "scales/zeros dtype must be fp16/bf16/fp32");
    const Tensor w = weight.contiguous();
    const int64_t N = w.size(0), K = w.size(1);
    const int64_t G = group_size > 0 ? cdiv(K, group_size) : 0;
    Tensor packed = at::empty({N, cdiv(K, 32) * bits}, w.options().dtype(at::kInt));
    Tensor scales = at::empty({N, G}, w.options().dtype(mdt));
    Tensor zeros = at::empty({N, G}, w.options().dtype(mdt));
    const int dev = w.get_device();
    ok(cbk_quantize_pack(w.data_ptr(), dtype_of(w.scalar_type()), N, K, (int)bits, (int)group_size, (int)scheme,
                         packed.data_ptr<int32_t>(), scales.data_ptr(), zeros.data_ptr(), dtype_of(mdt), dev,
                         stream_of(dev)));
    return {packed, scales, zeros};
}

// The launch a decode call would make: (kernel family, K splits, workgroups, threads, LDS bytes,
// launches per call).  out_features / bits: one value, or (q, k, v) for kind "qkv".
py::tuple decode_plan(py::object dtype, int64_t batch, int64_t in_features, int64_t group_size,
                      const py::object& out_features, const py::object& bits, const std::string& kind,
                      int64_t split_k, int64_t rho) {
    auto triple = [](const py::object& o) {
        std::vector<int64_t> v;
        if (py::isinstance<py::int_>(o)) v.assign(3, o.cast<int64_t>());
        else v = o.cast<std::vector<int64_t>>();
        TORCH_CHECK(v.size() == 3, "expected one value or a (q, k, v) triple");
        return v;
    };
    const auto ns = triple(out_features), bs = triple(bits);
    const int dt = dtype_of(torch::python::detail::py_object_to_dtype(dtype));
    TORCH_CHECK(dt >= 0, "dtype must be fp16/bf16/fp32");
    int32_t out[6] = {0, 0, 0, 0, 0, 0};
    ok(cbk_decode_plan(dt, batch, in_features, (int)group_size, ns[0], ns[1], ns[2], (int)bs[0], (int)bs[1],
                       (int)bs[2], kind_code(kind), (int)split_k, (int)rho, current_device(), out));
    static const char* families[] = {"?", "stream", "bstream", "mfma", "generic", "batch"};
    const char* fam = out[0] >= 1 && out[0] <= 5 ? families[out[0]] : "?";
    return py::make_tuple(fam, out[1], out[2], out[3], out[4], out[5]);
}

void timer_start(int64_t capacity) { ok(cbk_timer_start((int)capacity)); }

// (total ms, per-launch durations in ms) of the launches since timer_start.
py::tuple timer_stop() {
    const int cap = 1 << 16;
    std::vector<double> d(cap);
    double total = 0.0;
    int n = 0;
    ok(cbk_timer_stop(&total, &n, d.data(), cap));
    d.resize(std::min(n, cap));
    return py::make_tuple(total, py::cast(d));
}

// One streaming launch over the bytes of a CUDA tensor (the measurement floor of
// cbk_stream_probe); `sink` is a CUDA int32 tensor of at least 1024 elements on the same device.
void stream_probe(const Tensor& src, int64_t unroll, int64_t block, bool store, Tensor& sink) {
    TORCH_CHECK(src.is_cuda() && src.is_contiguous(), "src must be a contiguous CUDA tensor");
    TORCH_CHECK(sink.is_cuda() && sink.device() == src.device() && sink.scalar_type() == at::kInt &&
                sink.is_contiguous() && sink.numel() >= 1024, "sink must be 1024 CUDA int32 on src's device");
    const int dev = src.get_device();
    ok(cbk_stream_probe(src.data_ptr(), src.numel() * src.element_size(), (int)unroll, (int)block, store ? 1 : 0,
                        reinterpret_cast<uint32_t*>(sink.data_ptr<int32_t>()), dev, stream_of(dev)));
}

}  // namespace

PYBIND11_MODULE(_ext, m) {
    m.doc() = "crispybits_kernels op bindings over libcrispybits_hip.so (gfx950)";
    m.def("packed_gemv", &packed_gemv, "Packed W2/W3/W4 decode GEMV (streaming, split-K by plan)");
    m.def("packed_gemm", &packed_gemm, "Packed W2/W3/W4 prefill GEMM (MFMA fp16/bf16, VALU fp32)");
    m.def("fused_gate_up", &fused_gate_up, "Fused gate/up decode GEMV with SiLU gating");
    m.def("packed_gemm_gate_up", &packed_gemm_gate_up,
          "Prefill gate-up: silu(x G^T) * (x U^T), one MFMA launch for fp16/bf16 x");
    m.def("fused_qkv", &fused_qkv, "Fused Q/K/V decode GEMV (GQA widths, biases, optional in-kernel RoPE)");
    m.def("sm_count", &sm_count, "Compute units of the current device");
    m.def("tile_n", &tile_n, "Virtual output rows per decode job tile (B_N of the underfill rule)");
    m.def("max_rho", &max_rho, "Occupancy-limited resident workgroups per CU", py::arg("bits"),
          py::arg("kind") = "gemv");
    m.def("unpack_codes", &unpack_codes, "int32 codes [N, K] of a packed matrix, decoded on the device");
    m.def("quantize_pack", &quantize_pack, "Group-affine quantizer + packer on the device", py::arg("weight"),
          py::arg("bits"), py::arg("group_size") = 128, py::arg("dtype") = py::none(), py::arg("scheme") = 0);
    m.def("decode_plan", &decode_plan, "The launch a decode call would make");
    m.def("timer_start", &timer_start, "Arm the per-launch kernel timer", py::arg("capacity") = 4096);
    m.def("timer_stop", &timer_stop, "Disarm the timer: (total ms, per-launch ms)");
    m.def("stream_probe", &stream_probe, "One streaming launch over a tensor's bytes (the measurement floor)",
          py::arg("src"), py::arg("unroll"), py::arg("block"), py::arg("store"), py::arg("sink"));
    m.attr("ABI_VERSION") = cbk_abi_version();
}
