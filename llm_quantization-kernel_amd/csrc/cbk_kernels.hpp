// cbk_kernels.hpp -- launchers exported by the kernel translation units to abi.cpp.
#pragma once

#include <hip/hip_runtime.h>
#include "cbk_device.hpp"

namespace cbk {

// abi.cpp: every kernel launch goes through here.  While the measurement timer is
// armed (cbk_timer_start) the launch records start/stop events inside the dispatch
// (hipExtLaunchKernel), so cbk_timer_stop reports pure kernel durations.
hipError_t launch(const void* f, dim3 grid, dim3 block, void** args, size_t lds, hipStream_t stream);

// abi.cpp: raises kernel f's dynamic-LDS limit (on the current device) to cover `bytes`,
// once per kernel and device; the limit is only ever raised.
hipError_t lds_limit_raise(const void* f, int bytes);

// gemv_stream.hip: batch 1 or 2 (mb staged activation rows), fp16 or bf16, group size % 32 == 0.  A job is rpw * st_rw
// virtual rows x one K split; its workgroup has st_ks * st_rw waves, each over rpw rows
// (STREAM_RPW, or STREAM_RPW_WIDE at batch 1) and one K slice of 64 * STREAM_CPL chunks.
#ifndef CBK_STREAM_CPL
#define CBK_STREAM_CPL 1
#endif
constexpr int STREAM_CPL = CBK_STREAM_CPL;
constexpr int STREAM_RPW = 4;
constexpr int STREAM_RPW_WIDE = 8;
const void* gemv_stream_kernel_for(int mode, int bits, bool mixed, int mb, int rpw, int dt);
// gemv_stream.hip: batch 3..16, fp16 or bf16, group size % 128 == 0.  A job is 16 * st_rw virtual
// rows x one K split (over 128-code units); its workgroup has st_ks * st_rw waves, each
// over 16 rows and one K slice of bsu (4 or 8) units.
const void* gemv_bstream_kernel_for(int mode, int bits, bool mixed, int bsu, int dt);

// gemv_any.hip: any dtype / group size / alignment, on the fp32 matrix cores.  A job is
// 16 virtual rows x 16 batch rows x one K split, one workgroup of 64 to ANY_MAX_THREADS
// threads (whole waves) that share the split's chunks.
constexpr int ANY_MAX_THREADS = 1024;
const void* gemv_any_kernel_for(int dt, int mode);

// gemv_any.hip: the combine launch of split-K partials (P > 1 without arrival counters).
hipError_t launch_gemv_combine(const GemvArgs& A, int dt, int mode, hipStream_t stream);

struct GemmArgs {
    const void* x;          // [M, K]
    const uint32_t* w;      // packed [N, wpr]
    const void* s;          // scales [N, G]
    const void* z;          // zeros [N, G]
    const void* b;          // bias [N] or nullptr
    void* out;              // [M, N]
    int M, N, K, C, G, gs, wpr, bits, act;
    int xvec;               // x is 16-byte aligned and K % 8 == 0 (vector activation loads)
    FastDiv divG;           // by the group size
    const uint32_t* w2;     // gate-up GEMM: the up projection's packed [N, wpr], scales, zeros
    const void* s2;
    const void* z2;
};

// gemm.hip: fp16 / bf16 on the 16-bit matrix cores, any alignment.
hipError_t launch_gemm_mfma(const GemmArgs& A, int dt, hipStream_t stream);

// gemm_f32.hip: any dtype, fp32 operands on the fp32 matrix cores, W-hat unrounded.
hipError_t launch_gemm_f32(const GemmArgs& A, int dt, hipStream_t stream);

// gemm_f16.hip: fp16 or bf16 (dt), K % 8 == 0, 16-byte aligned x.  gate_up: out =
// silu(x . W-hat^T) * (x . W2-hat^T), each factor rounded to the dtype first (no bias).
bool gemm_f16_supported(const GemmArgs& A);
hipError_t launch_gemm_f16(const GemmArgs& A, int dt, hipStream_t stream, bool gate_up = false);

// quant.hip: group-affine quantizer + bit packer (the format's producer).
struct QuantArgs {
    const void* w;          // [N, K] weights (fp16 / bf16 / fp32)
    uint32_t* packed;       // [N, wpr]
    void* scales;           // [N, G] in the metadata dtype
    void* zeros;            // [N, G]
    int N, K, G, gs, bits, wpr;
    int scheme;             // 0: reference.py quantize_affine, 1: crispybits_quant affine
};
hipError_t launch_quant_pack(const QuantArgs& A, int dt, int mdt, int cus, hipStream_t stream);

// unpack.hip
hipError_t launch_unpack(const uint32_t* packed, int N, int K, int bits, int32_t* codes, hipStream_t stream);

// probe.hip: one read-only streaming launch over `bytes` (the measurement floor).
hipError_t launch_stream_probe(const void* src, uint32_t bytes, int unroll, int block, bool store, uint32_t* sink,
                               hipStream_t stream);

}  // namespace cbk
