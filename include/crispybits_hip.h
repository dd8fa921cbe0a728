/*
 * crispybits_hip.h -- C ABI of the MI355X (gfx950) packed W2/W3/W4 linear kernels.
 *
 * This is the drop-in boundary that replaces the reference's pybind11 module
 * `crispybits_kernels._C` (/root/reference/Crispybits/Kernel/csrc/bindings.cpp:32-40).
 * Every entry point takes plain device pointers, sizes and a hipStream_t (as void*),
 * launches asynchronously on that stream and returns a status code; no torch types
 * cross this boundary.  The Python host layer (crispybits_kernels/_C.py, a PyTorch-ROCm
 * C++ extension over this header, csrc/torch_ext.cpp) binds it and keeps the reference's
 * argument order and error behaviour.
 *
 * Conventions shared by all entry points
 *   - dtype: CBK_F16 / CBK_BF16 / CBK_F32 is the type of x, scales, zeros, bias and
 *     out (host_utils.h:60,84 require them to match).
 *   - packed: int32 [N, ceil(K/32)*bits] row-major, LSB-first bitstream, rows padded
 *     to 32-code chunks; base alignment 16/4/8 bytes for W4/W3/W2 (host_utils.h:63-68).
 *   - scales / zeros: [N, ceil(K/group_size)] row-major; zeros hold exact integers.
 *   - bias: [N] or NULL ("no bias" is an empty tensor in the reference, host_utils.h:80-81).
 *   - act: CBK_ACT_NONE / CBK_ACT_RELU / CBK_ACT_SILU (ops.py:24, common.cuh:10).
 *   - rho: the reference's persistence factor (host_utils.h:90-93).  Every decode kernel
 *     here runs one workgroup per job (the jobs are assigned statically and its
 *     workgroups gain nothing from persistence), so rho is accepted and never changes the
 *     launch or the results.
 *   - workspace: the caller's int32[2] job-queue word pair (host_utils.h:38-47).  Jobs are
 *     distributed statically here, so the workspace is accepted, never written, and its
 *     [0,0] contract holds trivially.  May be NULL.
 *   - partial: fp32 scratch of cbk_gemv_partial_floats(...) elements, required only when
 *     that query returns a positive count (split-K partial sums, packed_gemv.cu:193-199).
 *     The decode kernels combine the splits inside their own dispatch, using arrival
 *     counters the library keeps per device in windows (256 windows of 4096 counters); a
 *     window belongs for good to one stream (its eager calls) or one graph capture, and is
 *     never shared.  A call that finds no window of its own and no free one, or whose row
 *     blocks outnumber a window's counters, combines in a second launch instead (the same
 *     bits).  A graph must not be replayed while another replay of it still runs.
 *   - device: HIP device ordinal the pointers live on (the reference's CUDAGuard,
 *     packed_gemv.cu:259); the calling thread's current device is restored on return.
 *   - return: CBK_OK, or an error code with a message from cbk_last_error().
 */
#ifndef CRISPYBITS_HIP_H
#define CRISPYBITS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { CBK_F16 = 0, CBK_BF16 = 1, CBK_F32 = 2 };
enum { CBK_ACT_NONE = 0, CBK_ACT_RELU = 1, CBK_ACT_SILU = 2 };
enum { CBK_MODE_GEMV = 0, CBK_MODE_QKV = 1, CBK_MODE_GATEUP = 2 };
enum { CBK_OK = 0, CBK_EINVAL = 1, CBK_EHIP = 2, CBK_ENOTSUP = 3 };

/* Message of the last failing call on this thread ("" if none). */
const char* cbk_last_error(void);

/* ABI revision; bumped when a signature changes. */
int cbk_abi_version(void);

/* Compute units of `device` (replaces crispybits_sm_count, packed_gemv.cu:339). */
int cbk_sm_count(int device, int* out);

/* Virtual output rows per decode job tile -- the B_N of the split-K policy
 * (replaces crispybits_tile_n, packed_gemv.cu:340). */
int cbk_tile_n(void);

/* Occupancy-limited resident workgroups per CU of the kernel an fp16 batch-1 decode call of
 * `mode` runs at the Llama-2-7B widths (K = 4096), at that call's workgroup size and LDS
 * (replaces crispybits_max_rho_mode, packed_gemv.cu:343-347). */
int cbk_max_rho(int device, int bits, int mode, int* out);

/* Decode kernel families reported by cbk_decode_plan: the streaming kernel at batch 1-2
 * (fp16 / bf16), the batched streaming kernel at batch 3-16 (fp16 / bf16, group sizes that
 * are multiples of 128), and the fp32 matrix-core kernel for every other call (fp32
 * activations, unaligned x, other group sizes at batch 3-16, batch > 16).  Values 3 and 5
 * named kernels this library no longer has and are not returned. */
enum { CBK_KERNEL_STREAM = 1, CBK_KERNEL_BSTREAM = 2, CBK_KERNEL_MFMA = 3, CBK_KERNEL_GENERIC = 4, CBK_KERNEL_BATCH = 5 };

/* Additive policy query (no counterpart in the reference, whose tuner infers launches from
 * (split_k, rho), autotune.py:55-88): the launch a decode call with these arguments makes,
 * without launching it.  out[6] = {kernel family, K splits, workgroups, threads per workgroup,
 * dynamic LDS bytes, launches per call}.  n1/n2 and bits1/bits2 are read for CBK_MODE_QKV
 * only; tensors are assumed allocated as torch allocates them (aligned bases). */
int cbk_decode_plan(int dtype, int64_t M, int64_t K, int group_size, int64_t n0, int64_t n1, int64_t n2,
                    int bits0, int bits1, int bits2, int mode, int split_k, int rho, int device, int32_t* out);

/* fp32 elements of `partial` that a decode call with these arguments needs
 * (0 = none).  `V` is the number of virtual rows (N, nq+nk+nv or 2N). */
int64_t cbk_gemv_partial_floats(int dtype, int64_t M, int64_t V, int64_t K, int group_size,
                                int split_k);

/* out[M,N] = act(x[M,K] . W-hat^T + bias) on the decode path
 * (replaces packed_gemv_cuda, packed_gemv.cu:252-269; bindings.cpp:4-6). */
int cbk_packed_gemv(const void* x, int dtype, int64_t M, int64_t K,
                    const int32_t* packed, const void* scales, const void* zeros, const void* bias,
                    int64_t N, int bits, int group_size, int split_k, int rho, int act,
                    int32_t* workspace, float* partial, void* out, int device, void* stream);

/* Allocation-free variant of cbk_packed_gemv.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The split-K partial sums live in a file-scope
 * device array of CBK_NOALLOC_PARTIAL_FLOATS fp32 values per GPU (8 MiB, held until the
 * process ends) instead of a caller buffer; calls whose cbk_gemv_partial_floats(...)
 * exceeds that return CBK_EINVAL.  The call allocates nothing (no hipMalloc, no library
 * allocation); every partial it reads it has written in the same call, so nothing needs
 * clearing between calls.  Calls that overlap on one GPU (concurrent streams, threads)
 * share the array and race. */
#define CBK_NOALLOC_PARTIAL_FLOATS (1 << 21)
int cbk_packed_gemv_noalloc(const void* x, int dtype, int64_t M, int64_t K,
                            const int32_t* packed, const void* scales, const void* zeros, const void* bias,
                            int64_t N, int bits, int group_size, int split_k, int rho, int act,
                            void* out, int device, void* stream);

/* out[M,N] = silu(x . G-hat^T) * (x . U-hat^T) with gate and up read in one pass
 * (replaces fused_gate_up_cuda, packed_gemv.cu:317-337; bindings.cpp:10-13). */
int cbk_fused_gate_up(const void* x, int dtype, int64_t M, int64_t K,
                      const int32_t* wg, const void* sg, const void* zg,
                      const int32_t* wu, const void* su, const void* zu,
                      int64_t N, int bits, int group_size, int split_k, int rho,
                      int32_t* workspace, float* partial, void* out, int device, void* stream);

/* Fused Q/K/V decode with per-projection bias and optional in-kernel RoPE on
 * pair-interleaved Q/K rows (replaces fused_qkv_cuda, packed_gemv.cu:271-315;
 * bindings.cpp:14-20).  rope_cos / rope_sin: fp32 [M, head_dim] or NULL.
 * perm_hd: head_dim the Q/K rows are stored permuted with (0 = not permuted). */
int cbk_fused_qkv(const void* x, int dtype, int64_t M, int64_t K,
                  const int32_t* wq, const void* sq, const void* zq, const void* bq, int64_t nq,
                  const int32_t* wk, const void* sk, const void* zk, const void* bk, int64_t nk,
                  const int32_t* wv, const void* sv, const void* zv, const void* bv, int64_t nv,
                  const float* rope_cos, const float* rope_sin, int head_dim, int perm_hd,
                  int bits, int group_size, int split_k, int rho,
                  int32_t* workspace, float* partial, void* out_q, void* out_k, void* out_v,
                  int device, void* stream);

/* Additive: fused Q/K/V with one bit-width per projection.  No counterpart in the
 * reference (its fused_qkv takes one `bits`, ops.py:240-241); used when a block's
 * projections were quantized to different widths. */
int cbk_fused_qkv_mixed(const void* x, int dtype, int64_t M, int64_t K,
                        const int32_t* wq, const void* sq, const void* zq, const void* bq, int64_t nq,
                        const int32_t* wk, const void* sk, const void* zk, const void* bk, int64_t nk,
                        const int32_t* wv, const void* sv, const void* zv, const void* bv, int64_t nv,
                        const float* rope_cos, const float* rope_sin, int head_dim, int perm_hd,
                        int bits_q, int bits_k, int bits_v, int group_size, int split_k, int rho,
                        int32_t* workspace, float* partial, void* out_q, void* out_k, void* out_v,
                        int device, void* stream);

/* Prefill: out[M,N] = act(x . W-hat^T + bias).  With use_matrix_cores and fp16/bf16 x,
 * W-hat = RN_T((q - z) * s) runs on the 16-bit matrix cores; otherwise (fp32 x, or
 * use_matrix_cores = 0) W-hat is kept unrounded in fp32 and the products run on the fp32
 * matrix cores with fp32 accumulation (replaces packed_gemm_cuda, packed_gemm.cu:182-203;
 * bindings.cpp:7-9). */
int cbk_packed_gemm(const void* x, int dtype, int64_t M, int64_t K,
                    const int32_t* packed, const void* scales, const void* zeros, const void* bias,
                    int64_t N, int bits, int group_size, int act, int use_matrix_cores,
                    void* out, int device, void* stream);

/* Prefill gate-up: out[M,N] = RN_T(RN_T(silu(x . G-hat^T)) * RN_T(x . U-hat^T)) in one launch,
 * bit-identical to two cbk_packed_gemm calls (the gate's with act = 2) followed by an
 * elementwise product in T.  No counterpart in the reference's _C: it replaces the
 * two-GEMM-and-multiply sequence of the reference's ops.fused_gate_up for batches above the
 * decode threshold (Kernel/crispybits_kernels/ops.py:216-220).  fp16 / bf16 x only, with
 * K % 8 == 0 and 16-byte aligned x, packed, scales and zeros; other calls return
 * CBK_ENOTSUP (nothing launched) and take the two-GEMM sequence. */
int cbk_packed_gemm_gate_up(const void* x, int dtype, int64_t M, int64_t K,
                            const int32_t* packed_gate, const void* scales_gate, const void* zeros_gate,
                            const int32_t* packed_up, const void* scales_up, const void* zeros_up,
                            int64_t N, int bits, int group_size, void* out, int device, void* stream);

/* Format producer on the device: group-affine quantization of w[N,K] (fp16 / bf16 /
 * fp32) to `bits`-bit codes, packed as the kernels read them, with fp16 / bf16 / fp32
 * scales and zeros [N, ceil(K/group_size)].  scheme 0 is bit-identical to the reference's
 * quantize_affine + pack_codes (Kernel/crispybits_kernels/reference.py:10-27, 37-55;
 * pack_linear_dict :70-82), scheme 1 to the paper quantizer
 * quantization/crispybits_quant/affine.py:28-71 (codes in the same chunked layout).  Both
 * run on the host CPU in the reference; no counterpart in its _C. */
int cbk_quantize_pack(const void* w, int dtype, int64_t N, int64_t K, int bits, int group_size, int scheme,
                      int32_t* packed, void* scales, void* zeros, int meta_dtype, int device, void* stream);

/* Additive test hook: codes[N,K] (int32) of a packed matrix, for the bit-exact
 * code check.  No counterpart in the reference's _C (reference.py:58-67 is its
 * CPU equivalent). */
int cbk_unpack_codes(const int32_t* packed, int64_t N, int64_t K, int bits, int32_t* codes,
                     int device, void* stream);

/* Additive measurement hook (no counterpart in the reference, which times with CUDA
 * events around whole calls, autotune.py:37-52).  cbk_timer_start arms a per-process
 * timer for up to `capacity` kernel launches: each launch made by this library
 * records start/stop events inside its own dispatch (hipExtLaunchKernel), so the
 * measured durations are kernel execution only.  cbk_timer_stop waits for those
 * launches, writes their summed milliseconds, their count, and optionally each
 * launch's duration, and disarms the timer.  Not for use under graph capture. */
int cbk_timer_start(int capacity);
int cbk_timer_stop(double* total_ms, int* launches, double* durations_ms, int max_durations);

/* Additive measurement hook (no counterpart in the reference): one launch that reads
 * `bytes` (at most 2^30) of device memory at `src` once, as 16-byte pieces -- the floor a
 * single launch needs to stream a decode call's bytes.  `unroll` (1, 2, 4, 8 or 16) is the
 * pieces each thread requests before it uses any, `block` the workgroup size (a multiple of
 * 64, at most 1024); the grid covers `bytes`.  store = 0: nothing is kept (sink[0] is
 * practically never written; the write keeps the loads alive); store = 1: each workgroup
 * reduces what it read and writes one word to sink[workgroup % 1024], as a decode
 * workgroup writes its results.  `sink` holds 1024 writable uint32. */
int cbk_stream_probe(const void* src, int64_t bytes, int unroll, int block, int store, uint32_t* sink,
                     int device, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CRISPYBITS_HIP_H */
