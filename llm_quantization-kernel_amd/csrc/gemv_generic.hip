// gemv_generic.hip -- VALU decode GEMV for every dtype / group size, and the
// split-K combine.
//
// The MFMA kernel (gemv_mfma.hip) covers fp16 activations with group sizes that
// are multiples of 128; this kernel covers the rest of the reference's contract
// (bf16 / fp32 activations, group sizes 32 and 64, Kernel/tests/test_correctness.py:
// 56-69) with fp32 arithmetic throughout, as cb_gemv_kernel does
// (Kernel/csrc/packed_gemv.cu:113-138): per chunk d = sum_j x_j q_j in j order,
// acc += s * (d - z * sum_j x_j).
//
// Job = (K split p, tile of 32 virtual rows, batch row b); a workgroup of 4 waves
// takes 8 rows per wave, lane = chunk (lane, lane + 64, ...), and the per-row sums
// are reduced across the wave with xor shuffles.
#include "cbk_device.hpp"
#include "cbk_kernels.hpp"

namespace cbk {
namespace {

constexpr int RPW = 8;                       // rows per wave
constexpr int WAVES = GENERIC_THREADS / 64;

template <int BITS>
__device__ __forceinline__ float chunk_contrib(const uint32_t* wrow, int c, const float (&xv)[32], float xsum,
                                               float s, float z) {
    uint32_t w[BITS];
#pragma unroll
    for (int i = 0; i < BITS; ++i) w[i] = wrow[(long)c * BITS + i];
    float d = 0.f;
#pragma unroll
    for (int j = 0; j < 32; ++j) d = fmaf(xv[j], (float)chunk_code<BITS>(w, j), d);
    return s * (d - z * xsum);
}

template <int DT, int MODE>
__global__ void __launch_bounds__(GENERIC_THREADS) gemv_generic_kernel(const GemvArgs A) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int job = blockIdx.x; job < A.jobs; job += gridDim.x) {
        const int p = job % A.P;
        const int rest = job / A.P;
        const int tile = rest % A.ntiles;
        const int b = rest / A.ntiles;
        const int c0 = (int)(((long)A.C * p) / A.P);
        const int c1 = (int)(((long)A.C * (p + 1)) / A.P);
        const int v0 = tile * GENERIC_ROWS + wave * RPW;

        float acc[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) acc[r] = 0.f;

        for (int c = c0 + lane; c < c1; c += 64) {
            float xv[32];
            float xsum = 0.f;
#pragma unroll
            for (int j = 0; j < 32; ++j) {
                const int k = c * 32 + j;
                xv[j] = k < A.K ? load_f<DT>(A.x, (long)b * A.K + k) : 0.f;
                xsum += xv[j];
            }
            const int g = (c * 32) / A.gs;
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                const int v = v0 + r;
                if (v < A.V) {
                    int proj, row;
                    vmap<MODE>(A, v, proj, row);
                    const uint32_t* wrow = CBK_SEL(A, proj, w) + (long)row * CBK_SEL(A, proj, wpr);
                    const float s = load_f<DT>(CBK_SEL(A, proj, s), (long)row * A.G + g);
                    const float z = load_f<DT>(CBK_SEL(A, proj, z), (long)row * A.G + g);
                    const int bits = CBK_SEL(A, proj, bits);
                    if (bits == 2) acc[r] += chunk_contrib<2>(wrow, c, xv, xsum, s, z);
                    else if (bits == 3) acc[r] += chunk_contrib<3>(wrow, c, xv, xsum, s, z);
                    else acc[r] += chunk_contrib<4>(wrow, c, xv, xsum, s, z);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) acc[r] += __shfl_xor(acc[r], off, 64);
        }
        float mine = 0.f, partner = 0.f;
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            if (r == lane) mine = acc[r];
            if ((r ^ 1) == lane) partner = acc[r];
        }
        const int v = v0 + lane;
        if (lane < RPW && v < A.V) {
            if (A.P == 1) epilogue<DT, MODE>(A, b, v, mine, partner);
            else A.partial[((long)p * A.M + b) * A.V + v] = mine;
        }
    }
}

// Sums partial[s, b, v] over s in ascending order (and the partner row v ^ 1 of the
// paired modes), then runs the epilogue (packed_gemv.cu:166-180 semantics).
template <int DT, int MODE>
__global__ void __launch_bounds__(256) gemv_reduce_kernel(const GemvArgs A) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long total = (long)A.M * A.V;
    if (i >= total) return;
    const int b = (int)(i / A.V), v = (int)(i - (long)b * A.V);
    const bool paired = (MODE == MODE_GATEUP) || (MODE == MODE_QKV && A.rope_cos != nullptr);
    float mine = 0.f, partner = 0.f;
    for (int s = 0; s < A.P; ++s) {
        const float* ps = A.partial + ((long)s * A.M + b) * A.V;
        mine += ps[v];
        if (paired && (v ^ 1) < A.V) partner += ps[v ^ 1];
    }
    epilogue<DT, MODE>(A, b, v, mine, partner);
}

template <int DT>
const void* generic_for_mode(int mode) {
    if (mode == MODE_QKV) return reinterpret_cast<const void*>(&gemv_generic_kernel<DT, MODE_QKV>);
    if (mode == MODE_GATEUP) return reinterpret_cast<const void*>(&gemv_generic_kernel<DT, MODE_GATEUP>);
    return reinterpret_cast<const void*>(&gemv_generic_kernel<DT, MODE_GEMV>);
}

template <int DT>
const void* reduce_for_mode(int mode) {
    if (mode == MODE_QKV) return reinterpret_cast<const void*>(&gemv_reduce_kernel<DT, MODE_QKV>);
    if (mode == MODE_GATEUP) return reinterpret_cast<const void*>(&gemv_reduce_kernel<DT, MODE_GATEUP>);
    return reinterpret_cast<const void*>(&gemv_reduce_kernel<DT, MODE_GEMV>);
}

}  // namespace

const void* gemv_generic_kernel_for(int dt, int mode) {
    if (dt == DT_F16) return generic_for_mode<DT_F16>(mode);
    if (dt == DT_BF16) return generic_for_mode<DT_BF16>(mode);
    return generic_for_mode<DT_F32>(mode);
}

hipError_t launch_gemv_generic(const GemvArgs& A, int dt, int mode, int grid, hipStream_t stream) {
    void* args[] = {const_cast<GemvArgs*>(&A)};
    return launch(gemv_generic_kernel_for(dt, mode), dim3(grid), dim3(GENERIC_THREADS), args, 0, stream);
}

hipError_t launch_gemv_reduce(const GemvArgs& A, int dt, int mode, hipStream_t stream) {
    const long total = (long)A.M * A.V;
    const void* f = dt == DT_F16 ? reduce_for_mode<DT_F16>(mode)
                  : dt == DT_BF16 ? reduce_for_mode<DT_BF16>(mode) : reduce_for_mode<DT_F32>(mode);
    void* args[] = {const_cast<GemvArgs*>(&A)};
    return launch(f, dim3((unsigned)((total + 255) / 256)), dim3(256), args, 0, stream);
}

}  // namespace cbk
