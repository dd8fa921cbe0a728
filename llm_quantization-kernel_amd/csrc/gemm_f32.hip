// gemm_f32.hip -- prefill packed GEMM with fp32 arithmetic: out[M,N] = act(x W-hat^T + bias),
// W-hat = (q - z) s kept in fp32 (never rounded to the activation dtype).
//
// The path for fp32 activations, and for fp16 / bf16 ones when the caller turns the
// 16-bit matrix cores off (use_tensor_cores=False): the reference's fp32 GEMM contract
// (Kernel/csrc/packed_gemm.cu:119-156, dispatched at :165-178), run on gfx950's fp32
// matrix cores (v_mfma_f32_16x16x4_f32: fp32 operands, fp32 accumulation).
//
// A workgroup of four waves owns a 64 x 64 output tile, wave (wm, wn) a 32 x 32 quarter
// as 2 x 2 MFMA blocks.  K advances one 32-code chunk at a time.  For chunk c, lane
// (j = l & 15, kq = l >> 4) serves MFMA step t (0..7) with code k = 32 c + 8 kq + t, so
// each lane reads 8 consecutive activations of its A rows (two 16-byte loads for fp32,
// one for fp16 / bf16) and 8 consecutive codes of its B rows (one word for W4, half a
// word for W2, 24 bits across at most two words for W3), which it turns into W-hat in
// registers: fma(q, s, -z s).  No LDS: operands come straight from the caches, and the
// next chunk's raw words and activations are requested before the current chunk's 32
// MFMAs, so the loads of one chunk overlap the matrix work of the previous one.
#include "cbk_device.hpp"
#include "cbk_kernels.hpp"

namespace cbk {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int TILE = 64;
constexpr int THREADS = 256;

// Raw operands of one chunk for one lane: 8 activations of each of its two A rows (as
// stored), and for each of its two B rows the word(s) holding its 8 codes plus the
// chunk's (scale, zero).
template <int DT>
struct Raw {
    uint32_t x[2][8];        // 16-bit dtypes use the low halves of x[a][0..3] as pairs
    uint32_t lo[2], hi[2];
    float s[2], z[2];
};

template <int DT, int BITS>
__device__ __forceinline__ void fetch(const GemmArgs& A, int c, int m0, int n0, int lane, Raw<DT>& R) {
    const int j = lane & 15, kq = lane >> 4;
    const int k0 = c * 32 + 8 * kq;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        const int m = m0 + a * 16 + j;
        const bool in = m < A.M;
        if constexpr (DT == DT_F32) {
            const float* row = reinterpret_cast<const float*>(A.x) + (long)m * A.K;
            if (A.xvec) {
                float4 u = make_float4(0.f, 0.f, 0.f, 0.f), v = u;
                if (in && k0 < A.K) {
                    u = *reinterpret_cast<const float4*>(row + k0);
                    v = *reinterpret_cast<const float4*>(row + k0 + 4);
                }
                R.x[a][0] = __float_as_uint(u.x); R.x[a][1] = __float_as_uint(u.y);
                R.x[a][2] = __float_as_uint(u.z); R.x[a][3] = __float_as_uint(u.w);
                R.x[a][4] = __float_as_uint(v.x); R.x[a][5] = __float_as_uint(v.y);
                R.x[a][6] = __float_as_uint(v.z); R.x[a][7] = __float_as_uint(v.w);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) R.x[a][e] = (in && k0 + e < A.K) ? __float_as_uint(row[k0 + e]) : 0u;
            }
        } else {
            const uint16_t* row = reinterpret_cast<const uint16_t*>(A.x) + (long)m * A.K;
            if (A.xvec) {
                uint4 u = make_uint4(0u, 0u, 0u, 0u);
                if (in && k0 < A.K) u = *reinterpret_cast<const uint4*>(row + k0);
                R.x[a][0] = u.x; R.x[a][1] = u.y; R.x[a][2] = u.z; R.x[a][3] = u.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t l = (in && k0 + 2 * e < A.K) ? row[k0 + 2 * e] : 0u;
                    const uint32_t h = (in && k0 + 2 * e + 1 < A.K) ? row[k0 + 2 * e + 1] : 0u;
                    R.x[a][e] = l | (h << 16);
                }
            }
        }
    }
    constexpr int OB = 8 * BITS;                       // bits of a lane's 8 codes
    const int ob = OB * kq, wi = ob >> 5, sh = ob & 31;
    const int g = (int)fdiv((uint32_t)(c * 32), A.divG);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int n = n0 + b * 16 + j;
        uint32_t lo = 0u, hi = 0u;
        float sc = 0.f, ze = 0.f;
        if (n < A.N) {
            const uint32_t* cw = A.w + (long)n * A.wpr + (long)c * BITS + wi;
            lo = cw[0];
            if (sh + OB > 32) hi = cw[1];
            sc = load_f<DT>(A.s, (long)n * A.G + g);
            ze = load_f<DT>(A.z, (long)n * A.G + g);
        }
        R.lo[b] = lo;
        R.hi[b] = hi;
        R.s[b] = sc;
        R.z[b] = ze;
    }
}

template <int DT>
__device__ __forceinline__ float x_at(const Raw<DT>& R, int a, int t) {
    if constexpr (DT == DT_F32) {
        return __uint_as_float(R.x[a][t]);
    } else {
        const uint32_t w = R.x[a][t >> 1];
        const uint16_t h = (t & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
        if constexpr (DT == DT_F16) return (float)__builtin_bit_cast(_Float16, h);
        else return __uint_as_float((uint32_t)h << 16);
    }
}

template <int DT, int BITS>
__device__ __forceinline__ void chunk_mma(const Raw<DT>& R, int kq, f4 (&acc)[2][2]) {
    constexpr int OB = 8 * BITS;
    const int sh = (OB * kq) & 31;
    constexpr uint32_t MASK = (1u << BITS) - 1u;
    float xa[2][8], wb[2][8];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int t = 0; t < 8; ++t) xa[a][t] = x_at<DT>(R, a, t);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const uint32_t f = (uint32_t)((((uint64_t)R.hi[b] << 32) | R.lo[b]) >> sh);
        const float nzs = -R.z[b] * R.s[b];
#pragma unroll
        for (int t = 0; t < 8; ++t) wb[b][t] = fmaf((float)((f >> (t * BITS)) & MASK), R.s[b], nzs);
    }
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[a][t], wb[b][t], acc[a][b], 0, 0, 0);
}

template <int DT, int BITS>
__global__ void __launch_bounds__(THREADS) gemm_f32_kernel(const GemmArgs A) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // one-dimensional grid, N tiles fastest (neighbouring workgroups share x rows)
    const int ntn = (A.N + TILE - 1) / TILE;
    const int mt = (int)(blockIdx.x / (uint32_t)ntn), nt = (int)(blockIdx.x - (uint32_t)mt * ntn);
    const int m0 = mt * TILE + wm * 32, n0 = nt * TILE + wn * 32;
    const int j = lane & 15, kq = lane >> 4;

    f4 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};

    Raw<DT> cur, nxt;
    fetch<DT, BITS>(A, 0, m0, n0, lane, cur);
    for (int c = 0; c < A.C; ++c) {
        if (c + 1 < A.C) fetch<DT, BITS>(A, c + 1, m0, n0, lane, nxt);
        chunk_mma<DT, BITS>(cur, kq, acc);
        cur = nxt;
    }

    // D: lane (j, kq) register r holds row 4 kq + r of a block, column j
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int n = n0 + b * 16 + j;
        if (n >= A.N) continue;
        const float bias = A.b ? load_f<DT>(A.b, n) : 0.f;
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + a * 16 + 4 * kq + r;
                if (m < A.M) store_f<DT>(A.out, (long)m * A.N + n, apply_act(acc[a][b][r] + bias, A.act));
            }
    }
}

template <int DT>
const void* f32_for_bits(int bits) {
    if (bits == 2) return reinterpret_cast<const void*>(&gemm_f32_kernel<DT, 2>);
    if (bits == 3) return reinterpret_cast<const void*>(&gemm_f32_kernel<DT, 3>);
    return reinterpret_cast<const void*>(&gemm_f32_kernel<DT, 4>);
}

}  // namespace

hipError_t launch_gemm_f32(const GemmArgs& A, int dt, hipStream_t stream) {
    const void* f = dt == DT_F16 ? f32_for_bits<DT_F16>(A.bits)
                  : dt == DT_BF16 ? f32_for_bits<DT_BF16>(A.bits) : f32_for_bits<DT_F32>(A.bits);
    const int64_t tiles = (int64_t)((A.N + TILE - 1) / TILE) * ((A.M + TILE - 1) / TILE);
    if (tiles >= INT32_MAX) return hipErrorInvalidValue;
    void* args[] = {const_cast<GemmArgs*>(&A)};
    return launch(f, dim3((unsigned)tiles), dim3(THREADS), args, 0, stream);
}

}  // namespace cbk
