// gemm.hip -- prefill packed GEMM: out[M,N] = act(x . W-hat^T + bias).
//
// The matrix-core prefill for fp16 / bf16 shapes gemm_f16.hip does not take (K % 8 != 0,
// x or metadata not 16-byte aligned): cb_gemm_tc_kernel's contract
// (Kernel/csrc/packed_gemm.cu:12-115).
//
// gemm_mfma_kernel (fp16 / bf16): 128x128 output tile, 4 waves in a 2x2 grid of
// 64x64 wave tiles, K staged one 32-code chunk at a time through double-buffered
// LDS.  The weight tile is dequantized while it is written to LDS:
// W-hat = RN_T((q - z) * s) -- the product of an integer in [-15, 15] and a 16-bit
// float is exact in fp32, so this equals the reference's rounding
// (packed_gemm.cu:56,60).  Products run on v_mfma_f32_16x16x32_{f16,bf16} with fp32
// accumulation; bias and activation are applied in fp32 before the final rounding.
#include "cbk_device.hpp"
#include "cbk_kernels.hpp"

namespace cbk {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int LDK = BK + 8;                 // LDS row pitch in halves (80 B): conflict-free b128 reads
constexpr int THREADS = 256;

template <int DT>
__device__ __forceinline__ f4 mfma(const u4& a, const u4& b, const f4& c) {
    if constexpr (DT == DT_F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const h8*>(&a),
                                                      *reinterpret_cast<const h8*>(&b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(*reinterpret_cast<const b8*>(&a),
                                                       *reinterpret_cast<const b8*>(&b), c, 0, 0, 0);
}

template <int DT>
__device__ __forceinline__ uint16_t to_bits(float f) {
    if constexpr (DT == DT_F16) {
        const _Float16 h = (_Float16)f;
        return *reinterpret_cast<const uint16_t*>(&h);
    } else {
        return Dt<DT_BF16>::from_f(f);
    }
}

struct StageRegs {
    u4 a[2];            // 16 activation halves of one row
    uint32_t w[4];      // packed chunk words (BITS used)
    float s, z;
};

template <int DT, int BITS>
__device__ __forceinline__ void load_stage(const GemmArgs& A, int m0, int n0, int kc, StageRegs& R) {
    const int t = threadIdx.x;
    // activation: row t/2, halves (t%2)*16 .. +16 of chunk kc
    {
        const int m = m0 + (t >> 1);
        const int k = kc * 32 + (t & 1) * 16;
        const uint16_t* x = reinterpret_cast<const uint16_t*>(A.x);
        if (m < A.M && k + 16 <= A.K && (A.K & 7) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
            const u4* p = reinterpret_cast<const u4*>(x + (long)m * A.K + k);
            R.a[0] = p[0];
            R.a[1] = p[1];
        } else {
            uint16_t v[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] = (m < A.M && k + e < A.K) ? x[(long)m * A.K + k + e] : (uint16_t)0;
#pragma unroll
            for (int q = 0; q < 2; ++q)
                R.a[q] = u4{v[8 * q] | ((uint32_t)v[8 * q + 1] << 16), v[8 * q + 2] | ((uint32_t)v[8 * q + 3] << 16),
                            v[8 * q + 4] | ((uint32_t)v[8 * q + 5] << 16), v[8 * q + 6] | ((uint32_t)v[8 * q + 7] << 16)};
        }
    }
    // weights: row t % 128 (both halves of the workgroup load the same chunk)
    {
        const int n = n0 + (t & 127);
        if (n < A.N) {
            const uint32_t* wp = A.w + (long)n * A.wpr + (long)kc * BITS;
#pragma unroll
            for (int i = 0; i < BITS; ++i) R.w[i] = wp[i];
            const int g = (kc * 32) / A.gs;
            R.s = load_f<DT>(A.s, (long)n * A.G + g);
            R.z = load_f<DT>(A.z, (long)n * A.G + g);
        } else {
#pragma unroll
            for (int i = 0; i < BITS; ++i) R.w[i] = 0u;
            R.s = 0.f;
            R.z = 0.f;
        }
    }
}

template <int DT, int BITS>
__device__ __forceinline__ void store_stage(const StageRegs& R, uint16_t* sa, uint16_t* sb) {
    const int t = threadIdx.x;
    u4* ad = reinterpret_cast<u4*>(sa + (t >> 1) * LDK + (t & 1) * 16);
    ad[0] = R.a[0];
    ad[1] = R.a[1];
    // dequantize codes 16h .. 16h+15 (h uniform per wave) of the chunk
    const int h = t >> 7;
    uint32_t w[BITS];
#pragma unroll
    for (int i = 0; i < BITS; ++i) w[i] = R.w[i];
    uint32_t outw[8];
    if (h == 0) {
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
            const float lo = ((float)chunk_code<BITS>(w, e) - R.z) * R.s;
            const float hi = ((float)chunk_code<BITS>(w, e + 1) - R.z) * R.s;
            outw[e >> 1] = to_bits<DT>(lo) | ((uint32_t)to_bits<DT>(hi) << 16);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
            const float lo = ((float)chunk_code<BITS>(w, 16 + e) - R.z) * R.s;
            const float hi = ((float)chunk_code<BITS>(w, 17 + e) - R.z) * R.s;
            outw[e >> 1] = to_bits<DT>(lo) | ((uint32_t)to_bits<DT>(hi) << 16);
        }
    }
    u4* bd = reinterpret_cast<u4*>(sb + (t & 127) * LDK + h * 16);
    bd[0] = u4{outw[0], outw[1], outw[2], outw[3]};
    bd[1] = u4{outw[4], outw[5], outw[6], outw[7]};
}

template <int DT, int BITS>
__global__ void __launch_bounds__(THREADS) gemm_mfma_kernel(const GemmArgs A) {
    __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN * LDK];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int i = lane & 15, kq = lane >> 4;

    f4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};

    StageRegs R;
    load_stage<DT, BITS>(A, m0, n0, 0, R);
    store_stage<DT, BITS>(R, sA[0], sB[0]);
    __syncthreads();

    for (int kc = 0; kc < A.C; ++kc) {
        const int cur = kc & 1;
        if (kc + 1 < A.C) load_stage<DT, BITS>(A, m0, n0, kc + 1, R);
        u4 af[4], bf[4];
#pragma unroll
        for (int a = 0; a < 4; ++a)
            af[a] = *reinterpret_cast<const u4*>(sA[cur] + (wm * 64 + a * 16 + i) * LDK + kq * 8);
#pragma unroll
        for (int b = 0; b < 4; ++b)
            bf[b] = *reinterpret_cast<const u4*>(sB[cur] + (wn * 64 + b * 16 + i) * LDK + kq * 8);
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b) acc[a][b] = mfma<DT>(af[a], bf[b], acc[a][b]);
        if (kc + 1 < A.C) store_stage<DT, BITS>(R, sA[cur ^ 1], sB[cur ^ 1]);
        __syncthreads();
    }

    // D layout: lane holds rows 4*kq + r of a 16x16 block, column i
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const int n = n0 + wn * 64 + b * 16 + i;
        if (n >= A.N) continue;
        const float bias = A.b ? load_f<DT>(A.b, n) : 0.f;
#pragma unroll
        for (int a = 0; a < 4; ++a) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * 64 + a * 16 + kq * 4 + r;
                if (m < A.M) store_f<DT>(A.out, (long)m * A.N + n, apply_act(acc[a][b][r] + bias, A.act));
            }
        }
    }
}

template <int DT>
const void* mfma_for_bits(int bits) {
    if (bits == 2) return reinterpret_cast<const void*>(&gemm_mfma_kernel<DT, 2>);
    if (bits == 3) return reinterpret_cast<const void*>(&gemm_mfma_kernel<DT, 3>);
    return reinterpret_cast<const void*>(&gemm_mfma_kernel<DT, 4>);
}

}  // namespace

hipError_t launch_gemm_mfma(const GemmArgs& A, int dt, hipStream_t stream) {
    const void* f = dt == DT_F16 ? mfma_for_bits<DT_F16>(A.bits) : mfma_for_bits<DT_BF16>(A.bits);
    void* args[] = {const_cast<GemmArgs*>(&A)};
    return launch(f, dim3((A.N + BN - 1) / BN, (A.M + BM - 1) / BM), dim3(THREADS), args, 0, stream);
}

}  // namespace cbk
