// gemv_mfma.hip -- fp16 decode GEMV / fused gate-up / fused QKV on gfx950 MFMA.
//
// Replaces cb_gemv_kernel (Kernel/csrc/packed_gemv.cu:83-163) for fp16 activations
// and group sizes that are multiples of 128.
//
// Work decomposition
//   job        = (batch tile of <=16 rows, tile of 16 virtual rows, K split p)
//   workgroup  = NW waves on one job; wave w takes 128-code units w, w+NW, ... of
//                the split's K range; the NW partial sums meet in LDS.
//   unit       = 4 chunks (128 codes) x 16 rows: one dwordx4/x3/x2 load per lane
//                (lane = row (l & 15), chunk (l >> 4)), 16 rows x 64/48/32
//                contiguous bytes per instruction.
//
// Arithmetic per unit: the chunk is decoded to packed fp16 1024+q (cbk_decode.hpp)
// and fed as the B operand of four v_mfma_f32_16x16x32_f16 whose A operand is the
// activation staged in LDS in the matching code order, so
//   D[i][j] = sum_k x[i][k] * (1024 + q[j][k])          (fp32 accumulate)
//   acc[i][j] += s[j] * (D[i][j] - (1024 + z[j]) * X[i])  with X[i] = sum_k x[i][k].
// This is the reference's per-chunk s*(sum x q - z sum x) (packed_gemv.cu:133-135)
// with the int->float conversion folded into the fp16 bit pattern.
//
// LDS: staged activation (units x 4 operands x 4 chunks x Mt x 16 B), per-unit
// activation sums (units x 16 floats) and the cross-wave reduction (NW x 1 KB).
#include "cbk_device.hpp"
#include "cbk_decode.hpp"
#include "cbk_kernels.hpp"

namespace cbk {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

constexpr int PF = 8;          // units in flight per wave

template <int BITS> struct Slot {
    uint32_t w[BITS];
    _Float16 s, z;
};

template <int BITS>
__device__ __forceinline__ void load_chunk(const uint32_t* p, uint32_t (&w)[BITS]) {
    if constexpr (BITS == 4) {
        const u4 v = __builtin_nontemporal_load(reinterpret_cast<const u4*>(p));
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (BITS == 2) {
        const u2 v = __builtin_nontemporal_load(reinterpret_cast<const u2*>(p));
        w[0] = v.x; w[1] = v.y;
    } else {
        w[0] = __builtin_nontemporal_load(p);
        w[1] = __builtin_nontemporal_load(p + 1);
        w[2] = __builtin_nontemporal_load(p + 2);
    }
}

// Per-lane view of the row this lane streams in the current job.
struct RowPtr {
    const uint32_t* w;      // packed row
    const _Float16* s;      // scales row
    const _Float16* z;      // zeros row
    int valid;
};

template <int MODE>
__device__ __forceinline__ RowPtr row_ptr(const GemvArgs& A, int v) {
    RowPtr rp;
    rp.valid = v < A.V;
    int proj = 0, r = 0;
    if (rp.valid) vmap<MODE>(A, v, proj, r);
    const uint32_t* w = CBK_SEL(A, proj, w);
    const int wpr = CBK_SEL(A, proj, wpr);
    rp.w = w + (long)r * wpr;
    rp.s = reinterpret_cast<const _Float16*>(CBK_SEL(A, proj, s)) + (long)r * A.G;
    rp.z = reinterpret_cast<const _Float16*>(CBK_SEL(A, proj, z)) + (long)r * A.G;
    return rp;
}

template <int BITS>
__device__ __forceinline__ void load_slot(const GemvArgs& A, const RowPtr& rp, int unit, int kq, Slot<BITS>& sl) {
    const int c = unit * 4 + kq;
    if (rp.valid && c < A.C) {
        load_chunk<BITS>(rp.w + (long)c * BITS, sl.w);
    } else {
#pragma unroll
        for (int i = 0; i < BITS; ++i) sl.w[i] = 0u;
    }
    if (rp.valid) {
        const int g = (unit * 128) / A.gs;
        sl.s = rp.s[g];
        sl.z = rp.z[g];
    } else {
        sl.s = (_Float16)0.f;
        sl.z = (_Float16)0.f;
    }
}

// Stage x[b0 + i][32c .. 32c+32) for the job's units into LDS in decode order
// (one task per (chunk, batch row)), then the per-unit activation sums
// X[u][i] = sum of the unit's 4 chunk sums, in a fixed order.
template <int BITS>
__device__ void stage_x(const GemvArgs& A, int b0, int mt, int u0, int nu, char* lds) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const _Float16* x = reinterpret_cast<const _Float16*>(A.x);
    u4* xs = reinterpret_cast<u4*>(lds);
    float* xsum = reinterpret_cast<float*>(lds + A.xs_bytes);
    float* csum = reinterpret_cast<float*>(lds + A.red_off);     // reuses the reduction area
    const int nthreads = blockDim.x;
    const bool vec = ((A.K & 7) == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0);
    const h2 one2 = {(_Float16)1.f, (_Float16)1.f};
    for (int task = threadIdx.x; task < nu * 4 * mt; task += nthreads) {
        const int i = task % mt, cl = task / mt;           // local chunk cl = 4*ul + kq
        const int ul = cl >> 2, kq = cl & 3;
        const _Float16* xr = x + (long)(b0 + i) * A.K;
        const int k0 = (u0 * 4 + cl) * 32;
        _Float16 xv[32];
        if (vec && k0 + 32 <= A.K) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const h8 v = *reinterpret_cast<const h8*>(xr + k0 + 8 * q);
#pragma unroll
                for (int e = 0; e < 8; ++e) xv[8 * q + e] = v[e];
            }
        } else {
#pragma unroll
            for (int e = 0; e < 32; ++e) xv[e] = (k0 + e < A.K) ? xr[k0 + e] : (_Float16)0.f;
        }
        float sum = 0.f;
#pragma unroll
        for (int e = 0; e < 32; e += 2) {
            const h2 pr = {xv[e], xv[e + 1]};
            sum = __builtin_amdgcn_fdot2(pr, one2, sum, false);
        }
        csum[cl * mt + i] = sum;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            h8 op;
#pragma unroll
            for (int p = 0; p < 8; ++p) op[p] = xv[Decode<BITS>::kappa(8 * m + p)];
            xs[((ul * 4 + m) * 4 + kq) * mt + i] = *reinterpret_cast<u4*>(&op);
        }
    }
    __syncthreads();
    for (int task = threadIdx.x; task < nu * 16; task += nthreads) {
        const int i = task & 15, ul = task >> 4;
        float X = 0.f;
        if (i < mt) {
#pragma unroll
            for (int kq = 0; kq < 4; ++kq) X += csum[(ul * 4 + kq) * mt + i];
        }
        xsum[ul * 16 + i] = X;
    }
}

template <int BITS, int MB>
__device__ __forceinline__ void unit_math(const Slot<BITS>& sl, const char* lds, int xs_bytes, int ul, int mt,
                                          int lane, f4& acc) {
    const u4* xs = reinterpret_cast<const u4*>(lds);
    const float* xsum = reinterpret_cast<const float*>(lds + xs_bytes);
    const int i = lane & 15, kq = lane >> 4;
    uint32_t h[16];
    Decode<BITS>::run(sl.w, h);
    f4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        u4 a = {0u, 0u, 0u, 0u};
        if (i < mt) a = xs[((ul * 4 + m) * 4 + kq) * mt + i];
        const u4 bw = {h[4 * m], h[4 * m + 1], h[4 * m + 2], h[4 * m + 3]};
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const h8*>(&a),
                                                   *reinterpret_cast<const h8*>(&bw), d, 0, 0, 0);
    }
    const f4 X = *reinterpret_cast<const f4*>(xsum + ul * 16 + 4 * kq);
    const float s = (float)sl.s;
    const float zb = 1024.f + (float)sl.z;
#pragma unroll
    for (int r = 0; r < (MB == 1 ? 1 : 4); ++r) acc[r] = fmaf(s, fmaf(-zb, X[r], d[r]), acc[r]);
}

template <int BITS, int MODE, int MB>
__device__ void run_job(const GemvArgs& A, int job, char* lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int NW = A.nw;
    const int p = job % A.P;
    const int rest = job / A.P;
    const int tile = rest % A.ntiles;
    const int mtile = rest / A.ntiles;
    const int b0 = mtile * 16;
    const int mt = min(16, A.M - b0);
    const int u0 = (int)(((long)A.units * p) / A.P);
    const int u1 = (int)(((long)A.units * (p + 1)) / A.P);
    const int nu = u1 - u0;

    const int j = lane & 15, kq = lane >> 4;
    const RowPtr rp = row_ptr<MODE>(A, tile * 16 + j);
    const int my = wave < nu ? (nu - wave + NW - 1) / NW : 0;    // units of this wave

    Slot<BITS> sl[PF];
#pragma unroll
    for (int s = 0; s < PF; ++s)
        if (s < my) load_slot<BITS>(A, rp, u0 + wave + s * NW, kq, sl[s]);

    stage_x<BITS>(A, b0, mt, u0, nu, lds);
    __syncthreads();

    f4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int base = 0; base < my; base += PF) {
#pragma unroll
        for (int s = 0; s < PF; ++s) {
            const int it = base + s;
            if (it < my) {
                unit_math<BITS, MB>(sl[s], lds, A.xs_bytes, wave + it * NW, mt, lane, acc);
                if (it + PF < my) load_slot<BITS>(A, rp, u0 + wave + (it + PF) * NW, kq, sl[s]);
            }
        }
    }

    // cross-wave sum in fixed wave order, then the epilogue on wave 0
    f4* red = reinterpret_cast<f4*>(lds + A.red_off);
    if (wave > 0) red[(wave - 1) * 64 + lane] = acc;
    __syncthreads();
    if (wave == 0) {
        for (int w = 1; w < NW; ++w) {
            const f4 o = red[(w - 1) * 64 + lane];
            acc[0] += o[0]; acc[1] += o[1]; acc[2] += o[2]; acc[3] += o[3];
        }
        const int v = tile * 16 + j;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float partner = __shfl_xor(acc[r], 1, 64);
            const int i = 4 * kq + r;
            if (i < mt && v < A.V) {
                if (A.P == 1) epilogue<DT_F16, MODE>(A, b0 + i, v, acc[r], partner);
                else A.partial[((long)p * A.M + b0 + i) * A.V + v] = acc[r];
            }
        }
    }
    __syncthreads();   // LDS is reused by the next job
}

template <int BITS, int MODE, int MB>
__global__ void __launch_bounds__(512) gemv_mfma_kernel(const GemvArgs A) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    for (int job = blockIdx.x; job < A.jobs; job += gridDim.x) run_job<BITS, MODE, MB>(A, job, lds);
}

// Mixed-width fused QKV: every 16-row tile lies inside one projection (the host
// checks nq and nk are multiples of 16), so the width is uniform per job.
template <int MB>
__global__ void __launch_bounds__(512) gemv_mfma_qkv_mixed_kernel(const GemvArgs A) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    for (int job = blockIdx.x; job < A.jobs; job += gridDim.x) {
        const int v0 = ((job / A.P) % A.ntiles) * 16;
        const int proj = v0 < A.p[0].n ? 0 : (v0 < A.p[0].n + A.p[1].n ? 1 : 2);
        const int bits = CBK_SEL(A, proj, bits);
        if (bits == 2) run_job<2, MODE_QKV, MB>(A, job, lds);
        else if (bits == 3) run_job<3, MODE_QKV, MB>(A, job, lds);
        else run_job<4, MODE_QKV, MB>(A, job, lds);
    }
}

template <int BITS, int MODE, int MB>
const void* pick_mb() { return reinterpret_cast<const void*>(&gemv_mfma_kernel<BITS, MODE, MB>); }

template <int MODE, int MB>
const void* pick_bits(int bits) {
    if (bits == 2) return pick_mb<2, MODE, MB>();
    if (bits == 3) return pick_mb<3, MODE, MB>();
    return pick_mb<4, MODE, MB>();
}

template <int MB>
const void* pick_mode(int mode, int bits, bool mixed) {
    if (mixed) return reinterpret_cast<const void*>(&gemv_mfma_qkv_mixed_kernel<MB>);
    if (mode == MODE_QKV) return pick_bits<MODE_QKV, MB>(bits);
    if (mode == MODE_GATEUP) return pick_bits<MODE_GATEUP, MB>(bits);
    return pick_bits<MODE_GEMV, MB>(bits);
}

}  // namespace

const void* gemv_mfma_kernel_for(int mode, int bits, bool mixed, int max_batch) {
    if (max_batch <= 1) return pick_mode<1>(mode, bits, mixed);
    return pick_mode<16>(mode, bits, mixed);
}

}  // namespace cbk
