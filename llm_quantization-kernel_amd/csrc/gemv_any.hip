// gemv_any.hip -- decode GEMV for every activation dtype, group size and row layout, on
// the fp32 matrix cores; and the launch that combines split-K partials.
//
// Takes the decode calls the streaming kernels (gemv_stream.hip) do not: fp32
// activations at any batch, fp16 / bf16 activations that are not 16-byte aligned (or
// K % 8 != 0), group sizes 32 and 64 at batch 3..16, and batches above 16.  It keeps
// the reference decode's arithmetic contract (Kernel/csrc/packed_gemv.cu:84-163): fp32
// throughout from the T inputs, one rounding to T at the end, for the plain, fused-QKV
// (mixed widths included) and fused gate-up modes.
//
// Every product runs on v_mfma_f32_16x16x4_f32, fp32 operands and fp32 accumulation:
//   D[i][j] += sum_kq A[i][kq] B[kq][j],   A 16 x 4 (activations), B 4 x 16 (weights).
// Job = (K split p, tile of 16 virtual rows, tile of 16 batch rows); a workgroup of NW
// waves (1..16, set by the host so the launch fills the CUs without extra splits) takes
// one job, wave w the chunks c0 + w, c0 + w + NW, ... of the split (the waves walk the
// rows' words side by side).  For chunk c, lane (j = l & 15, kq = l >> 4)
// serves MFMA step t (0..7) with code k = 32 c + 8 kq + t:
//   * A[j][kq] = x[batch row j][k], converted to fp32 (8 consecutive activations per
//     lane and chunk: one 16-byte load for fp16 / bf16, two for fp32);
//   * B[kq][j] = (q - z) s for virtual row j at code k -- the lane's 8 codes are the
//     8 BITS consecutive bits at 8 kq BITS of the chunk (one word for W4, half a word
//     for W2, 24 bits across at most two words for W3), extracted by v_bfe_u32, and
//     W-hat = fma(q, s, -z s) (exactly (q - z) s in fp32 for fp16 / bf16 metadata with
//     integer zeros; one fp32 rounding otherwise, as the reference's s (d - z sum x));
// so the lane's eight MFMAs cover the chunk's 32 codes.  Group sizes are multiples of
// 32, so a chunk lies in one group and a lane needs one (scale, zero) per chunk.
// D's lane (j, kq) register r holds batch row 4 kq + r of virtual row j.  The waves'
// tiles meet in LDS and are added in wave order; then a finish unit (a row, or a row pair
// in the fused modes) per thread is finished (finish), or with P > 1 the fp32 partials
// are stored and the last split of the block combines them in the dispatch
// (split_arrive), or a combine launch does.
#include "cbk_device.hpp"
#include "cbk_kernels.hpp"

namespace cbk {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int MAX_WAVES = ANY_MAX_THREADS / 64;

// The lane's 8 activations of chunk c for batch row b, as fp32 (zero past M or K).
// `vec`: x is 16-byte aligned and K % 8 == 0, so an 8-code piece lies wholly before or
// past K and is one (fp16 / bf16) or two (fp32) aligned 16-byte loads.
template <int DT>
__device__ __forceinline__ void load_x8(const GemvArgs& A, bool vec, int b, int k0, float (&xf)[8]) {
    using S = typename Dt<DT>::S;
    const S* row = reinterpret_cast<const S*>(A.x) + (long)b * A.K;
    const bool in = b < A.M;
    if (vec) {
        if (in && k0 < A.K) {
            if constexpr (DT == DT_F32) {
                const float4 u = *reinterpret_cast<const float4*>(row + k0);
                const float4 v = *reinterpret_cast<const float4*>(row + k0 + 4);
                xf[0] = u.x; xf[1] = u.y; xf[2] = u.z; xf[3] = u.w;
                xf[4] = v.x; xf[5] = v.y; xf[6] = v.z; xf[7] = v.w;
            } else {
                const uint4 u = *reinterpret_cast<const uint4*>(row + k0);
                const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    xf[2 * e] = Dt<DT>::to_f((S)(uint16_t)(w[e] & 0xffffu));
                    xf[2 * e + 1] = Dt<DT>::to_f((S)(uint16_t)(w[e] >> 16));
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) xf[e] = 0.f;
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[e] = (in && k0 + e < A.K) ? Dt<DT>::to_f(row[k0 + e]) : 0.f;
    }
}

// fp16 bit patterns reinterpreted: the storage type of DT_F16 is _Float16, so a raw
// 16-bit pattern needs a bit cast rather than a value conversion.
template <>
__device__ __forceinline__ void load_x8<DT_F16>(const GemvArgs& A, bool vec, int b, int k0, float (&xf)[8]) {
    const _Float16* row = reinterpret_cast<const _Float16*>(A.x) + (long)b * A.K;
    const bool in = b < A.M;
    if (vec) {
        if (in && k0 < A.K) {
            typedef _Float16 h8 __attribute__((ext_vector_type(8)));
            const h8 h = *reinterpret_cast<const h8*>(row + k0);
#pragma unroll
            for (int e = 0; e < 8; ++e) xf[e] = (float)h[e];
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) xf[e] = 0.f;
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[e] = (in && k0 + e < A.K) ? (float)row[k0 + e] : 0.f;
    }
}

template <int DT, int MODE>
__global__ void __launch_bounds__(ANY_MAX_THREADS) gemv_any_kernel(const GemvArgs A) {
    __shared__ f4 red[MAX_WAVES][64];
    __shared__ int flag;
    const int tid = threadIdx.x, lane = tid & 63, nthr = (int)blockDim.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nw = nthr >> 6;
    const int j = lane & 15, kq = lane >> 4;

    // job -> (split p, row tile, batch tile), the splits of a block adjacent
    const uint32_t job = blockIdx.x;
    const uint32_t blk = fdiv(job, A.divP);
    const int p = (int)(job - blk * (uint32_t)A.P);
    const int bt = (int)fdiv(blk, A.divT);
    const int tile = (int)(blk - (uint32_t)bt * (uint32_t)A.ntiles);
    const int c0 = (int)(((int64_t)A.C * p) / A.P);
    const int c1 = (int)(((int64_t)A.C * (p + 1)) / A.P);

    // the lane's weight row (virtual row tile * 16 + j) and activation row (bt * 16 + j)
    const int v = tile * 16 + j;
    const bool vin = v < A.V;
    int proj, r;
    vmap<MODE>(A, vin ? v : 0, proj, r);
    const Src S = src_of(A, proj);
    const uint32_t* wrow = S.w + (long)r * S.wpr;
    const int bits = bits_of(A, proj);
    const int ob = 8 * kq * bits;                   // bit offset of the lane's codes in a chunk
    const int wi = ob >> 5, sh = ob & 31;
    const bool two_words = sh + 8 * bits > 32;      // W3, kq = 1 and 2
    const uint32_t mask = (1u << bits) - 1u;
    const int b = bt * 16 + j;
    const bool vec = A.st_xvec != 0;

    f4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int c = c0 + wave; c < c1; c += nw) {
        float xf[8];
        load_x8<DT>(A, vec, b, c * 32 + 8 * kq, xf);
        float wh[8];
        if (vin) {
            const int g = (int)fdiv((uint32_t)c, A.divGS);
            const float s = load_f<DT>(S.s, (long)r * A.G + g);
            const float nzs = -load_f<DT>(S.z, (long)r * A.G + g) * s;
            const uint32_t* cw = wrow + (long)c * bits + wi;
            const uint32_t lo = cw[0];
            const uint32_t hi = two_words ? cw[1] : 0u;
            const uint32_t f = (uint32_t)((((uint64_t)hi << 32) | lo) >> sh);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const uint32_t q = (f >> (t * bits)) & mask;         // v_bfe_u32
                wh[t] = fmaf((float)q, s, nzs);
            }
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) wh[t] = 0.f;
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[t], wh[t], acc, 0, 0, 0);
    }

    // the waves' tiles meet in LDS, added in wave order
    red[wave][lane] = acc;
    __syncthreads();
    const float* rf = reinterpret_cast<const float*>(&red[0][0]);
    const int mt = min(16, A.M - bt * 16);           // batch rows of this tile
    const int vbase = tile * 16;
    // a finish unit (a row, or a row pair in the fused modes) per thread: t -> (batch
    // row i, unit); the value of (i, row) sits in lane row + 16 (i >> 2), register i & 3
    constexpr int U = FINISH_ROWS<MODE>;
    constexpr int NU = 16 / U;
    for (int t = tid; t < 16 * NU; t += nthr) {
        const int i = t / NU, row = U * (t % NU);
        const int v0 = vbase + row;
        if (i < mt && v0 < A.V) {
            const int l0 = row + 16 * (i >> 2), q = i & 3;
            float y0 = 0.f, y1 = 0.f;
            for (int w = 0; w < nw; ++w) {
                y0 += rf[(w * 64 + l0) * 4 + q];
                if constexpr (U == 2) y1 += rf[(w * 64 + l0 + 1) * 4 + q];
            }
            const bool two = U == 2 && v0 + 1 < A.V;
            if (A.P == 1) finish<DT, MODE>(A, bt * 16 + i, v0, y0, y1, two);
            else put_unit(A, p, bt * 16 + i, v0, y0, y1, two);
        }
    }
    if (A.P > 1 && A.split_cnt && split_arrive(A, (int)blk, &flag)) {
        for (int t = tid; t < 16 * NU; t += nthr) {
            const int i = t / NU, v0 = vbase + U * (t % NU);
            if (i < mt && v0 < A.V) finish_from_partials<DT, MODE>(A, bt * 16 + i, v0);
        }
    }
}

// The combine launch (P > 1 without arrival counters): a finish unit of one batch row
// per thread, the P partials added in split order.
template <int DT, int MODE>
__global__ void __launch_bounds__(256) gemv_combine_kernel(const GemvArgs A) {
    constexpr int U = FINISH_ROWS<MODE>;
    const int64_t nu = (A.V + U - 1) / U;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= (int64_t)A.M * nu) return;
    const int b = (int)(t / nu);
    const int v0 = (int)(U * (t - (int64_t)b * nu));
    finish_from_partials<DT, MODE>(A, b, v0);
}

template <int DT>
const void* any_for_mode(int mode) {
    if (mode == MODE_QKV) return reinterpret_cast<const void*>(&gemv_any_kernel<DT, MODE_QKV>);
    if (mode == MODE_GATEUP) return reinterpret_cast<const void*>(&gemv_any_kernel<DT, MODE_GATEUP>);
    return reinterpret_cast<const void*>(&gemv_any_kernel<DT, MODE_GEMV>);
}

template <int DT>
const void* combine_for_mode(int mode) {
    if (mode == MODE_QKV) return reinterpret_cast<const void*>(&gemv_combine_kernel<DT, MODE_QKV>);
    if (mode == MODE_GATEUP) return reinterpret_cast<const void*>(&gemv_combine_kernel<DT, MODE_GATEUP>);
    return reinterpret_cast<const void*>(&gemv_combine_kernel<DT, MODE_GEMV>);
}

}  // namespace

const void* gemv_any_kernel_for(int dt, int mode) {
    if (dt == DT_F16) return any_for_mode<DT_F16>(mode);
    if (dt == DT_BF16) return any_for_mode<DT_BF16>(mode);
    return any_for_mode<DT_F32>(mode);
}

hipError_t launch_gemv_combine(const GemvArgs& A, int dt, int mode, hipStream_t stream) {
    const int64_t total = (int64_t)A.M * (mode == MODE_GEMV ? A.V : (A.V + 1) >> 1);
    const void* f = dt == DT_F16 ? combine_for_mode<DT_F16>(mode)
                  : dt == DT_BF16 ? combine_for_mode<DT_BF16>(mode) : combine_for_mode<DT_F32>(mode);
    void* args[] = {const_cast<GemvArgs*>(&A)};
    return launch(f, dim3((unsigned)((total + 255) / 256)), dim3(256), args, 0, stream);
}

}  // namespace cbk
