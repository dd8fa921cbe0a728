// quant.hip -- on-device group-affine quantizer and bit packer (the format's producer).
//
// The GPU form of Kernel/crispybits_kernels/reference.py:10-27 (quantize_affine) and
// :37-55 (pack_codes), bit-identical to them: per row and group of gs codes along K
//   scale = max((max - min) / qmax, 1e-8),  zero = clamp(round(-min / scale), 0, qmax),
//   q = clamp(round(w / scale) + zero, 0, qmax)
// in IEEE fp32 (correctly rounded division, round-half-to-even), then each row's codes
// as an LSB-first bitstream of ceil(K/32) chunks of `bits` words, codes past K zero.
// The reference pads K to whole groups by repeating the last column; a repeated value
// is already in its group, so the min/max over the group's real columns are the same.
// Scheme 1 is the paper quantizer of quantization/crispybits_quant/affine.py:28-71 instead:
// min clamped to <= 0 and max to >= 0, scale 1 where (max - min) / qmax < 1e-8, and
// q = clamp(round(w / scale + zero), 0, qmax) (the zero added before rounding); the
// output layout is the same chunked bitstream.
//
// Vector path (group size 32..512 dividing 512, K % 8 == 0, 16-byte aligned weights): the
// weights are cut into pieces of 512 consecutive elements of a row, one 16-byte octet per
// lane.  A persistent grid sweeps the pieces in wave-strided order (at any moment the
// whole GPU reads one contiguous stretch), each wave keeping QUANT_DEPTH pieces in flight:
// a piece's registers are refilled with the load of a later piece as soon as they are
// consumed.  A group is gs/8 adjacent lanes: min/max by DPP inside it, then every lane
// quantizes its 8 codes into one 8*bits-bit field; the 4 lanes of a 32-code chunk see
// each other's fields by quad DPP broadcasts and lane j (< bits) assembles and stores word j.
//
// General path (any other shape): one wave per (row, group): lanes stride the group for
// the min/max, then quantize one code each, 32-code chunks two at a time, and OR the codes
// into the chunk's words in a per-wave LDS slot (a code that straddles two words ORs into
// both), which lanes 0 .. bits-1 store.
#include <algorithm>

#include "cbk_device.hpp"
#include "cbk_kernels.hpp"

namespace cbk {
namespace {

constexpr int WAVES = 4;
constexpr int PIECE = 512;          // elements per wave-wide piece (64 lanes x 8)
#ifndef CBK_QUANT_DEPTH
#define CBK_QUANT_DEPTH 4
#endif
constexpr int QUANT_DEPTH = CBK_QUANT_DEPTH;     // pieces in flight per wave
#ifndef CBK_QUANT_WGS_PER_CU
#define CBK_QUANT_WGS_PER_CU 8
#endif

// one lane's octet as loaded: 16 bytes (fp16 / bf16) or 32 (fp32)
template <int DT>
struct RawOctet {
    uint4 u[DT == DT_F32 ? 2 : 1];
};

template <int DT>
__device__ __forceinline__ void load_raw(const void* w, long e, RawOctet<DT>& r) {
    const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(w) +
                                                    e * (long)sizeof(typename Dt<DT>::S));
#pragma unroll
    for (int i = 0; i < (DT == DT_F32 ? 2 : 1); ++i) r.u[i] = p[i];
}

template <int DT>
__device__ __forceinline__ void unpack_raw(const RawOctet<DT>& r, float (&v)[8]) {
    if constexpr (DT == DT_F32) {
        const uint32_t h[8] = {r.u[0].x, r.u[0].y, r.u[0].z, r.u[0].w, r.u[1].x, r.u[1].y, r.u[1].z, r.u[1].w};
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(h[i]);
    } else {
        const uint32_t h[4] = {r.u[0].x, r.u[0].y, r.u[0].z, r.u[0].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint16_t a = (uint16_t)(h[i] & 0xffffu), b = (uint16_t)(h[i] >> 16);
            if constexpr (DT == DT_F16) {
                v[2 * i] = (float)__builtin_bit_cast(_Float16, a);
                v[2 * i + 1] = (float)__builtin_bit_cast(_Float16, b);
            } else {
                v[2 * i] = Dt<DT_BF16>::to_f(a);
                v[2 * i + 1] = Dt<DT_BF16>::to_f(b);
            }
        }
    }
}

template <int I>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {       // lane I of each quad
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x55 * I, 0xF, 0xF, false);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// min / max of two values as one med3 against -inf / +inf (no NaN canonicalisation of the
// DPP-moved operand, which fminf / fmaxf would add)
__device__ __forceinline__ float min2(float a, float b) { return __builtin_amdgcn_fmed3f(a, b, -__builtin_huge_valf()); }
__device__ __forceinline__ float max2(float a, float b) { return __builtin_amdgcn_fmed3f(a, b, __builtin_huge_valf()); }

// min and max over each aligned group of L lanes (L = 4 .. 64): quad xor 1 and 2, then
// row half-mirror (joins the two quads of 8 lanes), row mirror (the two halves of 16),
// then xor shuffles across rows.
template <int L>
__device__ __forceinline__ void group_minmax(float& lo, float& hi) {
    lo = min2(lo, dpp_f<0xB1>(lo)); hi = max2(hi, dpp_f<0xB1>(hi));              // quad_perm [1,0,3,2]
    lo = min2(lo, dpp_f<0x4E>(lo)); hi = max2(hi, dpp_f<0x4E>(hi));              // quad_perm [2,3,0,1]
    if constexpr (L >= 8) { lo = min2(lo, dpp_f<0x141>(lo)); hi = max2(hi, dpp_f<0x141>(hi)); }
    if constexpr (L >= 16) { lo = min2(lo, dpp_f<0x140>(lo)); hi = max2(hi, dpp_f<0x140>(hi)); }
    if constexpr (L >= 32) { lo = min2(lo, __shfl_xor(lo, 16, 64)); hi = max2(hi, __shfl_xor(hi, 16, 64)); }
    if constexpr (L >= 64) { lo = min2(lo, __shfl_xor(lo, 32, 64)); hi = max2(hi, __shfl_xor(hi, 32, 64)); }
}

// scale and zero of one group in the metadata dtype (fp16 / bf16 by their RNE conversions)
__device__ __forceinline__ void store_meta2(int mdt, void* sp, void* zp, long i, float s, float z) {
    if (mdt == DT_F32) {
        store_f<DT_F32>(sp, i, s);
        store_f<DT_F32>(zp, i, z);
    } else {
        const bool bf = mdt == DT_BF16;
        const uint16_t sb = bf ? Dt<DT_BF16>::from_f(s) : __builtin_bit_cast(uint16_t, Dt<DT_F16>::from_f(s));
        const uint16_t zb = bf ? Dt<DT_BF16>::from_f(z) : __builtin_bit_cast(uint16_t, Dt<DT_F16>::from_f(z));
        reinterpret_cast<uint16_t*>(sp)[i] = sb;
        reinterpret_cast<uint16_t*>(zp)[i] = zb;
    }
}

// word J of a 32-code chunk from the fields f[i] of its 4 lanes (field i at bit 8*BITS*i)
template <int BITS, int J>
__device__ __forceinline__ uint32_t chunk_word(const uint32_t (&f)[4]) {
    uint32_t w = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int sh = 8 * BITS * i - 32 * J;
        if (sh > -32 && sh < 32) w |= sh >= 0 ? f[i] << sh : f[i] >> -sh;
    }
    return w;
}

// One piece: the group min/max, scale and zero (stored by the group's first lane), the
// codes, and the chunk words.  rint(v / scale) must be that of the IEEE quotient X:
// y = fma(v, inv, zero), inv = 1/scale after a Newton step, satisfies
// |y - (X + zero)| <= (|X| + zero) 2^-22 < tol = (max|v| inv + qmax + 1) 2^-21, so a y
// farther than tol from every half-integer rounds to rint(X) + zero, and (scheme 1) to
// rint(fl(X + zero)), which lies within |X + zero| 2^-24 of X + zero; a lane holding a
// code within tol of a half-integer redoes its 8 with the IEEE division.
template <int DT, int L, int BITS>
__device__ __forceinline__ void quant_piece(const QuantArgs& A, int mdt, const RawOctet<DT>& raw, int row, int k,
                                            int lane) {
    constexpr float qmax = (float)((1 << BITS) - 1);
    float v[8];
    unpack_raw<DT>(raw, v);
    const bool ok = k < A.K;
    float lo = __builtin_huge_valf(), hi = -__builtin_huge_valf();
    if (ok) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            lo = min2(lo, v[e]);
            hi = max2(hi, v[e]);
        }
    }
    group_minmax<L>(lo, hi);
    const bool paper = A.scheme == 1;
    if (paper) {
        lo = fminf(lo, 0.f);
        hi = fmaxf(hi, 0.f);
    }
    float scale = (hi - lo) / qmax;
    scale = paper ? (scale < 1e-8f ? 1.f : scale) : fmaxf(scale, 1e-8f);
    const float zero = __builtin_amdgcn_fmed3f(rintf(-lo / scale), 0.f, qmax);
    if (ok && (lane & (L - 1)) == 0)
        store_meta2(mdt, A.scales, A.zeros, (long)row * A.G + k / (8 * L), scale, zero);
    float inv = __builtin_amdgcn_rcpf(scale);
    inv = fmaf(fmaf(-scale, inv, 1.f), inv, inv);
    const float lim = 0.5f - fmaf(fmaxf(fabsf(lo), fabsf(hi)), inv, qmax + 1.f) * 0x1p-21f;
    float r[8], dmax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float y = fmaf(v[e], inv, zero);
        r[e] = rintf(y);
        dmax = fmaxf(dmax, fabsf(y - r[e]));
    }
    if (!(dmax < lim)) {
        if (paper) {
#pragma unroll
            for (int e = 0; e < 8; ++e) r[e] = rintf(v[e] / scale + zero);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) r[e] = rintf(v[e] / scale) + zero;
        }
    }
    uint32_t field = 0;                                        // code e at bit e*BITS (8*BITS <= 32)
#pragma unroll
    for (int e = 0; e < 8; ++e) field |= (uint32_t)__builtin_amdgcn_fmed3f(r[e], 0.f, qmax) << (e * BITS);
    if (!ok) field = 0;
    const uint32_t f[4] = {quad_bcast<0>(field), quad_bcast<1>(field), quad_bcast<2>(field), quad_bcast<3>(field)};
    const int j = lane & 3;
    uint32_t word = chunk_word<BITS, 0>(f);
    if (j == 1) word = chunk_word<BITS, 1>(f);
    if (j == 2) word = chunk_word<BITS, 2>(f);
    if (j == 3) word = chunk_word<BITS, 3>(f);
    const int chunk_k = k & ~31;
    if (chunk_k < A.K && j < BITS) A.packed[(long)row * A.wpr + (long)(chunk_k >> 5) * BITS + j] = word;
}

template <int DT, int L, int BITS>
__global__ void __launch_bounds__(64 * WAVES) quant_pack_fast_kernel(const QuantArgs A, int mdt, FastDiv div_tpr,
                                                                     int npieces) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * WAVES + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nw = gridDim.x * WAVES;
    const int tpr = (int)div_tpr.d;
    RawOctet<DT> buf[QUANT_DEPTH];
    // a piece past the end reads the last piece again (in bounds) and is not processed;
    // an octet past K (ragged last piece of a row) reads the row's last octet, masked
    auto issue = [&](RawOctet<DT>& b, int p) {
        p = min(p, npieces - 1);
        const int row = (int)fdiv((uint32_t)p, div_tpr);
        const int k = (p - row * tpr) * PIECE + lane * 8;
        load_raw<DT>(A.w, (long)row * A.K + min(k, A.K - 8), b);
    };
    // issued in buffer order (the scheduler must not reorder them: the first piece's
    // wait would otherwise cover every load)
#pragma unroll
    for (int d = 0; d < QUANT_DEPTH; ++d) {
        issue(buf[d], wave + d * nw);
        __builtin_amdgcn_sched_barrier(0);
    }
    // full rounds of QUANT_DEPTH pieces, then the remainder from buffers 0 .. rem-1 (no
    // branch out of the loop body, so every round waits only for its own piece)
    const int mine = wave < npieces ? (npieces - wave + nw - 1) / nw : 0;
    const int rounds = mine / QUANT_DEPTH, rem = mine - rounds * QUANT_DEPTH;
    int p = wave;
    for (int it = 0; it < rounds; ++it) {
#pragma unroll
        for (int d = 0; d < QUANT_DEPTH; ++d, p += nw) {
            const int row = (int)fdiv((uint32_t)p, div_tpr);
            quant_piece<DT, L, BITS>(A, mdt, buf[d], row, (p - row * tpr) * PIECE + lane * 8, lane);
            issue(buf[d], p + QUANT_DEPTH * nw);
        }
    }
#pragma unroll
    for (int d = 0; d < QUANT_DEPTH - 1; ++d, p += nw) {
        if (d < rem) {
            const int row = (int)fdiv((uint32_t)p, div_tpr);
            quant_piece<DT, L, BITS>(A, mdt, buf[d], row, (p - row * tpr) * PIECE + lane * 8, lane);
        }
    }
}

template <int DT, int MDT>
__global__ void __launch_bounds__(64 * WAVES) quant_pack_kernel(const QuantArgs A) {
    __shared__ uint32_t words[WAVES][2][4];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const long item = (long)blockIdx.x * WAVES + wv;
    if (item >= (long)A.N * A.G) return;
    const int n = (int)(item / A.G), g = (int)(item - (long)n * A.G);
    const int k0 = g * A.gs, k1 = min(k0 + A.gs, A.K);
    const long row = (long)n * A.K;

    float lo = __builtin_huge_valf(), hi = -__builtin_huge_valf();
    for (int k = k0 + lane; k < k1; k += 64) {
        const float v = load_f<DT>(A.w, row + k);
        lo = fminf(lo, v);
        hi = fmaxf(hi, v);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        lo = fminf(lo, __shfl_xor(lo, off, 64));
        hi = fmaxf(hi, __shfl_xor(hi, off, 64));
    }
    const float qmax = (float)((1 << A.bits) - 1);
    const bool paper = A.scheme == 1;
    if (paper) {
        lo = fminf(lo, 0.f);
        hi = fmaxf(hi, 0.f);
    }
    float scale = (hi - lo) / qmax;
    scale = paper ? (scale < 1e-8f ? 1.f : scale) : fmaxf(scale, 1e-8f);
    const float zero = fminf(fmaxf(rintf(-lo / scale), 0.f), qmax);
    if (lane == 0) {
        store_f<MDT>(A.scales, (long)n * A.G + g, scale);
        store_f<MDT>(A.zeros, (long)n * A.G + g, zero);
    }

    // chunks of the group: [k0 / 32, ceil(k1 / 32)); lane half h takes chunk c + h
    const int cb = k0 >> 5, ce = (k1 + 31) >> 5;
    const int h = lane >> 5, j = lane & 31;
    for (int c = cb; c < ce; c += 2) {
        const int cc = c + h;
        const int k = 32 * cc + j;
        uint32_t q = 0;
        if (cc < ce && k < k1) {
            const float v = load_f<DT>(A.w, row + k);
            const float r = paper ? rintf(v / scale + zero) : rintf(v / scale) + zero;
            q = (uint32_t)fminf(fmaxf(r, 0.f), qmax);
        }
        if (j < 4) words[wv][h][j] = 0u;
        __builtin_amdgcn_wave_barrier();
        const int pos = j * A.bits, wi = pos >> 5, sh = pos & 31;
        atomicOr(&words[wv][h][wi], q << sh);
        if (sh + A.bits > 32) atomicOr(&words[wv][h][wi + 1], q >> (32 - sh));
        __builtin_amdgcn_wave_barrier();
        if (cc < ce && j < A.bits) A.packed[(long)n * A.wpr + (long)cc * A.bits + j] = words[wv][h][j];
        __builtin_amdgcn_wave_barrier();
    }
}

template <int DT, int BITS>
const void* fast_kernel_for_gs(int gs) {
    switch (gs) {
        case 32: return reinterpret_cast<const void*>(&quant_pack_fast_kernel<DT, 4, BITS>);
        case 64: return reinterpret_cast<const void*>(&quant_pack_fast_kernel<DT, 8, BITS>);
        case 128: return reinterpret_cast<const void*>(&quant_pack_fast_kernel<DT, 16, BITS>);
        case 256: return reinterpret_cast<const void*>(&quant_pack_fast_kernel<DT, 32, BITS>);
        default: return reinterpret_cast<const void*>(&quant_pack_fast_kernel<DT, 64, BITS>);
    }
}

template <int DT>
const void* fast_kernel_for(int gs, int bits) {
    return bits == 2 ? fast_kernel_for_gs<DT, 2>(gs) : bits == 3 ? fast_kernel_for_gs<DT, 3>(gs)
                                                                 : fast_kernel_for_gs<DT, 4>(gs);
}

template <int DT>
const void* kernel_for_meta(int mdt) {
    if (mdt == DT_BF16) return reinterpret_cast<const void*>(&quant_pack_kernel<DT, DT_BF16>);
    if (mdt == DT_F32) return reinterpret_cast<const void*>(&quant_pack_kernel<DT, DT_F32>);
    return reinterpret_cast<const void*>(&quant_pack_kernel<DT, DT_F16>);
}

}  // namespace

bool quant_fast_supported(const QuantArgs& A, uintptr_t w_addr) {
    const long pieces = (long)A.N * ((A.K + PIECE - 1) / PIECE);
    return A.gs >= 32 && A.gs <= PIECE && PIECE % A.gs == 0 && A.K % 8 == 0 && w_addr % 16 == 0 &&
           pieces < (1l << 30);
}

hipError_t launch_quant_pack(const QuantArgs& A, int dt, int mdt, int cus, hipStream_t stream) {
    if (quant_fast_supported(A, reinterpret_cast<uintptr_t>(A.w))) {
        const int tpr = (A.K + PIECE - 1) / PIECE;
        int npieces = A.N * tpr;
        FastDiv div_tpr = make_fastdiv((uint32_t)tpr);
        const void* f = dt == DT_BF16 ? fast_kernel_for<DT_BF16>(A.gs, A.bits)
                      : dt == DT_F32  ? fast_kernel_for<DT_F32>(A.gs, A.bits)
                                      : fast_kernel_for<DT_F16>(A.gs, A.bits);
        const int wgs = std::max(1, std::min((npieces + WAVES - 1) / WAVES, cus * CBK_QUANT_WGS_PER_CU));
        void* args[] = {const_cast<QuantArgs*>(&A), &mdt, &div_tpr, &npieces};
        return launch(f, dim3((unsigned)wgs), dim3(64 * WAVES), args, 0, stream);
    }
    const void* f = dt == DT_BF16 ? kernel_for_meta<DT_BF16>(mdt)
                  : dt == DT_F32  ? kernel_for_meta<DT_F32>(mdt)
                                  : kernel_for_meta<DT_F16>(mdt);
    const long items = (long)A.N * A.G;
    void* args[] = {const_cast<QuantArgs*>(&A)};
    return launch(f, dim3((unsigned)((items + WAVES - 1) / WAVES)), dim3(64 * WAVES), args, 0, stream);
}

}  // namespace cbk
