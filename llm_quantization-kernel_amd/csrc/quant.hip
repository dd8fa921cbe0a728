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
//
// One wave per (row, group): lanes stride the group for the min/max (reduced across the
// wave by xor shuffles), then quantize one code each, 32-code chunks two at a time, and
// OR the codes into the chunk's words in a per-wave LDS slot (a code that straddles two
// words ORs into both), which lanes 0 .. bits-1 store.
#include "cbk_device.hpp"
#include "cbk_kernels.hpp"

namespace cbk {
namespace {

constexpr int WAVES = 4;

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
    const float scale = fmaxf((hi - lo) / qmax, 1e-8f);
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
            q = (uint32_t)fminf(fmaxf(rintf(v / scale) + zero, 0.f), qmax);
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

template <int DT>
const void* kernel_for_meta(int mdt) {
    if (mdt == DT_BF16) return reinterpret_cast<const void*>(&quant_pack_kernel<DT, DT_BF16>);
    if (mdt == DT_F32) return reinterpret_cast<const void*>(&quant_pack_kernel<DT, DT_F32>);
    return reinterpret_cast<const void*>(&quant_pack_kernel<DT, DT_F16>);
}

}  // namespace

hipError_t launch_quant_pack(const QuantArgs& A, int dt, int mdt, hipStream_t stream) {
    const void* f = dt == DT_BF16 ? kernel_for_meta<DT_BF16>(mdt)
                  : dt == DT_F32  ? kernel_for_meta<DT_F32>(mdt)
                                  : kernel_for_meta<DT_F16>(mdt);
    const long items = (long)A.N * A.G;
    void* args[] = {const_cast<QuantArgs*>(&A)};
    return launch(f, dim3((unsigned)((items + WAVES - 1) / WAVES)), dim3(64 * WAVES), args, 0, stream);
}

}  // namespace cbk
