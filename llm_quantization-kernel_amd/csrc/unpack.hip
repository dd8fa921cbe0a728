// unpack.hip -- codes[N, K] of a packed matrix through the MFMA kernels' decode.
//
// Test hook for the bit-exact code check (the reference's CPU equivalent is
// Kernel/crispybits_kernels/reference.py:58-67).  Each thread decodes one 32-code
// chunk with cbk_decode.hpp -- the same packed-fp16 path the GEMV streams through
// its matrix cores -- and scatters the halves back to code order with kappa, so a
// wrong shift, mask or straddle join in the decode shows up as a wrong code.
#include "cbk_decode.hpp"
#include "cbk_kernels.hpp"

namespace cbk {
namespace {

template <int BITS>
__global__ void __launch_bounds__(256) unpack_kernel(const uint32_t* __restrict__ packed, int N, int K, int C,
                                                      int32_t* __restrict__ codes) {
    const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long)N * C) return;
    const int n = (int)(t / C), c = (int)(t - (long)n * C);
    const uint32_t* p = packed + (long)n * C * BITS + (long)c * BITS;
    uint32_t w[BITS];
#pragma unroll
    for (int i = 0; i < BITS; ++i) w[i] = p[i];
    uint32_t h[16];
    Decode<BITS>::run(w, h, MAGIC2);
#pragma unroll
    for (int q = 0; q < 32; ++q) {
        const int k = c * 32 + Decode<BITS>::kappa(q);
        const uint32_t half = (q & 1) ? (h[q >> 1] >> 16) : (h[q >> 1] & 0xFFFFu);
        // half = fp16 bits of 1024 + 2^e * code; anything else reads back as -1
        if (k < K) codes[(long)n * K + k] = code_of_half<BITS>(half, q);
    }
}

}  // namespace

hipError_t launch_unpack(const uint32_t* packed, int N, int K, int bits, int32_t* codes, hipStream_t stream) {
    const int C = (K + 31) / 32;
    const long total = (long)N * C;
    const dim3 grid((unsigned)((total + 255) / 256)), block(256);
    const void* f = bits == 2 ? reinterpret_cast<const void*>(&unpack_kernel<2>)
                  : bits == 3 ? reinterpret_cast<const void*>(&unpack_kernel<3>)
                              : reinterpret_cast<const void*>(&unpack_kernel<4>);
    void* args[] = {&packed, &N, &K, const_cast<int*>(&C), &codes};
    return launch(f, grid, block, args, 0, stream);
}

}  // namespace cbk
