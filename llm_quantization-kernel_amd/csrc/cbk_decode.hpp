// cbk_decode.hpp -- packed-fp16 decode of one 32-code chunk for the MFMA kernels.
//
// A chunk (BITS int32 words holding codes 0..31 LSB-first, Kernel/crispybits_kernels/
// reference.py:37-55) is turned into 16 packed fp16 pairs whose halves are exactly
// 1024 + q: OR-ing a 3/4-bit field into the mantissa of 0x6400 (= 1024.0 in fp16,
// whose ulp is 1) is an exact int -> fp16 conversion of two codes per VALU op.
// The halves come out in a BITS-specific order, kappa(p) = code index held by half
// slot p (pair p/2, lo when p is even); the activation is staged in the same order
// so the dot product is unchanged.  MFMA operand m (8 halves) is pairs 4m..4m+3.
//
// Per 32 codes: W4 28 VALU ops, W2 30, W3 38 (W3 aligns its 10-code runs to
// 16-bit lanes with one bitfield insert per word and joins the two straddling
// codes, 10 and 21, with alignbit).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cbk {

constexpr uint32_t MAGIC2 = 0x64006400u;   // (1024.0h, 1024.0h)

template <int BITS> struct Decode;

template <> struct Decode<4> {
    // word t holds codes 8t..8t+7 as nibbles; pair 4t+s = (nibble s, nibble s+4)
    static constexpr int kappa(int p) { return 8 * (p >> 3) + ((p >> 1) & 3) + 4 * (p & 1); }
    static __device__ __forceinline__ void run(const uint32_t (&w)[4], uint32_t (&h)[16]) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int s = 0; s < 4; ++s) h[4 * t + s] = ((w[t] >> (4 * s)) & 0x000F000Fu) | MAGIC2;
        }
    }
};

template <> struct Decode<2> {
    // word t holds codes 16t..16t+15; pair 8t+s = (field s, field s+8)
    static constexpr int kappa(int p) { return 16 * (p >> 4) + ((p >> 1) & 7) + 8 * (p & 1); }
    static __device__ __forceinline__ void run(const uint32_t (&w)[2], uint32_t (&h)[16]) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int s = 0; s < 8; ++s) h[8 * t + s] = ((w[t] >> (2 * s)) & 0x00030003u) | MAGIC2;
        }
    }
};

template <> struct Decode<3> {
    // pairs 0-4: (k, k+5); 5-9: (11+k, 16+k); 10-14: (22+k, 27+k); 15: (10, 21)
    static constexpr int kappa(int p) {
        return (p >> 1) == 15 ? ((p & 1) ? 21 : 10)
             : 11 * ((p >> 1) / 5) + ((p >> 1) % 5) + 5 * (p & 1);
    }
    static __device__ __forceinline__ void run(const uint32_t (&w)[3], uint32_t (&h)[16]) {
        // lo 16 bits: codes (base + k) at bit 3k; hi 16 bits: codes (base + 5 + k) at bit 16 + 3k
        const uint32_t v0 = (w[0] & 0x0000FFFFu) | ((w[0] << 1) & 0xFFFF0000u);
        const uint32_t v1 = ((w[1] >> 1) & 0x0000FFFFu) | (w[1] & 0xFFFF0000u);
        const uint32_t v2 = ((w[2] >> 2) & 0x0000FFFFu) | ((w[2] >> 1) & 0xFFFF0000u);
#pragma unroll
        for (int k = 0; k < 5; ++k) {
            h[k] = ((v0 >> (3 * k)) & 0x00070007u) | MAGIC2;
            h[5 + k] = ((v1 >> (3 * k)) & 0x00070007u) | MAGIC2;
            h[10 + k] = ((v2 >> (3 * k)) & 0x00070007u) | MAGIC2;
        }
        const uint32_t c10 = __builtin_amdgcn_alignbit(w[1], w[0], 30);   // w0[31:30] | w1[0] << 2
        const uint32_t c21 = __builtin_amdgcn_alignbit(w[2], w[1], 31);   // w1[31]    | w2[1:0] << 1
        h[15] = (__builtin_amdgcn_perm(c21, c10, 0x05040100u) & 0x00070007u) | MAGIC2;
    }
};

}  // namespace cbk
