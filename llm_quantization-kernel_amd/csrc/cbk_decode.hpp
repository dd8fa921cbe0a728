// cbk_decode.hpp -- packed-fp16 decode of one 32-code chunk for the MFMA kernels.
//
// A chunk (BITS int32 words holding codes 0..31 LSB-first, Kernel/crispybits_kernels/
// reference.py:37-55) becomes 16 packed fp16 pairs.  OR-ing a field that sits at
// bit offset e (0..5) of a 16-bit half into the bit pattern of 1024.0 (0x6400,
// ulp 1) gives the exact fp16 value 1024 + 2^e q = 2^e (2^(10-e) + q), so each half
// keeps its field where it lies and most fields need no shift.  The activation
// that meets half slot p is staged as x * 2^-e(p) in fp16 (a power-of-two scale: exact
// while the product stays a normal fp16, |x| 2^-e >= 2^-14; below that it rounds to a
// subnormal and keeps fewer bits), so the MFMA sums x * (B(p) + q) with the slot offset
// B(p) = 2^(10 - e(p)); the kernels remove sum_p x * B(p) together with the zero point.
//
// Half slot p (pair p >> 1, high half when p & 1) holds code kappa(p) at offset
// expo(p).  MFMA operand m (8 halves) is pairs 4m .. 4m+3.  Each output pair is
// one v_and_or_b32 (mask in an SGPR, 0x64006400 in a VGPR -- gfx9 VOP3 takes
// neither a literal nor two SGPRs); per 32 codes: W4 20 VALU ops, W2 20, W3 26.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cbk {

constexpr uint32_t MAGIC2 = 0x64006400u;   // (1024.0h, 1024.0h)

// a BITS-wide field at offset a of the low half and b of the high half
__host__ __device__ constexpr uint32_t field2(int bits, int a, int b) {
    return (((1u << bits) - 1u) << a) | ((((1u << bits) - 1u) << b) << 16);
}

// 0x64006400 held in a VGPR (hoistable; the asm only keeps the compiler from
// folding it back into a literal operand).
__device__ __forceinline__ uint32_t magic_vreg() {
    uint32_t r;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(r));
    return r;
}

// Slot offset B(p) = 2^(10 - e) of a field decoded at offset e.
__host__ __device__ constexpr float slot_offset(int e) { return (float)(1024 >> e); }

template <int BITS> struct Decode;

template <> struct Decode<4> {
    // word t = codes 8t..8t+7 (nibble n at bit 4n); pair 4t+s = (nibble s, nibble s+4),
    // nibbles 0/4 at offset 0 of w, 1/5 at offset 4 of w, 2/6 and 3/7 likewise of w >> 8
    static constexpr int kappa(int p) { return 8 * (p >> 3) + ((p >> 1) & 3) + 4 * (p & 1); }
    static constexpr int expo(int p) { return ((p >> 1) & 1) ? 4 : 0; }
    static __device__ __forceinline__ void run(const uint32_t (&w)[4], uint32_t (&h)[16], uint32_t g) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t v = w[t] >> 8;
            h[4 * t + 0] = (w[t] & field2(4, 0, 0)) | g;
            h[4 * t + 1] = (w[t] & field2(4, 4, 4)) | g;
            h[4 * t + 2] = (v & field2(4, 0, 0)) | g;
            h[4 * t + 3] = (v & field2(4, 4, 4)) | g;
        }
    }
};

template <> struct Decode<2> {
    // word t = codes 16t..16t+15 (field f at bit 2f); pair 8t+s = (field s, field s+8),
    // taken at offset 2*(s % 3) of w >> (6 * (s / 3))
    static constexpr int kappa(int p) { return 16 * (p >> 4) + ((p >> 1) & 7) + 8 * (p & 1); }
    static constexpr int expo(int p) { return 2 * (((p >> 1) & 7) % 3); }
    static __device__ __forceinline__ void run(const uint32_t (&w)[2], uint32_t (&h)[16], uint32_t g) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint32_t a = w[t], b = a >> 6, c = a >> 12;
            h[8 * t + 0] = (a & field2(2, 0, 0)) | g;
            h[8 * t + 1] = (a & field2(2, 2, 2)) | g;
            h[8 * t + 2] = (a & field2(2, 4, 4)) | g;
            h[8 * t + 3] = (b & field2(2, 0, 0)) | g;
            h[8 * t + 4] = (b & field2(2, 2, 2)) | g;
            h[8 * t + 5] = (b & field2(2, 4, 4)) | g;
            h[8 * t + 6] = (c & field2(2, 0, 0)) | g;
            h[8 * t + 7] = (c & field2(2, 2, 2)) | g;
        }
    }
};

template <> struct Decode<3> {
    // code c at chunk bit 3c: w0 holds codes 0-9 (10 straddles into w1), w1 codes
    // 11-20 at bit 1 + 3i (21 straddles into w2), w2 codes 22-31 at bit 2 + 3i.
    // Pairs 0-13 come from w_i, w_i >> 6 and w_i >> 12 at the offsets below; pairs
    // 14 and 15 join (4, 10) and (5, 21): the straddling codes are aligned with
    // alignbit, merged with one bitfield insert and placed in the high half by perm.
    static constexpr int kappa(int p) {
        constexpr int lo[16] = {0, 1, 2, 3, 11, 12, 13, 14, 15, 22, 23, 24, 25, 26, 4, 5};
        constexpr int hi[16] = {6, 7, 8, 9, 16, 17, 18, 19, 20, 27, 28, 29, 30, 31, 10, 21};
        return (p & 1) ? hi[p >> 1] : lo[p >> 1];
    }
    static constexpr int expo(int p) {
        constexpr int lo[16] = {0, 3, 0, 3, 1, 4, 1, 4, 1, 2, 5, 2, 5, 2, 0, 3};
        constexpr int hi[16] = {2, 5, 2, 5, 0, 3, 0, 3, 0, 1, 4, 1, 4, 1, 0, 3};
        return (p & 1) ? hi[p >> 1] : lo[p >> 1];
    }
    static __device__ __forceinline__ void run(const uint32_t (&w)[3], uint32_t (&h)[16], uint32_t g) {
        const uint32_t a0 = w[0], b0 = w[0] >> 6, c0 = w[0] >> 12;
        const uint32_t a1 = w[1], b1 = w[1] >> 6, c1 = w[1] >> 12;
        const uint32_t a2 = w[2], b2 = w[2] >> 6, c2 = w[2] >> 12;
        h[0] = (a0 & field2(3, 0, 2)) | g;    // codes  0,  6
        h[1] = (a0 & field2(3, 3, 5)) | g;    //        1,  7
        h[2] = (b0 & field2(3, 0, 2)) | g;    //        2,  8
        h[3] = (b0 & field2(3, 3, 5)) | g;    //        3,  9
        h[4] = (a1 & field2(3, 1, 0)) | g;    //       11, 16
        h[5] = (a1 & field2(3, 4, 3)) | g;    //       12, 17
        h[6] = (b1 & field2(3, 1, 0)) | g;    //       13, 18
        h[7] = (b1 & field2(3, 4, 3)) | g;    //       14, 19
        h[8] = (c1 & field2(3, 1, 0)) | g;    //       15, 20
        h[9] = (a2 & field2(3, 2, 1)) | g;    //       22, 27
        h[10] = (a2 & field2(3, 5, 4)) | g;   //       23, 28
        h[11] = (b2 & field2(3, 2, 1)) | g;   //       24, 29
        h[12] = (b2 & field2(3, 5, 4)) | g;   //       25, 30
        h[13] = (c2 & field2(3, 2, 1)) | g;   //       26, 31
        const uint32_t t10 = __builtin_amdgcn_alignbit(w[1], w[0], 30);   // code 10 at bit 0
        const uint32_t t21 = __builtin_amdgcn_alignbit(w[2], w[1], 28);   // code 20 at 0, 21 at 3
        const uint32_t tt = (t10 & 7u) | (t21 & ~7u);                     // code 10 at 0, 21 at 3
        const uint32_t q = __builtin_amdgcn_perm(tt, c0, 0x05040100u);    // lo: c0 (codes 4, 5), hi: tt
        h[14] = (q & field2(3, 0, 0)) | g;    //        4, 10
        h[15] = (q & field2(3, 3, 3)) | g;    //        5, 21
    }
};

// Code of half slot p from its decoded fp16 bits, or -1 if the bits are not
// exactly 1024 + 2^e q with q < 2^BITS (the unpack test hook's check).
template <int BITS>
__device__ __forceinline__ int32_t code_of_half(uint32_t half, int p) {
    const int e = Decode<BITS>::expo(p);
    const uint32_t d = half - 0x6400u;
    if (d >= ((1u << BITS) << e) || (d & ((1u << e) - 1u))) return -1;
    return (int32_t)(d >> e);
}

}  // namespace cbk
