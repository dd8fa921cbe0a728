// cbk_device.hpp -- device helpers shared by the gfx950 packed-linear kernels.
//
// Covers the reference's device helpers (Kernel/csrc/common.cuh:10-70 and
// bitpack.cuh:10-46) re-designed for CDNA4: storage-type conversion, epilogue
// activations, the virtual-row map of the fused modes, RoPE un-permutation, and
// scalar code extraction for the VALU kernels.  The packed-fp16 MFMA decode lives
// in cbk_decode.hpp.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cbk {

enum { DT_F16 = 0, DT_BF16 = 1, DT_F32 = 2 };
enum { ACT_NONE = 0, ACT_RELU = 1, ACT_SILU = 2 };
enum { MODE_GEMV = 0, MODE_QKV = 1, MODE_GATEUP = 2 };

// ---------------------------------------------------------------- storage types
template <int DT> struct Dt;

template <> struct Dt<DT_F16> {
    using S = _Float16;
    static __device__ __forceinline__ float to_f(S v) { return (float)v; }
    static __device__ __forceinline__ S from_f(float f) { return (S)f; }      // v_cvt_f16_f32, RNE
};

template <> struct Dt<DT_BF16> {
    using S = uint16_t;
    static __device__ __forceinline__ float to_f(S v) { return __uint_as_float((uint32_t)v << 16); }
    static __device__ __forceinline__ S from_f(float f) {                     // RNE, quiet NaN
        uint32_t u = __float_as_uint(f);
        if ((u & 0x7fffffffu) > 0x7f800000u) return (S)((u >> 16) | 0x40u);
        u += 0x7fffu + ((u >> 16) & 1u);
        return (S)(u >> 16);
    }
};

template <> struct Dt<DT_F32> {
    using S = float;
    static __device__ __forceinline__ float to_f(S v) { return v; }
    static __device__ __forceinline__ S from_f(float f) { return f; }
};

template <int DT>
__device__ __forceinline__ float load_f(const void* p, long i) {
    return Dt<DT>::to_f(reinterpret_cast<const typename Dt<DT>::S*>(p)[i]);
}
template <int DT>
__device__ __forceinline__ void store_f(void* p, long i, float v) {
    reinterpret_cast<typename Dt<DT>::S*>(p)[i] = Dt<DT>::from_f(v);
}

// ---------------------------------------------------------------- epilogue math
// SiLU uses the device exp (v_exp_f32 path); checked against float64 SiLU in the tests.
__device__ __forceinline__ float silu(float v) { return v / (1.0f + __expf(-v)); }

__device__ __forceinline__ float apply_act(float v, int act) {
    if (act == ACT_RELU) return v > 0.f ? v : 0.f;
    if (act == ACT_SILU) return silu(v);
    return v;
}

// Stored (pair-interleaved) row r of a head -> original row (the inverse of
// ops.rope_row_order; same map as common.cuh:66-70).
__device__ __forceinline__ int rope_unperm(int r, int hd) {
    if (hd <= 0) return r;
    const int head = r / hd, p = r - head * hd;
    return head * hd + ((p & 1) ? (p >> 1) + (hd >> 1) : (p >> 1));
}

// ---------------------------------------------------------------- invariant division
// n / d for 32-bit unsigned n and a divisor fixed per launch, as one multiply-high
// and three shifts/adds (Granlund & Montgomery, "Division by Invariant Integers
// using Multiplication", PLDI 1994, fig. 4.1): with l = ceil(log2 d),
// m = floor(2^32 (2^l - d) / d) + 1, t = mulhi(m, n), q = (t + ((n - t) >> 1)) >> (l - 1)
// (shifts 0 and 0 for d = 1).  Job and unit indices are divided this way instead
// of by the generic 32/64-bit division sequences, which cost hundreds of scalar
// instructions per wave.
struct FastDiv {
    uint32_t m;
    uint32_t s1, s2;
    uint32_t d;
};

__host__ inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f;
    uint32_t l = 0;
    while (l < 32 && (1ull << l) < d) ++l;
    f.m = (uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1);
    f.s1 = l < 1 ? l : 1;
    f.s2 = l > 1 ? l - 1 : 0;
    f.d = d;
    return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
    const uint32_t t = __umulhi(n, f.m);
    return (t + ((n - t) >> f.s1)) >> f.s2;
}

// ---------------------------------------------------------------- decode-call arguments
struct Proj {
    const uint32_t* w;   // packed [n, wpr]
    const void* s;       // scales [n, G]
    const void* z;       // zeros  [n, G]
    const void* b;       // bias [n] or nullptr
    void* out;           // [M, n]
    int n;               // rows
    int bits;            // 2 / 3 / 4
    int wpr;             // words per row = C * bits
    int pad_;
};

struct GemvArgs {
    Proj p[3];
    const void* x;         // [M, K]
    float* partial;        // [P, M, V] fp32 when P > 1
    const float* rope_cos; // [M, head_dim] or nullptr
    const float* rope_sin;
    int M, K, V;           // batch rows, in_features, virtual rows
    int C, G, gs;          // 32-code chunks per row, groups per row, group size
    int P, act;            // K splits, activation (GEMV mode)
    int head_dim, perm_hd;
    int ntiles, mtiles, jobs;
    int nw;                // waves per workgroup (MFMA kernel)
    int units;             // 128-code units per row (MFMA kernel)
    int xs_bytes;          // per-wave LDS: bytes of the staged activations (unit sums follow)
    int meta_off;          // per-wave LDS: offset of the (scale, zero) pairs
    int ring_off;          // per-wave LDS: offset of the weight ring
    int wave_bytes;        // per-wave LDS region size
    int red_off;           // workgroup LDS: offset of the cross-wave reduction area
    int lds_bytes;         // dynamic LDS bytes per workgroup
    int ring;              // weight-ring slots per wave (MFMA kernel), 1 .. Ring<>::RMAX
    // batch-1 MFMA layout: workgroup-shared staging areas (offsets into the LDS)
    int sum_off;           // unit sums [unit][2] fp32
    int tab_off;           // masked scales [unit][tile row][kq] fp32
    int raw_off;           // raw (scale, zero) row spans [tensor][tile row][piece] x 16 B
    int raw_np;            // 16-byte pieces per row span
    int pad_;
    FastDiv divP, divT, divW, divG;   // by P, ntiles, nw and gs / 128 (MFMA kernel)
    FastDiv divNP;                    // by raw_np
    // batch-1 streaming kernel (gemv_stream.hip)
    int st_ks;             // K slices per job (waves per row group)
    int st_rw;             // row groups per workgroup (one wave's rows each)
    int st_xvec;           // x is 16-byte aligned with K % 8 == 0 (vector activation loads)
    int pad2_;
    FastDiv divRW, divGS;             // by st_rw and gs / 32
    // streaming kernels with P > 1: one arrival counter per row block (zero between
    // calls); the splits combine inside the dispatch.  nullptr: a reduce launch combines.
    uint32_t* split_cnt;
};

// Per-wave weight ring of the MFMA decode kernel (host and device).  A stage is
// S consecutive 128-code units of the 16 rows of a job tile, copied HBM -> LDS
// with direct-to-LDS dwordx4 loads: 16-byte piece p of a stage lands at byte 16p,
// row r of the tile owns pieces [r*PITCH, r*PITCH + PPR) and one pad piece that
// staggers the rows across LDS banks.  Up to RMAX stages are in flight per wave
// (RMAX * NDMA stays well inside the 6-bit vmcnt counter).
template <int BITS> struct Ring {
    static constexpr int S = 4;                       // units per stage
    static constexpr int RMAX = 8;                    // ring slots per wave, at most
    static constexpr int RMAX1 = 4;                   // ... at batch 1 (units as MFMA rows)
    static constexpr int PPR = S * BITS;              // 16-byte pieces of one row per stage
    static constexpr int PITCH = PPR + 1;             // LDS row pitch in pieces
    static constexpr int NDMA = (16 * PITCH + 63) / 64;   // dwordx4 LDS-DMA instructions per stage
    static constexpr int SLOT = NDMA * 64 * 16;       // LDS bytes of one stage
};

__host__ __device__ constexpr int ring_slot_bytes(int bits) {
    return bits == 2 ? Ring<2>::SLOT : (bits == 3 ? Ring<3>::SLOT : Ring<4>::SLOT);
}

// Projection field select between values of the kernel-argument struct.  The
// empty asm pins each loaded field as an SGPR value, so LLVM cannot fold the
// choice into a load from a chosen field address -- an address select into the
// kernarg struct would force a copy of the whole struct to scratch.
template <typename T>
__device__ __forceinline__ T kernarg_value(T v) {
    asm("" : "+s"(v));
    return v;
}
#define CBK_SEL(A, proj, field)                                                                      \
    ((proj) == 0 ? kernarg_value((A).p[0].field)                                                     \
                 : ((proj) == 1 ? kernarg_value((A).p[1].field) : kernarg_value((A).p[2].field)))

// Virtual row v -> (projection, local row): QKV concatenates [q; k; v], gate-up
// interleaves gate row n -> 2n and up row n -> 2n+1 (packed_gemv.cu:33-42).
template <int MODE>
__device__ __forceinline__ void vmap(const GemvArgs& A, int v, int& proj, int& r) {
    if constexpr (MODE == MODE_GATEUP) {
        proj = v & 1; r = v >> 1;
    } else if constexpr (MODE == MODE_QKV) {
        const int n0 = A.p[0].n, n1 = A.p[1].n;
        if (v < n0) { proj = 0; r = v; }
        else if (v < n0 + n1) { proj = 1; r = v - n0; }
        else { proj = 2; r = v - n0 - n1; }
    } else {
        proj = 0; r = v;
    }
}

// Final value of virtual row v for batch row b.  `partner` is the fp32 sum of row
// v ^ 1 (the up row of a gate row; the RoPE partner of a Q/K row), before bias.
template <int DT, int MODE>
__device__ __forceinline__ void epilogue(const GemvArgs& A, int b, int v, float mine, float partner) {
    int proj, r;
    vmap<MODE>(A, v, proj, r);
    if constexpr (MODE == MODE_GEMV) {
        const float bias = A.p[0].b ? load_f<DT>(A.p[0].b, r) : 0.f;
        store_f<DT>(A.p[0].out, (long)b * A.p[0].n + r, apply_act(mine + bias, A.act));
    } else if constexpr (MODE == MODE_GATEUP) {
        if (proj != 0) return;
        store_f<DT>(A.p[0].out, (long)b * A.p[0].n + r, silu(mine) * partner);
    } else {
        const void* bias = CBK_SEL(A, proj, b);
        void* out = CBK_SEL(A, proj, out);
        const int n = CBK_SEL(A, proj, n);
        float y = mine + (bias ? load_f<DT>(bias, r) : 0.f);
        const int hd = proj < 2 ? A.perm_hd : 0;
        const int orig = rope_unperm(r, hd);
        if (A.rope_cos != nullptr && proj < 2) {
            const float yp = partner + (bias ? load_f<DT>(bias, r ^ 1) : 0.f);
            const int d = orig % A.head_dim;
            const float c = A.rope_cos[(long)b * A.head_dim + d];
            const float s = A.rope_sin[(long)b * A.head_dim + d];
            y = (d < (A.head_dim >> 1)) ? (y * c - yp * s) : (y * c + yp * s);
        }
        store_f<DT>(out, (long)b * n + orig, y);
    }
}

// ---------------------------------------------------------------- split-K combine in the dispatch
// The P workgroups of a row block (one per K split, on any XCD) combine their fp32
// partials without the reduce launch that cb_reduce_kernel (packed_gemv.cu:166-180)
// stands for.  Partials are written and read with agent-scope accesses (stores and
// loads coherent across the XCDs' L2s, `sc1`), so no L2 write-back or invalidation is
// needed: a release / acquire pair at agent scope would write back and invalidate the
// whole L2 of the XCD per workgroup, which serialises (a K-split batch-1 GEMV went from
// 7.6 to 38 us that way).  Each wave waits until its partial stores have completed,
// the workgroup meets at a barrier, and one thread counts the workgroup in; the
// workgroup that arrives last (old count P - 1) sets the counter back to zero for the
// next call and adds the P partials in split order 0 .. P - 1 -- gemv_reduce_kernel's
// order, so both paths give the same bits.  No workgroup waits for another.
__device__ __forceinline__ void partial_put(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float partial_get(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// After the workgroup's partial_put calls: returns, in every thread, whether this
// workgroup combines row block `blk`.  `flag` is a word of LDS that no thread reads or
// writes across this call.
__device__ __forceinline__ bool split_arrive(const GemvArgs& A, int blk, int* flag) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");      // this wave's partials are stored
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t* c = A.split_cnt + blk;
        const uint32_t old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = old + 1u == (uint32_t)A.P;
        if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = last ? 1 : 0;
    }
    __syncthreads();
    return *flag != 0;
}

// Sum of split partials p = 0 .. P - 1 of (batch row b, virtual row v), in that order.
__device__ __forceinline__ float split_sum(const GemvArgs& A, int b, int v) {
    float s = 0.f;
    for (int p = 0; p < A.P; ++p) s += partial_get(A.partial + ((long)p * A.M + b) * A.V + v);
    return s;
}

// The combining workgroup's epilogue: rows [vbase, vbase + RB) of every batch row,
// `nthr` threads, outputs of dtype DT.
template <int DT, int MODE>
__device__ __forceinline__ void split_epilogue(const GemvArgs& A, int vbase, int RB, int nthr) {
    for (int t = threadIdx.x; t < A.M * RB; t += nthr) {
        const int b = t / RB, v = vbase + (t - b * RB);
        if (v < A.V) {
            const bool paired = MODE == MODE_GATEUP || (MODE == MODE_QKV && A.rope_cos != nullptr);
            const float partner = paired && (v ^ 1) < A.V ? split_sum(A, b, v ^ 1) : 0.f;
            epilogue<DT, MODE>(A, b, v, split_sum(A, b, v), partner);
        }
    }
}

// ---------------------------------------------------------------- scalar code access
// Code j (0..31) of a chunk held in BITS registers (straddling codes of W3 are
// joined with a 64-bit funnel shift).
template <int BITS>
__device__ __forceinline__ uint32_t chunk_code(const uint32_t (&w)[BITS], int j) {
    const int pos = j * BITS, wi = pos >> 5, off = pos & 31;
    uint32_t v = w[wi] >> off;
    if (off + BITS > 32) v |= w[wi + 1] << (32 - off);
    return v & ((1u << BITS) - 1u);
}

// Random-access code k of one packed row (bitpack.cuh:10-18 semantics).
__device__ __forceinline__ uint32_t row_code(const uint32_t* row, long k, int bits) {
    const long pos = k * bits;
    const long wi = pos >> 5;
    const int off = (int)(pos & 31);
    uint32_t v = row[wi] >> off;
    if (off + bits > 32) v |= row[wi + 1] << (32 - off);
    return v & ((1u << bits) - 1u);
}

}  // namespace cbk
