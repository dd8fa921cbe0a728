// cbk_device.hpp -- device helpers shared by the gfx950 packed-linear kernels.
//
// Covers the reference's device helpers (Kernel/csrc/common.cuh:10-70 and
// bitpack.cuh:10-46) re-designed for CDNA4: storage-type conversion, epilogue
// activations, the virtual-row map of the fused modes, RoPE un-permutation, the
// row-pair finish stage every decode kernel ends with, the in-dispatch split-K
// combine, and scalar code extraction.  The packed-fp16 in-place decode lives in
// cbk_decode.hpp.
#pragma once

#include <hip/hip_runtime.h>
#include <type_traits>
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
// A decode call has up to three projections (plain GEMV: one; gate-up: gate and up;
// QKV: q, k and v).  Each has a weight side, which the K loop of every kernel streams,
// and an output side, which only the finish stage writes; the two are kept apart so
// that the finish stage (finish) sees nothing of the weights and the K loops
// nothing of the outputs.
struct Src {
    const uint32_t* w;   // packed codes [n, wpr]
    const void* s;       // scales [n, G], x's dtype
    const void* z;       // zeros  [n, G]
    int n;               // rows
    int wpr;             // 32-bit words per row = C * bits
};

struct Dst {
    void* y;             // outputs [M, ld]
    const void* bias;    // [ld] or nullptr
    int ld;              // row stride of y (the projection's rows)
    int pad_;
};

// The fields every decode kernel reads at its start come first and densely, with no
// padding and nothing a kernel leaves unused between them: the compiler merges
// neighbouring kernel-argument loads into wide scalar loads, and an unused word inside
// one lets it recycle that register for a later load, which then has to wait for the
// first -- a serialised memory round trip at the start of every launch.
struct GemvArgs {
    Src src[3];
    const void* x;         // [M, K]
    float* partial;        // [P, M, V] fp32 when P > 1
    // K-split calls combining in the dispatch: one arrival counter per row block (zero
    // between calls).  nullptr: a combine launch adds the partials.
    uint32_t* split_cnt;
    int M, K, V, C;        // batch rows, in_features, virtual rows, 32-code chunks per row
    int G, gs, P, act;     // groups per row, group size, K splits, activation (GEMV mode)
    int st_ks;             // streaming kernels: K slices per job (waves per row group)
    int st_rw;             // streaming kernels: row groups per workgroup
    int st_xvec;           // x is 16-byte aligned with K % 8 == 0 (vector activation loads)
    int ntiles;            // fp32 matrix-core kernel: 16-row tiles
    FastDiv divP, divRW, divGS, divG, divT;   // by P, st_rw, gs / 32, gs / 128, ntiles
    Dst dst[3];
    const float* rope_cos; // [M, head_dim] or nullptr
    const float* rope_sin;
    int head_dim, perm_hd;
    FastDiv divHD;         // by perm_hd (1 when the Q/K rows are not pair-interleaved)
    int mtiles, jobs;      // fp32 matrix-core kernel: 16-row batch tiles, jobs
    int bits[3];           // code width of each projection
    int pad_;
};

// ---------------------------------------------------------------- projection views
// A projection's fields as values.  Each candidate field is pinned as an SGPR value
// first (the empty asm), so LLVM selects between values rather than between addresses
// inside the kernel-argument block -- an address select there would copy the whole
// block to scratch.  The select is bit masks, not a conditional: written as `?:` LLVM
// sinks each pinned value into its own arm and the wave branches (a chain of scalar
// branches in front of the first weight load of every fused-QKV wave).  `p` may differ
// between lanes (the select is then per lane).
template <typename T>
__device__ __forceinline__ T pinned(T v) {
    asm("" : "+s"(v));
    return v;
}
template <typename T>
__device__ __forceinline__ T pick3(int p, T a, T b, T c) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "pick3 selects 32- or 64-bit values");
    using U = typename std::conditional<sizeof(T) == 8, uint64_t, uint32_t>::type;
    const U ua = __builtin_bit_cast(U, pinned(a)), ub = __builtin_bit_cast(U, pinned(b));
    const U uc = __builtin_bit_cast(U, pinned(c));
    const U m1 = (U)0 - (U)(p == 1), m2 = (U)0 - (U)(p == 2);
    return __builtin_bit_cast(T, (U)((ua & ~(m1 | m2)) | (ub & m1) | (uc & m2)));
}

__device__ __forceinline__ Src src_of(const GemvArgs& A, int p) {
    Src r;
    r.w = pick3(p, A.src[0].w, A.src[1].w, A.src[2].w);
    r.s = pick3(p, A.src[0].s, A.src[1].s, A.src[2].s);
    r.z = pick3(p, A.src[0].z, A.src[1].z, A.src[2].z);
    r.n = pick3(p, A.src[0].n, A.src[1].n, A.src[2].n);
    r.wpr = pick3(p, A.src[0].wpr, A.src[1].wpr, A.src[2].wpr);
    return r;
}

__device__ __forceinline__ int bits_of(const GemvArgs& A, int p) {
    return pick3(p, A.bits[0], A.bits[1], A.bits[2]);
}

__device__ __forceinline__ Dst dst_of(const GemvArgs& A, int p) {
    Dst r;
    r.y = pick3(p, A.dst[0].y, A.dst[1].y, A.dst[2].y);
    r.bias = pick3(p, A.dst[0].bias, A.dst[1].bias, A.dst[2].bias);
    r.ld = pick3(p, A.dst[0].ld, A.dst[1].ld, A.dst[2].ld);
    r.pad_ = 0;
    return r;
}

// Virtual row v -> (projection, local row): QKV concatenates [q; k; v], gate-up
// interleaves gate row n -> 2n and up row n -> 2n+1 (packed_gemv.cu:33-42).
template <int MODE>
__device__ __forceinline__ void vmap(const GemvArgs& A, int v, int& proj, int& r) {
    if constexpr (MODE == MODE_GATEUP) {
        proj = v & 1; r = v >> 1;
    } else if constexpr (MODE == MODE_QKV) {
        // branch-free: a = v past Q, b = v past K
        const int n0 = A.src[0].n, n1 = A.src[1].n;
        const int a = v >= n0, b = v >= n0 + n1;
        proj = a + b;
        r = v - (n0 & -a) - (n1 & -b);
    } else {
        proj = 0; r = v;
    }
}

// ---------------------------------------------------------------- finish stage
// Every decode kernel ends here, finishing outputs from fp32 K sums taken before bias.
// The unit of work is what a mode's outputs depend on:
//  * plain GEMV: one row, act(y + bias) -- rows are independent;
//  * gate-up: the pair of virtual rows (2n, 2n + 1) = (gate n, up n), which gives the one
//    output silu(g) * u (the fused module has no bias);
//  * QKV: the pair (v0, v0 + 1), v0 even.  With RoPE, Q and K rows are stored
//    pair-interleaved per head, so the pair holds the original rows
//    (h hd + d, h hd + d + hd/2) that the rotation mixes -- both outputs come from one
//    thread, each row's bias read once.  Without RoPE the two rows are finished one after
//    the other (Q and K rows still go back to their original order).
// A unit is FINISH_ROWS<MODE> consecutive virtual rows; `two` is false when the second row
// of a pair is past V (an odd V).
template <int MODE>
constexpr int FINISH_ROWS = MODE == MODE_GEMV ? 1 : 2;

// QKV pair (v0, v0 + 1), v0 even.  When Q and K are stored pair-interleaved (perm_hd > 0,
// widths multiples of the even perm_hd: host check), a Q or K pair is stored rows (r, r + 1)
// of one head, r even, holding original rows o = head hd + (r - head hd) / 2 and o + hd / 2
// (the inverse of ops.rope_row_order, common.cuh:66-70): with RoPE the two are rotated
// together, without it they are stored back in place.  Otherwise rows keep their order and
// the pair may straddle two projections (odd widths).  One projection lookup per row, the
// head by an invariant division: no generic integer division.
template <int DT>
__device__ __forceinline__ void qkv_finish(const GemvArgs& A, int b, int v0, float y0, float y1, bool two) {
    int p, r;
    vmap<MODE_QKV>(A, v0, p, r);
    const Dst D = dst_of(A, p);
    if (p < 2 && A.perm_hd > 0) {
        if (D.bias) {
            y0 += load_f<DT>(D.bias, r);
            y1 += load_f<DT>(D.bias, r + 1);
        }
        const int hd = A.perm_hd, half = hd >> 1;
        const int head = (int)fdiv((uint32_t)r, A.divHD);
        const int d = (r - head * hd) >> 1;               // < hd / 2
        const long o = (long)b * D.ld + head * hd + d;    // original rows o and o + hd / 2
        if (A.rope_cos != nullptr) {                      // head_dim == perm_hd (host check)
            const float* cs = A.rope_cos + (long)b * hd;
            const float* sn = A.rope_sin + (long)b * hd;
            const float c0 = cs[d], s0 = sn[d], c1 = cs[d + half], s1 = sn[d + half];
            store_f<DT>(D.y, o, y0 * c0 - y1 * s0);
            store_f<DT>(D.y, o + half, y1 * c1 + y0 * s1);
        } else {
            store_f<DT>(D.y, o, y0);
            store_f<DT>(D.y, o + half, y1);
        }
        return;
    }
    if (D.bias) y0 += load_f<DT>(D.bias, r);
    store_f<DT>(D.y, (long)b * D.ld + r, y0);
    if (two) {
        int p1, r1;
        vmap<MODE_QKV>(A, v0 + 1, p1, r1);
        const Dst D1 = p1 == p ? D : dst_of(A, p1);
        if (D1.bias) y1 += load_f<DT>(D1.bias, r1);
        store_f<DT>(D1.y, (long)b * D1.ld + r1, y1);
    }
}

template <int DT, int MODE>
__device__ __forceinline__ void finish(const GemvArgs& A, int b, int v0, float y0, float y1, bool two) {
    if constexpr (MODE == MODE_GATEUP) {
        store_f<DT>(A.dst[0].y, (long)b * A.dst[0].ld + (v0 >> 1), silu(y0) * y1);
    } else if constexpr (MODE == MODE_GEMV) {
        const void* bias = A.dst[0].bias;
        if (bias) y0 += load_f<DT>(bias, v0);
        store_f<DT>(A.dst[0].y, (long)b * A.dst[0].ld + v0, apply_act(y0, A.act));
    } else {
        qkv_finish<DT>(A, b, v0, y0, y1, two);
    }
}

// ---------------------------------------------------------------- split-K combine in the dispatch
// The P workgroups of a row block (one per K split, on any XCD) combine their fp32
// partials without a second launch.  Partials are written and read with agent-scope
// accesses (stores and loads coherent across the XCDs' L2s, `sc1`), so no L2
// write-back or invalidation is needed: a release / acquire pair at agent scope would
// write back and invalidate the whole L2 of the XCD per workgroup, which serialises
// (a K-split batch-1 GEMV went from 7.6 to 38 us that way).  Each wave waits until its
// partial stores have completed, the workgroup meets at a barrier, and one thread
// counts the workgroup in; the workgroup that arrives last (old count P - 1) sets the
// counter back to zero for the next call and adds the P partials in split order
// 0 .. P - 1 -- the order of the combine launch, so both paths give the same bits.  No
// workgroup waits for another.
__device__ __forceinline__ void partial_put(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float partial_get(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A split's sums of a finish unit (v0, and v0 + 1 when `two`) of batch row b into the
// partial buffer.
__device__ __forceinline__ void put_unit(const GemvArgs& A, int p, int b, int v0, float y0, float y1, bool two) {
    float* row = A.partial + ((long)p * A.M + b) * A.V;
    partial_put(row + v0, y0);
    if (two) partial_put(row + v0 + 1, y1);
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

// The finish unit starting at v0 of batch row b summed over splits 0 .. P - 1 in that
// order, then finished.
template <int DT, int MODE>
__device__ __forceinline__ void finish_from_partials(const GemvArgs& A, int b, int v0) {
    const bool two = FINISH_ROWS<MODE> == 2 && v0 + 1 < A.V;
    const long stride = (long)A.M * A.V;
    const float* q = A.partial + (long)b * A.V + v0;
    float y0 = 0.f, y1 = 0.f;
    for (int p = 0; p < A.P; ++p, q += stride) {
        y0 += partial_get(q);
        if (two) y1 += partial_get(q + 1);
    }
    finish<DT, MODE>(A, b, v0, y0, y1, two);
}

// The combining workgroup's finish: the units of rows [vbase, vbase + RB) (vbase and RB
// even) of every batch row, over `nthr` threads.
template <int DT, int MODE>
__device__ __forceinline__ void split_finish(const GemvArgs& A, int vbase, int RB, int nthr) {
    constexpr int U = FINISH_ROWS<MODE>;
    const int nu = RB / U;
    for (int t = threadIdx.x; t < A.M * nu; t += nthr) {
        const int b = t / nu, v0 = vbase + U * (t - b * nu);
        if (v0 < A.V) finish_from_partials<DT, MODE>(A, b, v0);
    }
}

// LDS barrier for code that keeps global loads in flight across it: waits for this
// wave's LDS accesses only (lgkmcnt), then meets the workgroup.  The compiler-level
// memory clobbers on both sides keep LLVM from moving LDS loads or stores across the
// barrier (the wait and barrier intrinsics alone do not order memory in the IR).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4));    // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
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
