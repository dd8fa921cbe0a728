// gemv_mfma.hip -- fp16 decode GEMV / fused gate-up / fused QKV on gfx950 MFMA.
//
// Replaces cb_gemv_kernel (Kernel/csrc/packed_gemv.cu:83-163) for fp16 activations
// and group sizes that are multiples of 128.
//
// Work decomposition
//   job        = (batch tile of <=16 rows, tile of 16 virtual rows, K split p)
//   workgroup  = NW waves on one job; wave w owns a contiguous range of 128-code
//                units of the split's K range; the NW partial sums meet in LDS.
//   stage      = S consecutive units of the tile's 16 rows, streamed HBM -> LDS by
//                direct-to-LDS dwordx4 loads (each instruction moves 1 KB of
//                consecutive 16-byte pieces of a few rows), up to A.ring stages
//                in flight per wave in a private LDS ring (cbk_device.hpp: Ring);
//                the host sizes the ring to hold a wave's whole range when the
//                LDS allows, so the entire weight stream is requested up front.
//
// Arithmetic per unit: lane (row j = l & 15, chunk kq = l >> 4) reads its chunk
// from the ring, decodes it in place to packed fp16 (cbk_decode.hpp) and feeds it
// as the B operand of four v_mfma_f32_16x16x32_f16 whose A operand is the
// activation staged in LDS in the matching code order and scaled per slot, so
//   D[i][j] = sum_k x[i][k] * (B(k) + q[j][k])              (fp32 accumulate)
//   acc[i][j] += s[j] * (D[i][j] - XB[i] - z[j] * X[i])
// with X[i] = sum_k x[i][k] and XB[i] = sum_k x[i][k] B(k).  This is the
// reference's per-chunk s*(sum x q - z sum x) (packed_gemv.cu:133-135) with the
// int->float conversion folded into the fp16 bit pattern.
//
// Loads are unconditional: rows past V and pieces past a row's end read a clamped,
// valid address and are cancelled arithmetically (scale 0, or a zero activation).
//
// LDS per workgroup: NW private wave regions (staged activations of the wave's
// units, their sums, the (scale, zero) pairs of its groups, its weight ring) and the
// cross-wave reduction area; the reduction is the only workgroup barrier of a job.
#include "cbk_device.hpp"
#include "cbk_decode.hpp"
#include "cbk_kernels.hpp"

namespace cbk {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;

// Explicit waits for the direct-to-LDS weight ring: the compiler does not order
// LDS reads after global_load_lds, so the ring protocol states them itself.
// s_waitcnt simm16 (gfx9): vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14].
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (((N >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8));
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4)); }

// Runtime wait for the ring: at most n stages (NDMA instructions each) may stay in
// flight.  n is wave-uniform, so the switch is scalar branches.
template <int NDMA>
__device__ __forceinline__ void wait_stages(int n) {
    static_assert(NDMA * Ring<4>::RMAX < 64, "vmcnt range");
    switch (n) {
        case 0: wait_vmcnt<0>(); break;
        case 1: wait_vmcnt<NDMA>(); break;
        case 2: wait_vmcnt<2 * NDMA>(); break;
        case 3: wait_vmcnt<3 * NDMA>(); break;
        case 4: wait_vmcnt<4 * NDMA>(); break;
        case 5: wait_vmcnt<5 * NDMA>(); break;
        case 6: wait_vmcnt<6 * NDMA>(); break;
        case 7: wait_vmcnt<7 * NDMA>(); break;
        default: wait_vmcnt<8 * NDMA>(); break;
    }
}

// ------------------------------------------------------------------ batch rows: per-wave staging
// With batch rows (M > 1) MFMA row i = batch row i and column j = tile row j.
// Each wave stages only what its own units need, in its private LDS region, so no
// workgroup barrier stands between the loads and the first MFMA:
//   x   : [unit][operand m][chunk kq][batch row i] x 16 B
//   X   : [unit][2][16] activation sums: plain, and weighted by the slot offsets
//   meta: [tile row j][unit] (scale, zero) halves
// (Batch 1 uses units as MFMA rows and workgroup-shared staging, further down.)
//
// The loads are issued before the weight DMA and consumed after it.  One x task
// = 32 activations (one chunk) of one batch row; tasks are chunk-fastest, so the
// 4 chunks of a unit sit in one lane quad and their sums meet by quad shuffles.
struct XTask {
    h8 v[4];
    int i, c;
    bool real;
};

// Vector path (K % 8 == 0, 16-byte aligned x): raw loads from clamped, valid
// addresses; store_x zeroes the pieces past K.
__device__ __forceinline__ void load_x(const GemvArgs& A, int b0, int ua, int nch, int ntask, int task, bool vec,
                                       XTask& t) {
    t.real = task < ntask;
    const int tk = t.real ? task : 0;
    t.i = (int)(((float)tk + 0.5f) / (float)nch);   // exact: tk < 2^12, nch <= 64
    t.c = tk - t.i * nch;
    const _Float16* xr = reinterpret_cast<const _Float16*>(A.x) + (long)(b0 + t.i) * A.K;
    const int k0 = (ua * 4 + t.c) * 32;
    if (vec) {
#pragma unroll
        for (int q = 0; q < 4; ++q) t.v[q] = *reinterpret_cast<const h8*>(xr + min(k0 + 8 * q, A.K - 8));
    } else {
#pragma unroll
        for (int e = 0; e < 32; ++e) t.v[e >> 3][e & 7] = (k0 + e < A.K) ? xr[k0 + e] : (_Float16)0.f;
    }
}

// Stage one x task: its chunk sums X = sum x and XB = sum x B(p) and its four MFMA
// operands, the activations in decode order scaled by 2^-expo (exact unless the fp16
// result is subnormal) to meet the in-place decoded fields (the MFMA then sums
// x (B(p) + q)).
template <int BITS>
__device__ __forceinline__ void store_x(const XTask& t, int ua, int K, int mt, char* xw, float* Xw) {
    u4* xs = reinterpret_cast<u4*>(xw);
    const int k0 = (ua * 4 + t.c) * 32;
    _Float16 xv[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) xv[e] = (t.real && k0 + (e & ~7) < K) ? t.v[e >> 3][e & 7] : (_Float16)0.f;
    const h2 one2 = {(_Float16)1.f, (_Float16)1.f};
    float sum = 0.f, sumb = 0.f;
#pragma unroll
    for (int e = 0; e < 32; e += 2) {
        const h2 pr = {xv[e], xv[e + 1]};
        sum = __builtin_amdgcn_fdot2(pr, one2, sum, false);
        const h2 ps = {xv[Decode<BITS>::kappa(e)], xv[Decode<BITS>::kappa(e + 1)]};
        const h2 bs = {(_Float16)slot_offset(Decode<BITS>::expo(e)), (_Float16)slot_offset(Decode<BITS>::expo(e + 1))};
        sumb = __builtin_amdgcn_fdot2(ps, bs, sumb, false);
    }
    // chunk sums -> unit sums over the lane quad (chunks 4u .. 4u+3), fixed order
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    sumb += __shfl_xor(sumb, 1, 64);
    sumb += __shfl_xor(sumb, 2, 64);
    const int ul = t.c >> 2, kq = t.c & 3;
    if (!t.real) return;
    if (kq == 0) {
        Xw[ul * 32 + t.i] = sum;
        Xw[ul * 32 + 16 + t.i] = sumb;
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        h8 op;
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            constexpr float kScale[6] = {1.f, 0.5f, 0.25f, 0.125f, 0.0625f, 0.03125f};
            op[p] = xv[Decode<BITS>::kappa(8 * m + p)] * (_Float16)kScale[Decode<BITS>::expo(8 * m + p)];
        }
        xs[((ul * 4 + m) * 4 + kq) * mt + t.i] = *reinterpret_cast<u4*>(&op);
    }
}

// ------------------------------------------------------------------ tile rows
// Virtual row v of the tile -> packed row pointer and metadata row pointers;
// rows past V are clamped to row V-1 (valid memory).
template <int MODE>
__device__ __forceinline__ void tile_row(const GemvArgs& A, int v, const uint32_t*& w, const _Float16*& s,
                                         const _Float16*& z) {
    int proj, r;
    vmap<MODE>(A, v < A.V ? v : A.V - 1, proj, r);
    w = CBK_SEL(A, proj, w) + (long)r * CBK_SEL(A, proj, wpr);
    s = reinterpret_cast<const _Float16*>(CBK_SEL(A, proj, s)) + (long)r * A.G;
    z = reinterpret_cast<const _Float16*>(CBK_SEL(A, proj, z)) + (long)r * A.G;
}

// (scale, zero) of the group of units e0 + (lane >> 4) + 4e, e < 4, of tile row
// lane & 15: one pass covers 16 units of the wave.  Addresses are clamped to the
// wave's last unit; the stores write only real entries and give rows past V
// scale 0, so they cancel.
struct MetaRegs {
    _Float16 s[4], z[4];
};

template <int MODE>
__device__ __forceinline__ void load_meta(const GemvArgs& A, int tile, int ua, int my, int e0, int lane,
                                          MetaRegs& m) {
    const uint32_t* w;
    const _Float16 *s, *z;
    tile_row<MODE>(A, tile * 16 + (lane & 15), w, s, z);
    const int ne = min(4, (my - e0 + 3) >> 2);          // wave-uniform: entries this pass holds
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if (e < ne) {
            const int g = (int)fdiv((uint32_t)(ua + min(e0 + (lane >> 4) + 4 * e, my - 1)), A.divG);
            m.s[e] = s[g];
            m.z[e] = z[g];
        }
    }
}

// batch-row layout: packed (scale, zero) halves
__device__ __forceinline__ void store_meta(const GemvArgs& A, const MetaRegs& m, int tile, int my, int e0, int lane,
                                           uint32_t* meta) {
    const bool row_ok = tile * 16 + (lane & 15) < A.V;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int ul = e0 + (lane >> 4) + 4 * e;
        const uint16_t sb = row_ok ? __builtin_bit_cast(uint16_t, m.s[e]) : (uint16_t)0;
        if (ul < my) meta[(lane & 15) * my + ul] = (uint32_t)sb | ((uint32_t)__builtin_bit_cast(uint16_t, m.z[e]) << 16);
    }
}

// ------------------------------------------------------------------ batch 1: workgroup-shared staging
// At batch 1 the waves of a job share the staged activations and scales (LDS
// offsets in GemvArgs, sizes per unit of the job's K split):
//   x    groups of 16 units (one MFMA activation operand), 4 KB each, fetched and
//        converted by wave g mod NW, one chunk per lane; within a group operand m
//        of chunk kq of unit u sits at slot (kq * 4 + m) * 16 + ((u + 4 kq) & 15)
//        (16 B slots), so the 16 units a lane group reads or writes together fill
//        16 distinct bank groups
//   sums [unit][2] fp32: sum x and sum x B(p) of each unit
//   tab  [unit][tile row j][kq] fp32 masked scales: the scale of (unit, row) in
//        slot kq = (unit >> 2) & 3, zero in the other slots, for units past the
//        split and for rows past V
//   raw  each tile row's span of (scale, zero) halves for the split's groups,
//        [tensor][tile row][piece] x 16 B, fetched as 16-byte pieces aligned to
//        16 bytes (the host checks the scale and zero tensors are 16-byte
//        aligned, so a piece never crosses a page and its first byte is inside
//        the tensor)
// Raw activations and spans arrive by direct-to-LDS loads issued before the
// weight ring, so the staging runs while the weights stream.

// Workgroup barrier after this wave's LDS traffic (no vmcnt wait: the weight ring
// stays in flight).
__device__ __forceinline__ void barrier_lds() {
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
}

// Raw activations of unit group g (16 units, 4 KB) -> x + 4096 g.  The buffer
// descriptor spans x[0, K), so pieces past K arrive as zeros.
__device__ __forceinline__ void dma_x_group(__amdgpu_buffer_rsrc_t xr, int u0, int g, int lane, char* xo) {
    const int voff = (u0 + 16 * g) * 256 + 16 * lane;
#pragma unroll
    for (int t = 0; t < 4; ++t)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(xo + g * 4096 + t * 1024), 16, voff, t * 1024, 0, 0);
}

// Convert group g in place: lane c holds chunk c (unit c >> 2, chunk c & 3) and
// writes its four operands to their slots, and lane 4u the sums of unit u.  Every
// lane's raw reads precede every write (one wave, in-order LDS).
template <int BITS>
__device__ __forceinline__ void stage_x_group(char* xo, float* sums, int g, int lane) {
    u4* grp = reinterpret_cast<u4*>(xo + g * 4096);
    const u4* blk = grp + lane * 4;
    _Float16 xv[32];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const h8 v = *reinterpret_cast<const h8*>(blk + q);
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[8 * q + e] = v[e];
    }
    const h2 one2 = {(_Float16)1.f, (_Float16)1.f};
    float sum = 0.f, sumb = 0.f;
#pragma unroll
    for (int e = 0; e < 32; e += 2) {
        const h2 pr = {xv[e], xv[e + 1]};
        sum = __builtin_amdgcn_fdot2(pr, one2, sum, false);
        const h2 ps = {xv[Decode<BITS>::kappa(e)], xv[Decode<BITS>::kappa(e + 1)]};
        const h2 bs = {(_Float16)slot_offset(Decode<BITS>::expo(e)), (_Float16)slot_offset(Decode<BITS>::expo(e + 1))};
        sumb = __builtin_amdgcn_fdot2(ps, bs, sumb, false);
    }
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    sumb += __shfl_xor(sumb, 1, 64);
    sumb += __shfl_xor(sumb, 2, 64);
    if ((lane & 3) == 0) {
        sums[(16 * g + (lane >> 2)) * 2] = sum;
        sums[(16 * g + (lane >> 2)) * 2 + 1] = sumb;
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        h8 op;
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            constexpr float kScale[6] = {1.f, 0.5f, 0.25f, 0.125f, 0.0625f, 0.03125f};
            op[p] = xv[Decode<BITS>::kappa(8 * m + p)] * (_Float16)kScale[Decode<BITS>::expo(8 * m + p)];
        }
        const int u = lane >> 2, kq = lane & 3;
        grp[(kq * 4 + m) * 16 + ((u + 4 * kq) & 15)] = *reinterpret_cast<u4*>(&op);
    }
}

// The raw spans: lane L of the job's 32 * np lanes fetches piece L % np of the
// span of tensor (L / np) >> 4 (0 scales, 1 zeros), tile row (L / np) & 15, to
// raw + 16 L; pieces past the span re-read its last piece.  Instruction i is
// issued by wave i mod NW.
template <int MODE>
__device__ __forceinline__ void dma_spans(const GemvArgs& A, int tile, int g0, int g1, int wave, int lane,
                                          char* raw) {
    const int np = A.raw_np, nl = 32 * np;
    for (int i = wave; i * 64 < nl; i += A.nw) {
        const int L = min(i * 64 + lane, nl - 1);
        const int tr = (int)fdiv((uint32_t)L, A.divNP);
        const int k = L - tr * np;
        const uint32_t* w;
        const _Float16 *s, *z;
        tile_row<MODE>(A, tile * 16 + (tr & 15), w, s, z);
        const uintptr_t row = reinterpret_cast<uintptr_t>(tr >> 4 ? z : s);
        const uintptr_t first = (row + 2 * g0) & ~(uintptr_t)15, last = (row + 2 * g1) & ~(uintptr_t)15;
        const uintptr_t piece = min(first + 16 * (uintptr_t)k, last);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(piece), (lds_void*)(raw + i * 1024), 16, 0, 0);
    }
}

// Masked scales of this wave's table entries (passes e0 = 64 (wave + NW i) over
// the 64 * nstg entries of the job; lane l takes entry e0 + l, tile row l & 15),
// and this lane's share of its tile row's offset term sum_u s (z X_u + XB_u).
template <int MODE>
__device__ __forceinline__ float stage_tab(const GemvArgs& A, int tile, int u0, int u1, int g0, int nstg, int wave,
                                           int lane, const char* raw, const float* sums, float* tab) {
    const int j = lane & 15;
    const bool row_ok = tile * 16 + j < A.V;
    const uint32_t* w;
    const _Float16 *s, *z;
    tile_row<MODE>(A, tile * 16 + j, w, s, z);
    // byte offset of group g0 within the row's first fetched piece
    const int sa = (int)((reinterpret_cast<uintptr_t>(s) + 2 * g0) & 15);
    const int za = (int)((reinterpret_cast<uintptr_t>(z) + 2 * g0) & 15);
    const _Float16* sr = reinterpret_cast<const _Float16*>(raw + j * A.raw_np * 16 + sa);
    const _Float16* zr = reinterpret_cast<const _Float16*>(raw + (16 + j) * A.raw_np * 16 + za);
    float corr = 0.f;
    for (int e0 = 64 * wave; e0 < 64 * nstg; e0 += 64 * A.nw) {
        const int e = e0 + lane, u = e >> 4;
        const int gi = (int)fdiv((uint32_t)min(u0 + u, u1 - 1), A.divG) - g0;
        const float sc = (u0 + u < u1 && row_ok) ? (float)sr[gi] : 0.f;
        const float zc = (float)zr[gi];
        corr = fmaf(sc, fmaf(zc, sums[2 * u], sums[2 * u + 1]), corr);
        const int blk = (u >> 2) & 3;
        const f4 v = {blk == 0 ? sc : 0.f, blk == 1 ? sc : 0.f, blk == 2 ? sc : 0.f, blk == 3 ? sc : 0.f};
        *reinterpret_cast<f4*>(tab + 4 * e) = v;
    }
    return corr;
}

// ------------------------------------------------------------------ weight ring
template <int BITS>
struct DmaLanes {
    const char* row[Ring<BITS>::NDMA];    // packed row of this lane's piece, per DMA instruction
    int q16[Ring<BITS>::NDMA];            // byte offset of the piece within the stage
};

template <int BITS, int MODE>
__device__ __forceinline__ void dma_setup(const GemvArgs& A, int tile, int lane, DmaLanes<BITS>& d) {
    using RG = Ring<BITS>;
#pragma unroll
    for (int t = 0; t < RG::NDMA; ++t) {
        const int p = 64 * t + lane;
        const int row = min(p / RG::PITCH, 15);
        int q = p - (p / RG::PITCH) * RG::PITCH;
        if (q >= RG::PPR || p >= 16 * RG::PITCH) q = 0;       // pad lanes re-read a live piece
        const uint32_t* w;
        const _Float16 *s, *z;
        tile_row<MODE>(A, tile * 16 + row, w, s, z);
        d.row[t] = reinterpret_cast<const char*>(w);
        d.q16[t] = 16 * q;
    }
}

// Stream stage (units us .. us+S-1 of the 16 rows) into a ring slot.  Pieces past a
// row's end re-read its last 16 bytes: they belong to chunks past C, whose staged
// activations are zero, or to units the wave scales by zero.
template <int BITS>
__device__ __forceinline__ void dma_stage(const DmaLanes<BITS>& d, int us, int rowbytes, char* slot) {
    using RG = Ring<BITS>;
    const int off = us * 16 * BITS;                     // byte offset of the stage in each row
#pragma unroll
    for (int t = 0; t < RG::NDMA; ++t) {
        const char* src = d.row[t] + min(off + d.q16[t], rowbytes - 16);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src),
                                         (lds_void*)(slot + t * 1024), 16, 0, 0);
    }
}

// The lane's chunk of unit t of a ring slot (lp = slot + lane offset).
template <int BITS>
__device__ __forceinline__ void ring_chunk(const char* lp, int t, uint32_t (&w)[BITS]) {
    const char* p = lp + t * 16 * BITS;
    if constexpr (BITS == 4) {
        const u4 v = *reinterpret_cast<const u4*>(p);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (BITS == 2) {
        const u2 v = *reinterpret_cast<const u2*>(p);
        w[0] = v.x; w[1] = v.y;
    } else {
        const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
        w[0] = q[0]; w[1] = q[1]; w[2] = q[2];
    }
}

template <int BITS>
__device__ __forceinline__ f4 unit_mfma(const uint32_t (&w)[BITS], const u4 (&a)[4], uint32_t g) {
    uint32_t h[16];
    Decode<BITS>::run(w, h, g);
    f4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const u4 bw = {h[4 * m], h[4 * m + 1], h[4 * m + 2], h[4 * m + 3]};
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const h8*>(&a[m]),
                                                   *reinterpret_cast<const h8*>(&bw), d, 0, 0, 0);
    }
    return d;
}

// ------------------------------------------------------------------ unit arithmetic, batch rows
template <int BITS>
struct UnitIn {
    uint32_t w[BITS];
    uint32_t sz;
    u4 a[4];
    f4 X, XB;
};

template <int BITS>
__device__ __forceinline__ void unit_load(const char* lp, int t, const uint32_t* meta, int my, const char* xw,
                                          const float* Xw, int ul, int mt, int lane, UnitIn<BITS>& u) {
    const int j = lane & 15, kq = lane >> 4;
    const int i = min(lane & 15, mt - 1);     // batch rows past mt read a staged row; their D rows are unused
    ring_chunk<BITS>(lp, t, u.w);
    u.sz = meta[j * my + ul];
    const u4* xs = reinterpret_cast<const u4*>(xw);
#pragma unroll
    for (int m = 0; m < 4; ++m) u.a[m] = xs[((ul * 4 + m) * 4 + kq) * mt + i];
    u.X = *reinterpret_cast<const f4*>(Xw + ul * 32 + 4 * kq);
    u.XB = *reinterpret_cast<const f4*>(Xw + ul * 32 + 16 + 4 * kq);
}

// acc[i][j] += s * (D[i][j] - XB[i] - z * X[i]); an invalid unit gets scale 0
template <int BITS>
__device__ __forceinline__ void unit_compute(const UnitIn<BITS>& u, bool valid, uint32_t g, f4& acc) {
    const f4 d = unit_mfma<BITS>(u.w, u.a, g);
    const float s = valid ? (float)__builtin_bit_cast(_Float16, (uint16_t)(u.sz & 0xFFFFu)) : 0.f;
    const float z = (float)__builtin_bit_cast(_Float16, (uint16_t)(u.sz >> 16));
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = fmaf(s, fmaf(-z, u.X[r], d[r] - u.XB[r]), acc[r]);
}

// The S units of one ring slot, software-pipelined one unit deep.  Units at or past
// the wave's end (us + t >= ub) read a staged unit and contribute zero.
template <int BITS>
__device__ __forceinline__ void stage_math(const char* lp, const uint32_t* meta, int my, const char* xw,
                                           const float* Xw, int ua, int us, int ub, int mt, int lane, uint32_t g,
                                           f4& acc) {
    constexpr int S = Ring<BITS>::S;
    UnitIn<BITS> u[2];
    unit_load<BITS>(lp, 0, meta, my, xw, Xw, min(us, ub - 1) - ua, mt, lane, u[0]);
#pragma unroll
    for (int t = 0; t < S; ++t) {
        if (t + 1 < S) unit_load<BITS>(lp, t + 1, meta, my, xw, Xw, min(us + t + 1, ub - 1) - ua, mt, lane, u[(t + 1) & 1]);
        unit_compute<BITS>(u[t & 1], us + t < ub, g, acc);
    }
}

// ------------------------------------------------------------------ unit arithmetic, units as rows
// A stage holds units lu .. lu+3 of the split (lu a multiple of 4): unit lu + t is
// MFMA row (lu & 15) + t of the activation operand of its group of 16 units, so its
// result is register t of the lanes with kq = (lu >> 2) & 3 (the masked scales
// zero the other lanes).  lp / mp: the lane's ring and scale addresses for the
// stage.
template <int BITS>
__device__ __forceinline__ void stage_math_units(const char* lp, const float* mp, const u4 (&a)[4], uint32_t g,
                                                 float (&acc)[4]) {
    constexpr int S = Ring<BITS>::S;
    uint32_t w[2][BITS];
    float sc[2];
    ring_chunk<BITS>(lp, 0, w[0]);
    sc[0] = mp[0];
#pragma unroll
    for (int t = 0; t < S; ++t) {
        if (t + 1 < S) {
            ring_chunk<BITS>(lp, t + 1, w[(t + 1) & 1]);
            sc[(t + 1) & 1] = mp[(t + 1) * 64];
        }
        const f4 d = unit_mfma<BITS>(w[t & 1], a, g);
        acc[t] = fmaf(sc[t & 1], d[t], acc[t]);
    }
}

// Waits until at most n vector-memory instructions of this wave are in flight,
// n rounded down to a multiple of 4 (waiting longer is always safe).
__device__ __forceinline__ void wait_vm_atmost(int n) {
    switch (min(n, 60) >> 2) {
        case 0: wait_vmcnt<0>(); break;
        case 1: wait_vmcnt<4>(); break;
        case 2: wait_vmcnt<8>(); break;
        case 3: wait_vmcnt<12>(); break;
        case 4: wait_vmcnt<16>(); break;
        case 5: wait_vmcnt<20>(); break;
        case 6: wait_vmcnt<24>(); break;
        case 7: wait_vmcnt<28>(); break;
        case 8: wait_vmcnt<32>(); break;
        case 9: wait_vmcnt<36>(); break;
        case 10: wait_vmcnt<40>(); break;
        case 11: wait_vmcnt<44>(); break;
        case 12: wait_vmcnt<48>(); break;
        case 13: wait_vmcnt<52>(); break;
        case 14: wait_vmcnt<56>(); break;
        default: wait_vmcnt<60>(); break;
    }
}

// Batch 1: job = (tile of 16 rows, K split p).  The packed bytes of the split's
// units, kbytes per row, travel to a workgroup-shared tile in LDS as row-aligned
// 1 KB blocks (16 * nb direct-to-LDS instructions, dealt round-robin to the
// waves): each block is 64 consecutive 16-byte pieces of one row, so the row
// pointer is scalar, the requests are contiguous, and pieces past the split
// re-read its last piece.  Row j of the tile sits at j * RP with RP = 1024 nb +
// 16, which staggers the rows over the LDS banks.
//
// Order: raw (scale, zero) spans and raw activations, then the tile; the shared
// staging runs while the tile streams; one wait and barrier; then wave w takes
// stages [nstg w / NW, nstg (w + 1) / NW) of S units from the tile and the
// waves' row sums meet in fixed order on wave 0.
template <int BITS, int MODE>
__device__ __forceinline__ void run_job_units(const GemvArgs& A, int job, char* lds) {
    constexpr int S = Ring<BITS>::S;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int NW = A.nw;
    const int tile = (int)fdiv((uint32_t)job, A.divP);   // one batch tile at batch 1
    const int p = job - tile * A.P;
    const int u0 = (int)fdiv((uint32_t)(A.units * p), A.divP);
    const int u1 = (int)fdiv((uint32_t)(A.units * (p + 1)), A.divP);
    const int nstg = (u1 - u0 + S - 1) / S;
    const int s0 = (int)fdiv((uint32_t)(nstg * wave), A.divW);
    const int ns = (int)fdiv((uint32_t)(nstg * (wave + 1)), A.divW) - s0;
    const int ngrp = (S * nstg + 15) >> 4;
    const int rowbytes = A.C * BITS * 4;
    const int kb0 = u0 * 16 * BITS;
    const int kbytes = min(u1 * 16 * BITS, rowbytes) - kb0;
    const int nb = (kbytes + 1023) >> 10;
    const int RP = A.wave_bytes;
    const int j = lane & 15, kq = lane >> 4;

    char* xo = lds;
    float* sums = reinterpret_cast<float*>(lds + A.sum_off);
    float* tab = reinterpret_cast<float*>(lds + A.tab_off);
    char* raw = lds + A.raw_off;
    float* red = reinterpret_cast<float*>(lds + A.red_off);
    char* tl = lds + A.ring_off;
    const int g0 = (int)fdiv((uint32_t)u0, A.divG), g1 = (int)fdiv((uint32_t)(u1 - 1), A.divG);

    // 1) raw spans, raw activations, then this wave's blocks of the tile
    dma_spans<MODE>(A, tile, g0, g1, wave, lane, raw);
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(A.x), (short)0, A.K * 2, 0x00020000);
    for (int g = wave; g < ngrp; g += NW) dma_x_group(xr, u0, g, lane, xo);
    int nt = 0;
    {
        int r = 0, b = wave;                              // block i = r * nb + b, i = wave mod NW
        while (b >= nb) { b -= nb; ++r; }
        while (r < 16) {
            const uint32_t* w;
            const _Float16 *sp, *zp;
            tile_row<MODE>(A, tile * 16 + r, w, sp, zp);
            const char* src = reinterpret_cast<const char*>(w) + kb0 + min(b * 1024 + 16 * lane, kbytes - 16);
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src), (lds_void*)(tl + r * RP + b * 1024),
                                             16, 0, 0);
            ++nt;
            b += NW;
            while (b >= nb) { b -= nb; ++r; }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2) shared staging while the tile streams
    wait_vm_atmost(nt);
    for (int g = wave; g < ngrp; g += NW) stage_x_group<BITS>(xo, sums, g, lane);
    barrier_lds();
    float corr = stage_tab<MODE>(A, tile, u0, u1, g0, nstg, wave, lane, raw, sums, tab);
    wait_vmcnt<0>();
    barrier_lds();

    // 3) this wave's stages from the tile; the activation operand (units 16 gc ..
    //    16 gc + 15 of the split) is reloaded when the group changes
    float ac[4] = {0.f, 0.f, 0.f, 0.f};
    if (ns > 0) {
        const uint32_t g2 = magic_vreg();
        const char* lrow = tl + j * RP + kq * 4 * BITS;
        const float* mlane = tab + j * 4 + kq;
        u4 a[4];
        int gc = -1;
        for (int k = 0; k < ns; ++k) {
            const int lu = S * (s0 + k);                  // first unit of the stage, split-relative
            if ((lu >> 4) != gc) {
                gc = lu >> 4;
                const u4* xs = reinterpret_cast<const u4*>(xo + gc * 4096) + kq * 64 + ((j + 4 * kq) & 15);
#pragma unroll
                for (int m = 0; m < 4; ++m) a[m] = xs[m * 16];
            }
            stage_math_units<BITS>(lrow + lu * 16 * BITS, mlane + lu * 64, a, g2, ac);
        }
    }

    // 4) per tile row: this wave's sum less its share of the offset term, then the
    //    workgroup sum in fixed order on wave 0
    float tot = (ac[0] + ac[1]) + (ac[2] + ac[3]);
    tot += __shfl_xor(tot, 16, 64);
    tot += __shfl_xor(tot, 32, 64);
    corr += __shfl_xor(corr, 16, 64);
    corr += __shfl_xor(corr, 32, 64);
    if (lane < 16) red[wave * 16 + lane] = tot - corr;
    barrier_lds();
    if (wave == 0) {
        const int h = lane >> 4;
        float v = 0.f;
        for (int w = h; w < NW; w += 4) v += red[w * 16 + j];
        v += __shfl_xor(v, 16, 64);
        v += __shfl_xor(v, 32, 64);
        const float partner = __shfl_xor(v, 1, 64);
        const int row = tile * 16 + j;
        if (kq == 0 && row < A.V) {
            if (A.P == 1) epilogue<DT_F16, MODE>(A, 0, row, v, partner);
            else A.partial[(long)p * A.V + row] = v;
        }
    }
    if (job + (int)gridDim.x < A.jobs) barrier_lds();   // the LDS is reused by the next job
}

// Batch rows (M = 2..16 per batch tile): job = (batch tile, tile of 16 rows, K
// split p); wave w owns a contiguous unit range of the split, its staged
// activations, scales and ring in a private LDS region.
template <int BITS, int MODE>
__device__ __forceinline__ void run_job_rows(const GemvArgs& A, int job, char* lds) {
    using RG = Ring<BITS>;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int NW = A.nw;
    // job = (mtile * ntiles + tile) * P + p; every division is by a launch invariant
    const int rest = (int)fdiv((uint32_t)job, A.divP);
    const int p = job - rest * A.P;
    const int mtile = (int)fdiv((uint32_t)rest, A.divT);
    const int tile = rest - mtile * A.ntiles;
    const int b0 = mtile * 16;
    const int mt = min(16, A.M - b0);
    const int u0 = (int)fdiv((uint32_t)(A.units * p), A.divP);
    const int u1 = (int)fdiv((uint32_t)(A.units * (p + 1)), A.divP);
    const int nu = u1 - u0;
    const int rowbytes = A.C * BITS * 4;
    const int j = lane & 15, kq = lane >> 4;

    // this wave's contiguous unit range, in stages of S units, and its LDS region
    const int ua = u0 + (int)fdiv((uint32_t)(nu * wave), A.divW);
    const int ub = u0 + (int)fdiv((uint32_t)(nu * (wave + 1)), A.divW);
    const int my = ub - ua;
    const int nst = (my + RG::S - 1) / RG::S;
    const int R = A.ring;
    char* wreg = lds + wave * A.wave_bytes;
    char* xw = wreg;
    float* Xw = reinterpret_cast<float*>(wreg + A.xs_bytes);
    char* meta = wreg + A.meta_off;
    char* ring = wreg + A.ring_off;

    f4 acc = {0.f, 0.f, 0.f, 0.f};
    if (my > 0) {
        DmaLanes<BITS> dl;
        dma_setup<BITS, MODE>(A, tile, lane, dl);
        const uint32_t g = magic_vreg();
        const int issued = max(R, nst);             // ring stages issued in all (extra slots re-read)
        const char* lring = ring + j * RG::PITCH * 16 + kq * 4 * BITS;
        int slot = 0;
        // 1) the first activation and metadata loads into registers, then the
        //    first R weight stages (loads before the DMA, consumed after it)
        const int nch = 4 * my, ntask = nch * mt;
        const bool vec = ((A.K & 7) == 0) && ((reinterpret_cast<uintptr_t>(A.x) & 15) == 0);
        XTask xt;
        load_x(A, b0, ua, nch, ntask, lane, vec, xt);
        MetaRegs mr;
        load_meta<MODE>(A, tile, ua, my, 0, lane, mr);
        dma_stage<BITS>(dl, ua, rowbytes, ring);
#pragma unroll
        for (int r = 1; r < RG::RMAX; ++r)
            if (r < R) dma_stage<BITS>(dl, ua + r * RG::S, rowbytes, ring + r * RG::SLOT);
        __builtin_amdgcn_sched_barrier(0);

        // 2) staging; passes past the first wait for the whole ring
        store_x<BITS>(xt, ua, A.K, mt, xw, Xw);
        for (int t0 = 64; t0 < ntask; t0 += 64) {
            load_x(A, b0, ua, nch, ntask, t0 + lane, vec, xt);
            store_x<BITS>(xt, ua, A.K, mt, xw, Xw);
        }
        uint32_t* mp = reinterpret_cast<uint32_t*>(meta);
        store_meta(A, mr, tile, my, 0, lane, mp);
        for (int e0 = 16; e0 < my; e0 += 16) {
            load_meta<MODE>(A, tile, ua, my, e0, lane, mr);
            store_meta(A, mr, tile, my, e0, lane, mp);
        }

        // 3) the ring
        for (int s = 0; s < nst; ++s) {
            wait_stages<RG::NDMA>(min(R - 1, issued - 1 - s));
            char* sp = ring + slot * RG::SLOT;
            stage_math<BITS>(lring + slot * RG::SLOT, mp, my, xw, Xw, ua, ua + s * RG::S, ub, mt, lane, g, acc);
            if (s + R < nst) {
                wait_lgkmcnt0();
                dma_stage<BITS>(dl, ua + (s + R) * RG::S, rowbytes, sp);
            }
            slot = slot + 1 == R ? 0 : slot + 1;
        }
    }

    // cross-wave sum in fixed wave order, then the epilogue on wave 0; lane (j, kq)
    // register r holds batch row 4kq + r of tile row j
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
    if (job + (int)gridDim.x < A.jobs) __syncthreads();   // the LDS is reused by the next job
}

template <int BITS, int MODE, int MB>
__device__ __forceinline__ void run_job(const GemvArgs& A, int job, char* lds) {
    if constexpr (MB == 1) run_job_units<BITS, MODE>(A, job, lds);
    else run_job_rows<BITS, MODE>(A, job, lds);
}

template <int BITS, int MODE, int MB>
__global__ void __launch_bounds__(MB == 1 ? 1024 : 512) gemv_mfma_kernel(const GemvArgs A) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    for (int job = blockIdx.x; job < A.jobs; job += gridDim.x) run_job<BITS, MODE, MB>(A, job, lds);
}

// Mixed-width fused QKV: every 16-row tile lies inside one projection (the host
// checks nq and nk are multiples of 16), so the width is uniform per job.
template <int MB>
__global__ void __launch_bounds__(MB == 1 ? 1024 : 512) gemv_mfma_qkv_mixed_kernel(const GemvArgs A) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    for (int job = blockIdx.x; job < A.jobs; job += gridDim.x) {
        const int rest = (int)fdiv((uint32_t)job, A.divP);
        const int v0 = (rest - (int)fdiv((uint32_t)rest, A.divT) * A.ntiles) * 16;
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
