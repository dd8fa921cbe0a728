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
    static_assert(NDMA * (Ring<4>::RMAX - 1) < 64, "vmcnt range");
    switch (n) {
        case 0: wait_vmcnt<0>(); break;
        case 1: wait_vmcnt<NDMA>(); break;
        case 2: wait_vmcnt<2 * NDMA>(); break;
        case 3: wait_vmcnt<3 * NDMA>(); break;
        case 4: wait_vmcnt<4 * NDMA>(); break;
        case 5: wait_vmcnt<5 * NDMA>(); break;
        case 6: wait_vmcnt<6 * NDMA>(); break;
        default: wait_vmcnt<7 * NDMA>(); break;
    }
}

// ------------------------------------------------------------------ per-wave staging
// Each wave stages only what its own units need, in its private LDS region, so no
// workgroup barrier stands between the loads and the first MFMA.  Two layouts:
//
// batch rows (MB = 16, M > 1): MFMA row i = batch row i, row j = tile row j
//   x   : [unit][operand m][chunk kq][batch row i] x 16 B
//   X   : [unit][2][16] activation sums: plain, and weighted by the slot offsets
//   meta: [tile row j][unit] (scale, zero) halves
// units as rows (MB = 1): MFMA row i = unit g0 + i of a group of 16 units, so the
//   activation operand is loaded once per 16 units and each unit keeps only its
//   own output row: lane (j, kq) scales D[4kq + r][j] by the scale of unit
//   g0 + 4kq + r and by zero in every other unit's step.
//   x   : [unit][chunk kq][operand m] x 16 B
//   X   : [unit][2] activation sums, plain and slot-offset weighted (staging only)
//   meta: [unit][tile row j][kq] fp32 scale, zero unless kq is the unit's
//         row block; units past the wave's range are all zero
//   The offset term sum_u s_u (XB_u + z_u X_u) of each tile row is formed at
//   staging and subtracted once after the main loop.
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
// operands, the activations in decode order scaled by 2^-expo (exact) to meet the
// in-place decoded fields (the MFMA then sums x (B(p) + q)).
template <int BITS, int MB>
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
        if constexpr (MB == 1) {
            Xw[ul * 2] = sum;
            Xw[ul * 2 + 1] = sumb;
        } else {
            Xw[ul * 32 + t.i] = sum;
            Xw[ul * 32 + 16 + t.i] = sumb;
        }
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        h8 op;
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            constexpr float kScale[6] = {1.f, 0.5f, 0.25f, 0.125f, 0.0625f, 0.03125f};
            op[p] = xv[Decode<BITS>::kappa(8 * m + p)] * (_Float16)kScale[Decode<BITS>::expo(8 * m + p)];
        }
        if constexpr (MB == 1) xs[(ul * 4 + kq) * 4 + m] = *reinterpret_cast<u4*>(&op);
        else xs[((ul * 4 + m) * 4 + kq) * mt + t.i] = *reinterpret_cast<u4*>(&op);
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

// unit-row layout: the masked fp32 scales of units up to npad (zero past my), and
// this lane's share of its tile row's zero-point term
__device__ __forceinline__ float store_meta_units(const GemvArgs& A, const MetaRegs& m, int tile, int my, int npad,
                                                  int e0, int lane, const float* Xw, float* meta) {
    const bool row_ok = tile * 16 + (lane & 15) < A.V;
    float corr = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int ul = e0 + (lane >> 4) + 4 * e;
        if (ul < npad) {
            float sv = 0.f;
            if (ul < my && row_ok) {
                sv = (float)m.s[e];
                corr = fmaf(sv, fmaf((float)m.z[e], Xw[ul * 2], Xw[ul * 2 + 1]), corr);
            }
            const int blk = (ul >> 2) & 3;
            const f4 v = {blk == 0 ? sv : 0.f, blk == 1 ? sv : 0.f, blk == 2 ? sv : 0.f, blk == 3 ? sv : 0.f};
            *reinterpret_cast<f4*>(meta + (ul * 16 + (lane & 15)) * 4) = v;
        }
    }
    return corr;
}

// ------------------------------------------------------------------ batch 1: staging by LDS-DMA
// At batch 1 the activations and the (scale, zero) pairs travel HBM -> LDS by
// direct-to-LDS loads like the weights, so no register load stands between the
// kernel start and the weight stream and the first stage's math waits only for
// its own data (an exact vmcnt; the compiler would wait for the whole ring).
//
// x: piece p (unit p >> 4, 16-byte piece p & 15 of the unit) -> xs + 16 p, read from
// a clamped, valid address; a task converts its own 64 bytes in place.
__device__ __forceinline__ int dma_x1(const GemvArgs& A, int ua, int npad, int lane, char* xs) {
    const char* xb = reinterpret_cast<const char*>(A.x);
    const int last = A.K * 2 - 16;
    const int n = npad >> 2;                  // 64 pieces = 4 units per instruction
    for (int t = 0; t < n; ++t) {
        const char* src = xb + min(ua * 256 + 1024 * t + 16 * lane, last);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src), (lds_void*)(xs + t * 1024), 16, 0, 0);
    }
    return n;
}

// meta: entry e = j * my + ul (tile row j, unit ul): its scale and zero land
// zero-extended in the dwords at sraw + 4e and zraw + 4e (the 2-byte LDS-DMA
// writes one dword per lane); lanes past 16 my re-read the last entry into the
// padding.  Returns the number of DMA instructions issued.
template <int MODE>
__device__ __forceinline__ int dma_meta1(const GemvArgs& A, int tile, int ua, int my, int lane, char* sraw,
                                         char* zraw) {
    const int n = 16 * my, ni = (n + 63) >> 6;
    const float rmy = 1.f / (float)my;
    for (int t = 0; t < ni; ++t) {
        const int e = min(64 * t + lane, n - 1);
        // e / my for e < 1024, my <= 16: the float quotient of (e + 0.5) is at least
        // 1 / 32 away from an integer, far beyond its rounding error
        const int j = (int)(((float)e + 0.5f) * rmy), ul = e - j * my;
        const uint32_t* w;
        const _Float16 *s, *z;
        tile_row<MODE>(A, tile * 16 + j, w, s, z);
        const int g = (int)fdiv((uint32_t)(ua + ul), A.divG);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(s + g), (lds_void*)(sraw + t * 256), 2, 0, 0);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(z + g), (lds_void*)(zraw + t * 256), 2, 0, 0);
    }
    return 2 * ni;
}

// Masked fp32 scales from the staged raw pairs, and this lane's share of its tile
// row's offset term.  All reads come before the first write: the raw pairs and
// sums sit inside the scale area being written (one pass, my <= 16).
__device__ __forceinline__ float stage_meta1(const GemvArgs& A, int tile, int my, int npad, int lane,
                                             const uint32_t* sraw, const uint32_t* zraw, const float* Xw,
                                             float* meta) {
    const int j = lane & 15;
    const bool row_ok = tile * 16 + j < A.V;
    float sv[4], corr = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int ul = (lane >> 4) + 4 * e;
        const int uc = min(ul, my - 1);
        const float sc = (float)__builtin_bit_cast(_Float16, (uint16_t)sraw[j * my + uc]);
        const float zc = (float)__builtin_bit_cast(_Float16, (uint16_t)zraw[j * my + uc]);
        sv[e] = (ul < my && row_ok) ? sc : 0.f;
        corr = fmaf(sv[e], fmaf(zc, Xw[uc * 2], Xw[uc * 2 + 1]), corr);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int ul = (lane >> 4) + 4 * e;
        const int blk = (ul >> 2) & 3;
        const f4 v = {blk == 0 ? sv[e] : 0.f, blk == 1 ? sv[e] : 0.f, blk == 2 ? sv[e] : 0.f, blk == 3 ? sv[e] : 0.f};
        if (ul < npad) *reinterpret_cast<f4*>(meta + (ul * 16 + j) * 4) = v;
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
// Stage s holds units 4s .. 4s+3 of the wave: unit 4s + t is MFMA row 4 (s & 3) + t
// of the current activation operand, so its result is register t of the lanes with
// kq = s & 3 (the masked scales zero the other lanes).  lp / mp: the lane's ring
// and scale addresses for the stage.
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

template <int BITS, int MODE, int MB>
__device__ __forceinline__ void run_job(const GemvArgs& A, int job, char* lds) {
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
    const int mt = MB == 1 ? 1 : min(16, A.M - b0);
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
        if constexpr (MB == 1) {
            // LDS region: xs = activation operands (raw x first), meta = masked scales,
            // whose first half holds the raw (scale, zero) pairs and then the unit
            // sums until the scales are written
            const int npad = nst * RG::S;
            float* ms = reinterpret_cast<float*>(meta);
            char* sraw = meta;
            char* zraw = meta + npad * 64;
            float* Xs = reinterpret_cast<float*>(meta + npad * 128);

            // 1) ring stage 0, the activations, the pairs, ring stages 1 .. R-1
            dma_stage<BITS>(dl, ua, rowbytes, ring);
            dma_x1(A, ua, npad, lane, xw);
            dma_meta1<MODE>(A, tile, ua, my, lane, sraw, zraw);
#pragma unroll
            for (int r = 1; r < RG::RMAX; ++r)
                if (r < R) dma_stage<BITS>(dl, ua + r * RG::S, rowbytes, ring + r * RG::SLOT);
            __builtin_amdgcn_sched_barrier(0);

            // 2) staging once stage 0, x and the pairs have landed
            wait_stages<RG::NDMA>(R - 1);
            {
                XTask xt;
                const int task = min(lane, 4 * my - 1);
                const h8* blk = reinterpret_cast<const h8*>(xw + task * 64);
#pragma unroll
                for (int q = 0; q < 4; ++q) xt.v[q] = blk[q];
                xt.i = 0;
                xt.c = task;
                xt.real = lane < 4 * my;
                store_x<BITS, 1>(xt, ua, A.K, 1, xw, Xs);
            }
            float corr = stage_meta1(A, tile, my, npad, lane, reinterpret_cast<const uint32_t*>(sraw),
                                     reinterpret_cast<const uint32_t*>(zraw), Xs, ms);
            corr += __shfl_xor(corr, 16, 64);
            corr += __shfl_xor(corr, 32, 64);

            // 3) the ring: stage s sits in slot s % R
            float ac[4] = {0.f, 0.f, 0.f, 0.f};
            u4 a[4];
            const u4* xs = reinterpret_cast<const u4*>(xw);
            const float* mlane = ms + j * 4 + kq;
            for (int s = 0; s < nst; ++s) {
                if ((s & 3) == 0) {          // activation operand of units 4s .. 4s+15
                    const int unit = min(4 * s + j, my - 1);
#pragma unroll
                    for (int m = 0; m < 4; ++m) a[m] = xs[(unit * 4 + kq) * 4 + m];
                }
                wait_stages<RG::NDMA>(min(R - 1, issued - 1 - s));
                char* sp = ring + slot * RG::SLOT;
                stage_math_units<BITS>(lring + slot * RG::SLOT, mlane + s * RG::S * 64, a, g, ac);
                if (s + R < nst) {
                    wait_lgkmcnt0();                // every read of this slot has returned
                    dma_stage<BITS>(dl, ua + (s + R) * RG::S, rowbytes, sp);
                }
                slot = slot + 1 == R ? 0 : slot + 1;
            }
            float tot = (ac[0] + ac[1]) + (ac[2] + ac[3]);
            tot += __shfl_xor(tot, 16, 64);
            tot += __shfl_xor(tot, 32, 64);
            acc[0] = kq == 0 ? tot - corr : 0.f;
        } else {
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
            store_x<BITS, MB>(xt, ua, A.K, mt, xw, Xw);
            for (int t0 = 64; t0 < ntask; t0 += 64) {
                load_x(A, b0, ua, nch, ntask, t0 + lane, vec, xt);
                store_x<BITS, MB>(xt, ua, A.K, mt, xw, Xw);
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
    }

    // cross-wave sum in fixed wave order, then the epilogue on wave 0; lane (j, kq)
    // register r holds batch row 4kq + r of tile row j
    // (at batch 1 a wave's slot is the start of its own activation area, dead by now)
    auto red = [&](int w) -> f4* {
        return MB == 1 ? reinterpret_cast<f4*>(lds + w * A.wave_bytes)
                       : reinterpret_cast<f4*>(lds + A.red_off) + (w - 1) * 64;
    };
    if (wave > 0) red(wave)[lane] = acc;
    __syncthreads();
    if (wave == 0) {
        for (int w = 1; w < NW; ++w) {
            const f4 o = red(w)[lane];
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
