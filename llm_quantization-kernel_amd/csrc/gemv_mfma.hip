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
//                consecutive 16-byte pieces of a few rows), R stages in flight
//                per wave in a private LDS ring (cbk_device.hpp: Ring).
//
// Arithmetic per unit: lane (row j = l & 15, chunk kq = l >> 4) reads its chunk
// from the ring, decodes it to packed fp16 1024+q (cbk_decode.hpp) and feeds it as
// the B operand of four v_mfma_f32_16x16x32_f16 whose A operand is the activation
// staged in LDS in the matching code order, so
//   D[i][j] = sum_k x[i][k] * (1024 + q[j][k])          (fp32 accumulate)
//   acc[i][j] += s[j] * (D[i][j] - (1024 + z[j]) * X[i])  with X[i] = sum_k x[i][k].
// This is the reference's per-chunk s*(sum x q - z sum x) (packed_gemv.cu:133-135)
// with the int->float conversion folded into the fp16 bit pattern.
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

// ------------------------------------------------------------------ per-wave staging
// Each wave stages only what its own units need, in its private LDS region, so no
// workgroup barrier stands between the loads and the first MFMA:
//   x   : its units' activations in decode order  [unit][operand m][chunk kq][row i] x 16 B
//   X   : per (unit, batch row) activation sums   [unit][16] floats
//   meta: its units' (scale, zero) pairs          [row j][group] x 4 B
// One x task = 32 activations (one chunk) of one batch row; tasks are chunk-fastest,
// so the 4 chunks of a unit sit in one lane quad and their sums meet by quad shuffles.
struct XTask {
    h8 v[4];
    int i, c;
    bool real;
};

__device__ __forceinline__ void load_x(const GemvArgs& A, int b0, int ua, int nch, int ntask, int task, bool vec,
                                       XTask& t) {
    t.real = task < ntask;
    const int tk = t.real ? task : 0;
    t.i = tk / nch;
    t.c = tk - t.i * nch;
    const _Float16* xr = reinterpret_cast<const _Float16*>(A.x) + (long)(b0 + t.i) * A.K;
    const int k0 = (ua * 4 + t.c) * 32;
    if (vec) {
        // K % 8 == 0: each 8-element piece is wholly inside or past K
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int k = k0 + 8 * q;
            const h8 v = *reinterpret_cast<const h8*>(xr + min(k, A.K - 8));
            t.v[q] = k < A.K ? v : h8{};
        }
    } else {
#pragma unroll
        for (int e = 0; e < 32; ++e) t.v[e >> 3][e & 7] = (k0 + e < A.K) ? xr[k0 + e] : (_Float16)0.f;
    }
}

template <int BITS>
__device__ __forceinline__ void store_x(const XTask& t, int mt, char* xw, float* Xw) {
    u4* xs = reinterpret_cast<u4*>(xw);
    _Float16 xv[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) xv[e] = t.real ? t.v[e >> 3][e & 7] : (_Float16)0.f;
    const h2 one2 = {(_Float16)1.f, (_Float16)1.f};
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 32; e += 2) {
        const h2 pr = {xv[e], xv[e + 1]};
        sum = __builtin_amdgcn_fdot2(pr, one2, sum, false);
    }
    // chunk sums -> unit sum over the lane quad (chunks 4u .. 4u+3), fixed order
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    const int ul = t.c >> 2, kq = t.c & 3;
    if (!t.real) return;
    if (kq == 0) Xw[ul * 16 + t.i] = sum;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        h8 op;
#pragma unroll
        for (int p = 0; p < 8; ++p) op[p] = xv[Decode<BITS>::kappa(8 * m + p)];
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

// One metadata task = (row, group) of the job; packed as (scale, zero) halves.
struct MetaTask {
    _Float16 s, z;
    int idx;
    bool real;
};

// Task (row, unit) of the wave's units [ua, ua + my): the (scale, zero) of the unit's
// group; rows past V get scale 0 so they cancel.
template <int MODE>
__device__ __forceinline__ void load_meta(const GemvArgs& A, int tile, int ua, int my, int gdiv, int task,
                                          MetaTask& t) {
    t.real = task < 16 * my;
    const int tk = t.real ? task : 0;
    const int row = tk / my, ul = tk - row * my;
    const uint32_t* w;
    const _Float16 *s, *z;
    tile_row<MODE>(A, tile * 16 + row, w, s, z);
    const int g = (ua + ul) / gdiv;
    t.s = tile * 16 + row < A.V ? s[g] : (_Float16)0.f;
    t.z = z[g];
    t.idx = tk;
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
// activations are zero, so they contribute nothing.
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

template <int BITS>
__device__ __forceinline__ void ring_chunk(const char* slot, int j, int t, int kq, uint32_t (&w)[BITS]) {
    const char* p = slot + j * Ring<BITS>::PITCH * 16 + t * 16 * BITS + kq * 4 * BITS;
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

// One unit: every LDS read is issued first (the chunk from the ring, its (scale,
// zero), the four activation operands and the activation sums), then the decode,
// four MFMAs and the affine correction.  ul is clamped to a staged unit, so every
// address is valid; units past the wave's range pass valid = false and scale 0.
template <int BITS, int MB>
__device__ __forceinline__ void unit_math(const char* slot, int t, const uint32_t* meta, int my, const char* xw,
                                          const float* Xw, int ul, bool valid, int mt, int lane, f4& acc) {
    const int j = lane & 15, kq = lane >> 4;
    const int i = min(lane & 15, mt - 1);     // batch rows past mt read a staged row; their D rows are unused
    const u4* xs = reinterpret_cast<const u4*>(xw);
    uint32_t w[BITS];
    ring_chunk<BITS>(slot, j, t, kq, w);
    const uint32_t sz = meta[j * my + ul];
    u4 a[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) a[m] = xs[((ul * 4 + m) * 4 + kq) * mt + i];
    const f4 X = *reinterpret_cast<const f4*>(Xw + ul * 16 + 4 * kq);

    uint32_t h[16];
    Decode<BITS>::run(w, h);
    f4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const u4 bw = {h[4 * m], h[4 * m + 1], h[4 * m + 2], h[4 * m + 3]};
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const h8*>(&a[m]),
                                                   *reinterpret_cast<const h8*>(&bw), d, 0, 0, 0);
    }
    const float s = valid ? (float)__builtin_bit_cast(_Float16, (uint16_t)(sz & 0xFFFFu)) : 0.f;
    const float zb = 1024.f + (float)__builtin_bit_cast(_Float16, (uint16_t)(sz >> 16));
#pragma unroll
    for (int r = 0; r < (MB == 1 ? 1 : 4); ++r) acc[r] = fmaf(s, fmaf(-zb, X[r], d[r]), acc[r]);
}

// The S units of one ring slot; units at or past the wave's end (us + t >= ub)
// contribute zero.
template <int BITS, int MB>
__device__ __forceinline__ void stage_math(const char* slot, const uint32_t* meta, int my, const char* xw,
                                           const float* Xw, int ua, int us, int ub, int mt, int lane, f4& acc) {
#pragma unroll
    for (int t = 0; t < Ring<BITS>::S; ++t) {
        const int u = us + t;
        unit_math<BITS, MB>(slot, t, meta, my, xw, Xw, min(u, ub - 1) - ua, u < ub, mt, lane, acc);
    }
}

template <int BITS, int MODE, int MB>
__device__ void run_job(const GemvArgs& A, int job, char* lds) {
    using RG = Ring<BITS>;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int NW = A.nw;
    const int p = job % A.P;
    const int rest = job / A.P;
    const int tile = rest % A.ntiles;
    const int mtile = rest / A.ntiles;
    const int b0 = mtile * 16;
    const int mt = min(16, A.M - b0);
    const int u0 = (int)(((long)A.units * p) / A.P);
    const int u1 = (int)(((long)A.units * (p + 1)) / A.P);
    const int nu = u1 - u0;
    const int gdiv = A.gs >> 7;                                  // units per quantization group
    const int rowbytes = A.C * BITS * 4;

    // this wave's contiguous unit range, in stages of S units, and its LDS region
    const int ua = u0 + (int)(((long)nu * wave) / NW);
    const int ub = u0 + (int)(((long)nu * (wave + 1)) / NW);
    const int my = ub - ua;
    const int nst = (my + RG::S - 1) / RG::S;
    char* wreg = lds + wave * A.wave_bytes;
    char* xw = wreg;
    float* Xw = reinterpret_cast<float*>(wreg + A.xs_bytes);
    uint32_t* meta = reinterpret_cast<uint32_t*>(wreg + A.meta_off);
    char* ring = wreg + A.ring_off;

    const int j = lane & 15;

    // 1) first activation + metadata tasks, 2) the first R weight stages, 3) staging
    const int nch = 4 * my, ntask = nch * mt;
    const bool vec = ((A.K & 7) == 0) && ((reinterpret_cast<uintptr_t>(A.x) & 15) == 0);
    XTask xt;
    load_x(A, b0, ua, max(nch, 1), ntask, lane, vec, xt);
    MetaTask mtk;
    load_meta<MODE>(A, tile, ua, max(my, 1), gdiv, lane, mtk);

    DmaLanes<BITS> dl;
    dma_setup<BITS, MODE>(A, tile, lane, dl);
#pragma unroll
    for (int r = 0; r < RG::R; ++r)
        if (r < nst) dma_stage<BITS>(dl, ua + r * RG::S, rowbytes, ring + r * RG::SLOT);

    // x and meta were loaded before the ring DMA; waiting for them leaves at most the
    // ring stages in flight, the only vector-memory operations the main loop waits on
    store_x<BITS>(xt, mt, xw, Xw);
    if (mtk.real)
        meta[mtk.idx] = (uint32_t)__builtin_bit_cast(uint16_t, mtk.s) | ((uint32_t)__builtin_bit_cast(uint16_t, mtk.z) << 16);
    for (int t0 = 64; t0 < ntask; t0 += 64) {
        load_x(A, b0, ua, nch, ntask, t0 + lane, vec, xt);
        store_x<BITS>(xt, mt, xw, Xw);
    }
    for (int t0 = 64; t0 < 16 * my; t0 += 64) {
        load_meta<MODE>(A, tile, ua, my, gdiv, t0 + lane, mtk);
        if (mtk.real)
            meta[mtk.idx] = (uint32_t)__builtin_bit_cast(uint16_t, mtk.s) | ((uint32_t)__builtin_bit_cast(uint16_t, mtk.z) << 16);
    }

    f4 acc = {0.f, 0.f, 0.f, 0.f};
    // ring of R = 2 slots, unrolled by two so each slot address is static
    for (int st = 0; st < nst; st += 2) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int s = st + r;
            if (s < nst) {
                // in flight, oldest first: stage s, then stage s+1 if it exists
                if (s + 1 < nst) wait_vmcnt<RG::NDMA>();
                else wait_vmcnt<0>();
                const int us = ua + s * RG::S;
                stage_math<BITS, MB>(ring + r * RG::SLOT, meta, my, xw, Xw, ua, us, ub, mt, lane, acc);
                if (s + 2 < nst) {
                    wait_lgkmcnt0();                // every read of this slot has returned
                    dma_stage<BITS>(dl, ua + (s + 2) * RG::S, rowbytes, ring + r * RG::SLOT);
                }
            }
        }
    }

    // cross-wave sum in fixed wave order, then the epilogue on wave 0
    f4* red = reinterpret_cast<f4*>(lds + A.red_off);
    if (wave > 0) red[(wave - 1) * 64 + lane] = acc;
    __syncthreads();
    if (wave == 0) {
        for (int w = 1; w < NW; ++w) {
            const f4 o = red[(w - 1) * 64 + lane];
            acc[0] += o[0]; acc[1] += o[1]; acc[2] += o[2]; acc[3] += o[3];
        }
        const int kq = lane >> 4;
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
    if (job + (int)gridDim.x < A.jobs) __syncthreads();   // the reduction area is reused by the next job
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
        const int v0 = ((job / A.P) % A.ntiles) * 16;
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
