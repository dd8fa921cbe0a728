// gemm_f16.hip -- fp16 / bf16 prefill packed GEMM on gfx950: out[M,N] = act(x . W-hat^T + bias).
//
// Replaces cb_gemm_tc_kernel (Kernel/csrc/packed_gemm.cu:12-117) for fp16 and bf16
// activations, with the reference's weight rounding W-hat = RN_T((q - z) * s)
// (packed_gemm.cu:56,60).
//
// Tile: 128 x 128 outputs per workgroup of eight waves, two per SIMD.  Wave w owns
// the 128 x 32 slab at columns 32 (w & 3) -- every tile row, so each column is
// dequantized once -- for k half w >> 2 of every stage: the two waves sharing a
// SIMD split each stage's k-steps, so while one waits on LDS or memory the other
// issues, and their partial sums meet in LDS at the end.
//
// Every wave computes and every wave loads.  Global traffic is direct-to-LDS
// buffer loads (one instruction per KB, no VGPR data).  A stage is 128 codes of K.
// Load group t holds the wave's eighth of activation stage t + 2 (128 rows x 128
// codes, XOR-swizzled 16-byte pieces, into a ring of three stage slots) and, at
// even t, of weight block t / 2 + 1 (256 codes of the tile's 128 packed rows,
// double-buffered) and of a scale / zero window (8 groups per row).  Group t's
// instructions go out in eight slots, two per k-step, between barrier t and the
// wait before barrier t + 1, so no wave stalls long on a full memory queue while
// the MFMAs starve.  Before barrier t + 1 a wave waits until at most group t is in
// flight, so group t - 1 -- everything stage t + 1 needs -- has landed for every
// wave once the barrier passes.  Every group of a parity holds the same number of
// loads, so the waits are constants.
//
// MFMA operand lane map (v_mfma_f32_32x32x16_f16): lane (r32 = lane & 31, hk =
// lane >> 5) holds column r32's B operand and the A operands of rows 32 a + r32
// (a < 4).  Step ks of a stage gives lane half hk the codes 64 hk + 8 ks .. +7
// (octet ks & 3 of chunk 4 s + 2 hk + (ks >> 2)), the same k order for both
// operands; the wave of k half kh runs steps 4 kh .. 4 kh + 3, so each lane needs
// one chunk (chunk 2 hk + kh of the stage) and one (scale, zero) per stage.
//
// Weight rounding: the codes of a pair are OR-ed into 0x6400 (1024 + q, exact),
// then (h - (1024 + z)) * s in packed fp16 when every zero point of the wave's
// columns is an integer below 1024 in magnitude (the reference quantizer's; each
// wave scans its columns' zeros once): the difference is an exact integer and the
// product rounds once, exactly RN_fp16((q - z) * s).  Other zero points take the
// fp32 product.  bf16 (v_mfma_f32_32x32x16_bf16): the codes go to fp32 (v_cvt_f32_ubyte),
// W-hat = RN_bf16(fma(q, s, -z s)) with integer zeros (both products exact in fp32, so
// the fma returns (q - z) s exactly), else RN_bf16((q - z) * s) in fp32 -- the
// reference's fp32 value rounded once.  Codes at k >= K meet zero activations, so
// the tail of the last weight block contributes nothing.
#include "cbk_decode.hpp"
#include "cbk_device.hpp"
#include "cbk_kernels.hpp"

namespace cbk {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef __bf16 b2 __attribute__((ext_vector_type(2)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef float f4x __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) char lds_t;            // LDS bytes: 32-bit addresses

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int WAVES = 8;                     // two per SIMD: four column slabs x two k halves
constexpr int THREADS = 64 * WAVES;
constexpr int NSTAGE = 3;                    // activation stage slots in LDS
constexpr int TILE = BM * BK * 2;            // bytes of an activation stage (32 KB)
constexpr int APR = BK * 2 / 16;             // 16-byte pieces per activation row of a stage
constexpr int A_Q = TILE / 1024 / WAVES;     // activation instructions per wave per stage (4)
constexpr int WBLK = 2;                      // stages per weight block (256 codes)
constexpr int SZG = 8;                       // groups per scale / zero window
constexpr int SZ_Q = 2 * BN * 2 / 64 / WAVES;   // window instructions per wave (1)
constexpr int SZ_BUF = 2 * BN * 32;          // [tensor][row] x 32 bytes
constexpr int SLOTS = 8;                     // issue slots of a load group (two per k-step)
constexpr int KSTEPS = 4;                    // k-steps of a stage per wave (its k half)

// Weight block geometry: a row's block is 32 * BITS bytes at phase 0 (W4), 0 / 8
// (W2) or 0 / 4 / 8 / 12 (W3) within its first aligned piece, PPR pieces (odd, so
// 32 rows read at one offset hit distinct banks).  The block's pieces are spread
// over the waves in whole instructions; the last ones re-read the last row
// into the padding.
template <int BITS> struct WGeo {
    static constexpr int PPR = BITS == 4 ? 9 : (BITS == 3 ? 7 : 5);
    static constexpr int PITCH = 16 * PPR;
    static constexpr int W_Q = (BN * PPR + 64 * WAVES - 1) / (64 * WAVES);
    static constexpr int BUF = W_Q * WAVES * 1024;
    static_assert(A_Q + W_Q + SZ_Q <= SLOTS, "slot budget");
};

constexpr int A_OFF = 0;
constexpr int W_OFF = NSTAGE * TILE;
template <int BITS> constexpr int SZ_OFF = W_OFF + 2 * WGeo<BITS>::BUF;
template <int BITS> constexpr int LDS_BYTES = SZ_OFF<BITS> + 2 * SZ_BUF;
static_assert(LDS_BYTES<4> <= 160 * 1024, "LDS budget");
// Epilogue: the two k halves' fp32 tile images, k half kh at kh * SUM_IMG.
constexpr int SUM_PITCH = BN + 8;
constexpr int SUM_IMG = BM * SUM_PITCH * 4;
static_assert(2 * SUM_IMG <= LDS_BYTES<2> && LDS_BYTES<2> <= LDS_BYTES<3>, "epilogue LDS");

__device__ __forceinline__ int swz(int r) { return r & (APR - 1); }

template <int N>
__device__ __forceinline__ void vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (((N >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier without a memory fence: __syncthreads() would make the compiler
// wait for every in-flight load of the wave (vmcnt(0)), draining the prefetch.
// This only completes the wave's own LDS traffic (lgkmcnt(0)) before the barrier.  The
// compiler-level memory clobbers on both sides keep LLVM from moving LDS accesses (or
// the direct-to-LDS loads) across it: the wait and barrier intrinsics alone do not
// order memory in the IR.
__device__ __forceinline__ void barrier_lds() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4));    // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// One 16-byte-per-lane direct-to-LDS buffer load into byte `dst` of the LDS.  A
// plain function: the builtin then appears in no template body, which the host
// pass would reject.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, lds_t* lds, uint32_t dst, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(lds + dst), 16, voff, soff, 0, 0);
}

// A byte offset past every buffer descriptor's range: such loads return zero.
constexpr int OOR = 0x7FFFFFF0;

// ------------------------------------------------------------------ the wave's loads
// Activations: wave v moves instructions A_Q v .. A_Q v + A_Q - 1 of a stage (its
// rows 16 v .. 16 v + 15); lane l of instruction t moves slot q = 64 t + l: row
// q >> 4, logical piece (q & 15) ^ swz(row), through a descriptor over the
// activations (row clamped to M).  In a partial last stage, pieces at k >= K read
// as zero (K % 8 == 0, so a piece is wholly inside or outside).
// Weights: wave v moves instructions W_Q v + t of a block; lane l moves piece
// q = 64 (W_Q v + t) + l, row q / PPR (clamped to the tile), piece q % PPR of the
// row's aligned span.  Windows: wave v moves instruction v of eight (the first four
// the scales, the rest the zeros); lane l moves piece q & 1 of tile row
// (q >> 1) & 127's span, the 16 halves from floor8(col * G) + 8 w.  The lane's
// offsets are fixed; the stage / block / window offset is a scalar.
template <int BITS>
struct Loads {
    __amdgpu_buffer_rsrc_t ar, szr;
    __amdgpu_buffer_rsrc_t wr[WGeo<BITS>::W_Q];   // per weight instruction (gate-up: gate or up)
    int avoff[A_Q];
    int atoff[A_Q];
    int woff[WGeo<BITS>::W_Q];
    int szoff[SZ_Q];
    uint32_t a_lds, w_lds, sz_lds;   // LDS byte of the wave's first instruction in a slot / buffer
};

// Gate-up (GU): the tile's rows 0..63 are gate rows n0 .. n0 + 63, rows 64..127 the up rows
// of the same outputs.  A weight block's pieces of rows 0..63 fill exactly PPR of its
// instructions (64 rows x PPR pieces), so every instruction reads one tensor; window
// instruction v covers rows 32 (v & 3) .. +31, so waves 0, 1, 4, 5 read the gate's scales
// and zeros and waves 2, 3, 6, 7 the up's.
template <int BITS, bool GU>
__device__ __forceinline__ void loads_setup(const GemmArgs& A, int m0, int n0, int nst, int wave, int lane,
                                            Loads<BITS>& L) {
    using G = WGeo<BITS>;
    L.ar = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(A.x), (short)0, A.M * A.K * 2, 0x00020000);
    const bool up_sz = GU && (wave & 3) >= 2;
    L.szr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(SZ_Q * wave >= 4 ? (up_sz ? A.z2 : A.z) : (up_sz ? A.s2 : A.s)), (short)0,
        A.N * A.G * 2, 0x00020000);
#pragma unroll
    for (int t = 0; t < G::W_Q; ++t) {
        const bool up_w = GU && G::W_Q * wave + t >= G::PPR;
        L.wr[t] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(up_w ? A.w2 : A.w), (short)0,
                                                    A.N * A.wpr * 4, 0x00020000);
    }
#pragma unroll
    for (int i = 0; i < A_Q; ++i) {
        const int q = 64 * (A_Q * wave + i) + lane;
        const int r = q / APR, p = (q & (APR - 1)) ^ swz(r);
        const int rowoff = min(m0 + r, A.M - 1) * A.K * 2;
        const int k = BK * (nst - 1) + 8 * p;
        L.avoff[i] = rowoff + 16 * p;
        L.atoff[i] = k < A.K ? rowoff + 2 * k : OOR;
    }
#pragma unroll
    for (int t = 0; t < G::W_Q; ++t) {
        const int q = 64 * (G::W_Q * wave + t) + lane;
        const int r = min(q / G::PPR, BN - 1), p = q - (q / G::PPR) * G::PPR;
        const int rr = GU ? (r & 63) : r;
        L.woff[t] = ((min(n0 + rr, A.N - 1) * A.wpr * 4) & ~15) + 16 * p;
    }
#pragma unroll
    for (int t = 0; t < SZ_Q; ++t) {
        const int q = 64 * (SZ_Q * wave + t) + lane;
        const int r = (q >> 1) & (BN - 1), p = q & 1;
        const int rr = GU ? (r & 63) : r;
        L.szoff[t] = ((min(n0 + rr, A.N - 1) * A.G) & ~7) * 2 + 16 * p;
    }
    L.a_lds = A_OFF + A_Q * wave * 1024;
    L.w_lds = W_OFF + G::W_Q * wave * 1024;
    L.sz_lds = SZ_OFF<BITS> + SZ_Q * wave * 1024;
}

// Load schedule (scalars).  Group t holds activation stage t + 2 (slot (t + 2) % 3,
// the stage clamped to the last) and, at even t, weight block j = t / 2 + 1
// (buffer j & 1, clamped to the last) and window win + (j % rp != 0) into its
// buffer: the window of block j when j starts one, else the next window ahead of
// time (its buffer held a window that ended at least one block before j - 1, and
// its live load comes later), so every even group moves the same bytes.  All
// buffers written by group t were last read in stages <= t - 1, which every wave
// has finished (LDS reads completed) when it meets barrier t.
struct Sched {
    int nst, nblk, rp;            // stages, weight blocks, blocks per window
    int aslot;                    // (t + 2) % 3 of the next group
    int blk_in_win, win;          // j % rp, j / rp of the next even group's block
};

struct Group {
    uint32_t a_dst, w_dst, sz_dst;   // LDS bytes of the wave's first instructions
    int a_soff, w_soff, sz_soff;     // scalar global byte offsets
    bool a_tail;                     // activations: the partial last stage
};

template <int BITS, bool TAIL, bool EVEN>
__device__ __forceinline__ void group_at(const Loads<BITS>& L, Sched& sc, int t, Group& g) {
    const int sa = min(t + 2, sc.nst - 1);
    g.a_tail = TAIL && sa == sc.nst - 1;
    g.a_dst = L.a_lds + sc.aslot * TILE;
    g.a_soff = g.a_tail ? 0 : BK * 2 * sa;
    sc.aslot = sc.aslot == NSTAGE - 1 ? 0 : sc.aslot + 1;
    if constexpr (EVEN) {
        const int j = t / 2 + 1;
        g.w_dst = L.w_lds + (j & 1) * WGeo<BITS>::BUF;
        g.w_soff = min(j, sc.nblk - 1) * (32 * BITS);
        const int w = sc.blk_in_win == 0 ? sc.win : sc.win + 1;
        g.sz_dst = L.sz_lds + (w & 1) * SZ_BUF;
        g.sz_soff = 2 * SZG * w;
        const bool wrap = sc.blk_in_win + 1 == sc.rp;
        sc.blk_in_win = wrap ? 0 : sc.blk_in_win + 1;
        sc.win += wrap ? 1 : 0;
    }
}

// Slot k (a constant after unrolling) of a group: activation instruction k
// (k < A_Q), then, in an even group, weight instruction k - A_Q, then the window.
template <int BITS, bool TAIL, bool EVEN>
__device__ __forceinline__ void issue_slot(const Loads<BITS>& L, const Group& g, int k, lds_t* lds) {
    constexpr int WQ = WGeo<BITS>::W_Q;
    if (k < A_Q) {
        dma16(L.ar, lds, g.a_dst + k * 1024, TAIL && g.a_tail ? L.atoff[k] : L.avoff[k], g.a_soff);
    } else if constexpr (EVEN) {
        const int e = k - A_Q;
        if (e < WQ) dma16(L.wr[e], lds, g.w_dst + e * 1024, L.woff[e], g.w_soff);
        else if (e < WQ + SZ_Q) dma16(L.szr, lds, g.sz_dst + (e - WQ) * 1024, L.szoff[e - WQ], g.sz_soff);
    }
}

template <int BITS, bool TAIL, bool EVEN>
__device__ __forceinline__ void issue_group(const Loads<BITS>& L, const Group& g, lds_t* lds) {
#pragma unroll
    for (int k = 0; k < SLOTS; ++k) issue_slot<BITS, TAIL, EVEN>(L, g, k, lds);
}

// Wait until at most group t (all of it issued) is in flight: group t - 1 landed.
template <int BITS, bool EVEN>
__device__ __forceinline__ void wait_group() {
    if constexpr (EVEN) vmcnt<A_Q + WGeo<BITS>::W_Q + SZ_Q>();
    else vmcnt<A_Q>();
}

// The 16 storage bits of v rounded to the output dtype.
template <int DT>
__device__ __forceinline__ uint32_t raw16(float v) {
    return (uint32_t)__builtin_bit_cast(uint16_t, Dt<DT>::from_f(v));
}

__device__ __forceinline__ _Float16 half_of(uint32_t v) {
    return __builtin_bit_cast(_Float16, (uint16_t)v);
}

// A scale or zero point of the activations' dtype (raw bits) as a float.
template <int DT>
__device__ __forceinline__ float meta_f(uint32_t bits) {
    if constexpr (DT == DT_BF16) return __uint_as_float(bits << 16);
    else return (float)half_of(bits);
}

// A zero point that allows the exact fast form: an integer below 1024 in magnitude.
template <int DT>
__device__ __forceinline__ bool zero_is_small_int(uint32_t zbits) {
    const float zf = meta_f<DT>(zbits & 0xFFFFu);
    return zf == __builtin_rintf(zf) && __builtin_fabsf(zf) < 1024.f;
}

// Whether every zero point of columns [c0, min(c0 + 32, N)) -- a contiguous range of
// the zeros tensor, whose start is 16-byte aligned -- allows the packed-fp16 form.
// scan_issue loads the lane's first SCAN_U pieces before the prologue's loads go
// out, so their latency hides behind them; scan_finish checks them and the rest.
constexpr int SCAN_U = 8;
struct ZScan {
    u4 v[SCAN_U];
};

__device__ __forceinline__ void scan_issue(const GemmArgs& A, const void* zt, int c0, int lane, ZScan& zs) {
    const uint16_t* z = reinterpret_cast<const uint16_t*>(zt);
    const long beg = (long)c0 * A.G, end = (long)min(c0 + 32, A.N) * A.G;   // beg % 8 == 0
#pragma unroll
    for (int u = 0; u < SCAN_U; ++u) {
        const long i = beg + 8 * lane + 512 * u;
        zs.v[u] = i + 8 <= end ? *reinterpret_cast<const u4*>(z + i) : u4{0, 0, 0, 0};
    }
}

template <int DT>
__device__ __forceinline__ bool scan_finish(const GemmArgs& A, const void* zt, int c0, int lane, const ZScan& zs) {
    const uint16_t* z = reinterpret_cast<const uint16_t*>(zt);
    const long beg = (long)c0 * A.G, end = (long)min(c0 + 32, A.N) * A.G;
    bool ok = true;
#pragma unroll
    for (int u = 0; u < SCAN_U; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            ok &= zero_is_small_int<DT>(zs.v[u][j] & 0xFFFFu) & zero_is_small_int<DT>(zs.v[u][j] >> 16);
    for (long i = beg + 8 * lane; i < end; i += 8 * 64) {
        if (i + 8 <= end) {
            if (i < beg + 512 * SCAN_U) continue;      // preloaded
            const u4 v = *reinterpret_cast<const u4*>(z + i);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                ok &= zero_is_small_int<DT>(v[j] & 0xFFFFu) & zero_is_small_int<DT>(v[j] >> 16);
        } else {
            for (long e = i; e < end; ++e) ok &= zero_is_small_int<DT>(z[e]);
        }
    }
    return __builtin_amdgcn_ballot_w64(!ok) == 0;
}

// ------------------------------------------------------------------ compute
// The lane's packed chunk of a stage and its scale and zero as raw fp16 bits.
template <int BITS>
struct WStage {
    uint32_t w[BITS];
    uint32_t s, z;
};

// Octet o (codes 8o .. 8o+7) of a chunk as 4 packed pairs (1024 + q, exact;
// g = 0x64006400 in a VGPR); o is a compile-time step index.
template <int BITS> struct Octet;

template <> struct Octet<4> {
    // word o holds codes 8o .. 8o+7 as nibbles; pair i = the two nibbles of byte i
    static __device__ __forceinline__ void run(const uint32_t (&w)[4], int o, uint32_t g, uint32_t (&h)[4]) {
        const uint32_t v = w[o], v4 = v >> 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t ps = (uint32_t)i | (0x0Cu << 8) | ((4u + i) << 16) | (0x0Cu << 24);
            h[i] = (__builtin_amdgcn_perm(v4, v, ps) & 0x000F000Fu) | g;
        }
    }
};

template <> struct Octet<2> {
    // word o >> 1 holds codes 16 (o >> 1) .. +15 at bits 2j; octet o is its half o & 1
    static __device__ __forceinline__ void run(const uint32_t (&w)[2], int o, uint32_t g, uint32_t (&h)[4]) {
        const uint32_t v0 = w[o >> 1] >> (16 * (o & 1));
        const uint32_t v2 = v0 >> 2, v4 = v0 >> 4, v6 = v0 >> 6;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // codes 2i, 2i+1 at bits 4i and 4i + 2
            const uint32_t b = (uint32_t)(i >> 1);
            const uint32_t ps = b | (0x0Cu << 8) | ((4u + b) << 16) | (0x0Cu << 24);
            const uint32_t lo = (i & 1) ? v4 : v0, hi = (i & 1) ? v6 : v2;
            h[i] = (__builtin_amdgcn_perm(hi, lo, ps) & 0x00030003u) | g;
        }
    }
};

template <> struct Octet<3> {
    // octet o = chunk bits 24o .. 24o+23 (octets 1 and 2 straddle words); pair i at
    // bits 6i .. 6i+5 of it
    static __device__ __forceinline__ void run(const uint32_t (&w)[3], int o, uint32_t g, uint32_t (&h)[4]) {
        const uint32_t a = o == 0 ? w[0]
                         : o == 1 ? __builtin_amdgcn_alignbit(w[1], w[0], 24)
                         : o == 2 ? __builtin_amdgcn_alignbit(w[2], w[1], 16)
                                  : (w[2] >> 8);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t x = (a >> (6 * i)) & 0x3Fu;
            h[i] = (((x << 13) | x) & 0x00070007u) | g;   // code 2i at bit 0, code 2i+1 at bit 16
        }
    }
};

// B operand of the wave's step kq: octet kq of the lane's chunk.  DQ: 0 fp16, 1 fp16
// with every zero point of the wave's columns an integer below 1024 in magnitude (the
// packed-fp16 form), 2 bf16, 3 bf16 with such zero points (the fma form).
template <int BITS, int DQ>
__device__ __forceinline__ u4 dequant_octet(const WStage<BITS>& r, int kq, uint32_t g) {
    if constexpr (DQ >= 2) {
        const float zf = meta_f<DT_BF16>(r.z), sf = meta_f<DT_BF16>(r.s);
        const float czs = -zf * sf;                   // exact when DQ == 3
        uint32_t h[4];
        Octet<BITS>::run(r.w, kq, 0u, h);             // codes 2i, 2i+1 at bits 0 and 16
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float lo = (float)(h[i] & 0xFFu), hi = (float)((h[i] >> 16) & 0xFFu);
            const float a = DQ == 3 ? fmaf(lo, sf, czs) : (lo - zf) * sf;
            const float b = DQ == 3 ? fmaf(hi, sf, czs) : (hi - zf) * sf;
            const b2 v = {(__bf16)a, (__bf16)b};
            o[i] = __builtin_bit_cast(uint32_t, v);
        }
        return u4{o[0], o[1], o[2], o[3]};
    }
    constexpr bool FAST = DQ == 1;
    const float zf = (float)half_of(r.z);
    const _Float16 cz = (_Float16)(1024.f + zf);      // exact when FAST: an integer below 2048
    const _Float16 sh = half_of(r.s);
    const h2 c2 = {cz, cz}, s2 = {sh, sh};
    const float sf = (float)sh;
    uint32_t h[4];
    Octet<BITS>::run(r.w, kq, g, h);
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (FAST) {
            const h2 v = (__builtin_bit_cast(h2, h[i]) - c2) * s2;
            o[i] = __builtin_bit_cast(uint32_t, v);
        } else {
            const float lo = ((float)(h[i] & 0x3FFu) - zf) * sf;
            const float hi = ((float)((h[i] >> 16) & 0x3FFu) - zf) * sf;
            const h2 v = {(_Float16)lo, (_Float16)hi};
            o[i] = __builtin_bit_cast(uint32_t, v);
        }
    }
    return u4{o[0], o[1], o[2], o[3]};
}

// Per-lane constants of a wave's column and its LDS reads.
struct ColInfo {
    int wlane;        // LDS byte of the lane's chunk in weight buffer 0, stage 0 of a block
    int szlane;       // LDS byte of the column's span in window buffer 0 plus (col * G) & 7 halves
    int soff;         // LDS byte of the row's span in a window buffer (general group sizes)
    int cix;          // the lane's chunk within a stage: 2 hk + kh
    long cg;          // col * G
    int aaddr[KSTEPS];   // LDS byte of the lane's A operand of step kq within a stage (row block 0)
};

// A operands of the wave's step kq of the stage in slot `slot`: af[a] = row 32 a +
// r32 (row blocks are 32 rows = 8 KB apart: immediate offsets).
__device__ __forceinline__ void read_a(const lds_t* lds, int slot, int kq, const ColInfo& ci, u4 (&af)[4]) {
    typedef __attribute__((address_space(3))) const u4 l4;
    const lds_t* at = lds + slot * TILE + ci.aaddr[kq];
#pragma unroll
    for (int a = 0; a < 4; ++a) af[a] = *reinterpret_cast<l4*>(at + a * 32 * APR * 16);
}

// The lane's chunk of stage s (chunk 4 (s % WBLK) + 2 hk + kh of block s / WBLK)
// and its (scale, zero).  GS128: the group size is 128, so the chunk's group is
// stage s's, at a lane-independent offset in window s >> 3.
template <int BITS, bool GS128>
__device__ __forceinline__ void read_w(const GemmArgs& A, const lds_t* lds, int s, const ColInfo& ci,
                                       WStage<BITS>& r) {
    typedef __attribute__((address_space(3))) const u4 l4;
    typedef __attribute__((address_space(3))) const u2 l2;
    typedef __attribute__((address_space(3))) const uint16_t l16;
    const int j = s / WBLK;
    const lds_t* p = lds + (j & 1) * WGeo<BITS>::BUF + (s % WBLK) * (16 * BITS) + ci.wlane;
    if constexpr (BITS == 4) {
        const u4 v = *reinterpret_cast<l4*>(p);
        r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
    } else if constexpr (BITS == 3) {
        // a 12-byte chunk is only word aligned
        typedef __attribute__((address_space(3))) const uint32_t l1;
        r.w[0] = *reinterpret_cast<l1*>(p);
        r.w[1] = *reinterpret_cast<l1*>(p + 4);
        r.w[2] = *reinterpret_cast<l1*>(p + 8);
    } else {
        const u2 v = *reinterpret_cast<l2*>(p);
        r.w[0] = v.x; r.w[1] = v.y;
    }
    if constexpr (GS128) {
        l16* q = reinterpret_cast<l16*>(lds + ((s >> 3) & 1) * SZ_BUF + 2 * (s & 7) + ci.szlane);
        r.s = q[0];
        r.z = q[BN * 16];      // the zeros follow the scales' 128 rows x 32 bytes
    } else {
        const int w = (int)(fdiv((uint32_t)(j * 256), A.divG) >> 3);       // j / (gs / 32)
        const lds_t* sb = lds + SZ_OFF<BITS> + (w & 1) * SZ_BUF;
        const long span = (ci.cg + SZG * w) & ~7L;
        const int gi = (int)fdiv((uint32_t)((4 * s + ci.cix) * 32), A.divG);
        l16* q = reinterpret_cast<l16*>(sb + ci.soff) + (int)(ci.cg + gi - span);
        r.s = q[0];
        r.z = q[BN * 16];
    }
}

// One k-step: 4 MFMAs of 32 x 32 x 16 (rows 32 a .. of the slab, the lane's column).
template <bool BF>
__device__ __forceinline__ void mma_step(const u4 (&af)[4], const u4& bw, f16x (&acc)[4]) {
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        if constexpr (BF)
            acc[a] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*reinterpret_cast<const b8*>(&af[a]),
                                                             *reinterpret_cast<const b8*>(&bw), acc[a], 0, 0, 0);
        else
            acc[a] = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const h8*>(&af[a]),
                                                            *reinterpret_cast<const h8*>(&bw), acc[a], 0, 0, 0);
    }
}

// Everything a stage needs besides its operands.
template <int BITS>
struct Ctx {
    const GemmArgs& A;
    lds_t* lds;
    const ColInfo& ci;
    uint32_t g;
    const Loads<BITS>& L;
    Sched& sc;
    int cslot;                    // slot of the stage being computed
};

// The wave's four k-steps of stage s as a software pipeline: the A operands of
// step kq are read two steps ahead (a[kq & 3] of four rotating sets) and its B
// operand dequantized one step ahead.  On entry a[0], a[1] hold steps 0 and 1, bw
// step 0, wc the chunk of stage s, gc the resolved group s.  NEXT: steps 0 and 1
// issue slots 4 .. 7 of group s; after step 1 (every read of stage s's activation
// slot issued; barrier_lds completes them) the wave waits for its group s - 1,
// meets barrier s + 1 and resolves group s + 1 into gn; steps 2 and 3 issue its
// slots 0 .. 3 (activation stage s + 3 into the slot of stage s), read steps 0 and
// 1 of stage s + 1 and its chunk (wn), and dequantize its step 0, leaving the entry
// state of stage s + 1.  The last stage (!NEXT) issues nothing.  ODD: s is odd.
template <int BITS, bool TAIL, bool GS128, int DQ, bool NEXT, bool ODD>
__device__ __forceinline__ void run_stage(Ctx<BITS>& c, int s, u4 (&a)[4][4], u4& bw, const WStage<BITS>& wc,
                                          WStage<BITS>& wn, const Group& gc, Group& gn, f16x (&acc)[4]) {
    const int nslot = c.cslot == NSTAGE - 1 ? 0 : c.cslot + 1;
#pragma unroll
    for (int kq = 0; kq < KSTEPS; ++kq) {
        if (kq + 2 < KSTEPS) read_a(c.lds, c.cslot, kq + 2, c.ci, a[(kq + 2) & 3]);
        else if (NEXT) read_a(c.lds, nslot, kq - 2, c.ci, a[(kq + 2) & 3]);
        if (NEXT && kq == 2) read_w<BITS, GS128>(c.A, c.lds, s + 1, c.ci, wn);
        u4 bwn = bw;
        if (kq + 1 < KSTEPS) bwn = dequant_octet<BITS, DQ>(wc, kq + 1, c.g);
        else if (NEXT) bwn = dequant_octet<BITS, DQ>(wn, 0, c.g);
        mma_step<(DQ >= 2)>(a[kq & 3], bw, acc);
        bw = bwn;
        if (NEXT && kq <= 1) {
            issue_slot<BITS, TAIL, !ODD>(c.L, gc, 4 + 2 * kq, c.lds);
            issue_slot<BITS, TAIL, !ODD>(c.L, gc, 5 + 2 * kq, c.lds);
        }
        if (NEXT && kq == 1) {
            wait_group<BITS, !ODD>();             // group s (parity of s) may stay in flight
            barrier_lds();                        // stage s + 1 published
            group_at<BITS, TAIL, ODD>(c.L, c.sc, s + 1, gn);
        }
        if (NEXT && kq >= 2) {
            issue_slot<BITS, TAIL, ODD>(c.L, gn, 2 * (kq - 2), c.lds);
            issue_slot<BITS, TAIL, ODD>(c.L, gn, 2 * (kq - 2) + 1, c.lds);
        }
    }
    c.cslot = nslot;
}

// The stages, unrolled by two so the chunk and group registers of stage s and
// stage s + 1 alternate without copies and the load-group parity is static; the
// last stage is peeled.
template <int BITS, bool TAIL, bool GS128, int DQ>
__device__ __forceinline__ void compute_loop(Ctx<BITS>& c, int nst, Group& g0, f16x (&acc)[4]) {
    u4 a[4][4], bw;
    WStage<BITS> w0, w1;
    Group g1;
    read_a(c.lds, 0, 0, c.ci, a[0]);
    read_a(c.lds, 0, 1, c.ci, a[1]);
    read_w<BITS, GS128>(c.A, c.lds, 0, c.ci, w0);
    bw = dequant_octet<BITS, DQ>(w0, 0, c.g);
    int s = 0;
    for (; s + 2 < nst; s += 2) {
        run_stage<BITS, TAIL, GS128, DQ, true, false>(c, s, a, bw, w0, w1, g0, g1, acc);
        run_stage<BITS, TAIL, GS128, DQ, true, true>(c, s + 1, a, bw, w1, w0, g1, g0, acc);
    }
    if (s + 1 < nst) {
        run_stage<BITS, TAIL, GS128, DQ, true, false>(c, s, a, bw, w0, w1, g0, g1, acc);
        run_stage<BITS, TAIL, GS128, DQ, false, true>(c, s + 1, a, bw, w1, w0, g1, g0, acc);
    } else {
        run_stage<BITS, TAIL, GS128, DQ, false, false>(c, s, a, bw, w0, w1, g0, g1, acc);
    }
}

// GU: the gate-up GEMM.  A tile covers 64 outputs n0 .. n0 + 63: slabs 0 and 1 are the
// gate's columns n0 + 32 (slab & 1) .., slabs 2 and 3 the up's of the same outputs, so
// each output's two sums end in one workgroup.
template <int BITS, bool TAIL, bool GS128, int DT, bool GU>
__global__ void __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemm_f16_kernel(const GemmArgs A) {
    extern __shared__ __attribute__((aligned(16))) char lds_raw[];
    lds_t* lds = (lds_t*)lds_raw;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int slab = wave & 3, kh = wave >> 2;    // column slab, k half of every stage
    const int mtiles = (A.M + BM - 1) / BM;
    constexpr int TN = GU ? BN / 2 : BN;          // outputs per tile
    const int m0 = (blockIdx.x % mtiles) * BM, n0 = (blockIdx.x / mtiles) * TN;
    const int nst = (A.K + BK - 1) / BK;
    const bool up = GU && slab >= 2;              // the slab's tensor
    const int c0 = n0 + (GU ? (slab & 1) : slab) * 32;   // the slab's first column

    // prologue: the zero scan's loads, then weight block 0, window 0 and stages 0, 1
    ZScan zs;
    scan_issue(A, up ? A.z2 : A.z, c0, lane, zs);
    Loads<BITS> L;
    loads_setup<BITS, GU>(A, m0, n0, nst, wave, lane, L);
    Sched sc;
    sc.nst = nst;
    sc.nblk = (nst + WBLK - 1) / WBLK;
    sc.rp = A.gs >> 5;
    sc.aslot = 0;
    sc.blk_in_win = 0;
    sc.win = 0;
    Group g0;
    group_at<BITS, TAIL, true>(L, sc, -2, g0);    // stage 0, block 0, window 0
    issue_group<BITS, TAIL, true>(L, g0, lds);
    group_at<BITS, TAIL, false>(L, sc, -1, g0);   // stage 1
    issue_group<BITS, TAIL, false>(L, g0, lds);

    // the 128 x 32 slab at columns slab * 32 of the tile, k half kh of every stage
    const int r32 = lane & 31;
    const int hk = lane >> 5;
    ColInfo ci;
    {
        const int r = slab * 32 + r32;            // the column's row of the tile's weight buffers
        const int col = min(c0 + r32, A.N - 1);
        const uintptr_t row = reinterpret_cast<uintptr_t>(up ? A.w2 : A.w) + (uintptr_t)col * A.wpr * 4;
        ci.cix = 2 * hk + kh;
        ci.wlane = W_OFF + r * WGeo<BITS>::PITCH + (int)(row & 15) + ci.cix * (4 * BITS);
        ci.cg = (long)col * A.G;
        ci.soff = r * 32;
        ci.szlane = SZ_OFF<BITS> + r * 32 + 2 * (int)(ci.cg & 7);
#pragma unroll
        for (int kq = 0; kq < KSTEPS; ++kq)
            ci.aaddr[kq] = A_OFF + r32 * APR * 16 + 16 * ((8 * hk + KSTEPS * kh + kq) ^ swz(r32));
    }
    const bool fast = scan_finish<DT>(A, up ? A.z2 : A.z, c0, lane, zs);

    f16x acc[4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[a][v] = 0.f;

    vmcnt<A_Q>();                                 // block 0, window 0 and stage 0 landed
    barrier_lds();                                // barrier 0: published
    group_at<BITS, TAIL, true>(L, sc, 0, g0);
#pragma unroll
    for (int k = 0; k < 4; ++k) issue_slot<BITS, TAIL, true>(L, g0, k, lds);

    Ctx<BITS> c{A, lds, ci, magic_vreg(), L, sc, 0};
    constexpr int DQ0 = DT == DT_BF16 ? 2 : 0;
    if (fast) compute_loop<BITS, TAIL, GS128, DQ0 + 1>(c, nst, g0, acc);
    else compute_loop<BITS, TAIL, GS128, DQ0>(c, nst, g0, acc);
    vmcnt<0>();                                   // the surplus loads land before the LDS is reused

    // both k halves write their partial sums row-major into a tile image of their own (fp32,
    // pitch SUM_PITCH: 4 pitches = 32 banks apart, so the two row groups a store instruction
    // touches hit distinct banks; tile column slab * 32 + r32 -- for GU the gate's 64 columns,
    // then the up's); the stage slots and buffers are free once every wave is past its last stage
    typedef __attribute__((address_space(3))) float lf;
    barrier_lds();
    lf* img = reinterpret_cast<lf*>(lds + kh * SUM_IMG);
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        // D layout of a 32x32 block: lane (j = lane & 31, h = lane >> 5), register 4q + r holds
        // row 8q + 4h + r, column j
#pragma unroll
        for (int v = 0; v < 16; ++v)
            img[(32 * a + 8 * (v >> 2) + 4 * hk + (v & 3)) * SUM_PITCH + slab * 32 + r32] = acc[a][v];
    }
    barrier_lds();
    const lf* sums = reinterpret_cast<const lf*>(lds);

    // every thread finishes runs of 8 consecutive outputs of a row: 16-byte stores when the
    // output's rows are 16-byte aligned, else element stores
    const bool vec = (reinterpret_cast<uintptr_t>(A.out) & 15) == 0 && (A.N & 7) == 0;
    constexpr int RUNS = TN / 8;                  // runs per tile row
    constexpr int ROWS = THREADS / RUNS;          // tile rows per pass
    const int tc = 8 * (tid % RUNS);            // the thread's first tile column
    const int n = n0 + tc;
    float bias[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) bias[e] = (!GU && A.b && n + e < A.N) ? load_f<DT>(A.b, n + e) : 0.f;
#pragma unroll
    for (int pass = 0; pass < BM / ROWS; ++pass) {
        const int r = pass * ROWS + tid / RUNS;
        const int m = m0 + r;
        typedef __attribute__((address_space(3))) const f4x lf4;
        const f4x s0 = *reinterpret_cast<lf4*>(sums + r * SUM_PITCH + tc) +
                       *reinterpret_cast<lf4*>(sums + SUM_IMG / 4 + r * SUM_PITCH + tc);
        const f4x s1 = *reinterpret_cast<lf4*>(sums + r * SUM_PITCH + tc + 4) +
                       *reinterpret_cast<lf4*>(sums + SUM_IMG / 4 + r * SUM_PITCH + tc + 4);
        float y[8];
        if constexpr (GU) {
            const f4x u0 = *reinterpret_cast<lf4*>(sums + r * SUM_PITCH + 64 + tc) +
                           *reinterpret_cast<lf4*>(sums + SUM_IMG / 4 + r * SUM_PITCH + 64 + tc);
            const f4x u1 = *reinterpret_cast<lf4*>(sums + r * SUM_PITCH + 64 + tc + 4) +
                           *reinterpret_cast<lf4*>(sums + SUM_IMG / 4 + r * SUM_PITCH + 64 + tc + 4);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                // the two GEMMs' outputs -- act(sum + 0) rounded, as a GEMM without bias forms
                // them (signed zeros included) -- and their product: both factors are dtype
                // values, so the product is exact in fp32 and the store rounds once
                const float gv = Dt<DT>::to_f(Dt<DT>::from_f(silu((e < 4 ? s0[e] : s1[e - 4]) + 0.f)));
                const float uv = Dt<DT>::to_f(Dt<DT>::from_f((e < 4 ? u0[e] : u1[e - 4]) + 0.f));
                y[e] = gv * uv;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) y[e] = apply_act((e < 4 ? s0[e] : s1[e - 4]) + bias[e], A.act);
        }
        if (m >= A.M) continue;
        if (vec) {
            if (n < A.N) {
                uint32_t o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    o[e] = raw16<DT>(y[2 * e]) | (raw16<DT>(y[2 * e + 1]) << 16);
                *reinterpret_cast<u4*>(reinterpret_cast<uint16_t*>(A.out) + (long)m * A.N + n) =
                    u4{o[0], o[1], o[2], o[3]};
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (n + e < A.N) store_f<DT>(A.out, (long)m * A.N + n + e, y[e]);
        }
    }
}

template <int BITS, int DT, bool GU>
const void* kernel_for(bool tail, bool gs128) {
    return tail ? (gs128 ? reinterpret_cast<const void*>(&gemm_f16_kernel<BITS, true, true, DT, GU>)
                       : reinterpret_cast<const void*>(&gemm_f16_kernel<BITS, true, false, DT, GU>))
                : (gs128 ? reinterpret_cast<const void*>(&gemm_f16_kernel<BITS, false, true, DT, GU>)
                       : reinterpret_cast<const void*>(&gemm_f16_kernel<BITS, false, false, DT, GU>));
}

template <int DT, bool GU>
const void* kernel_for_bits(int bits, bool tail, bool gs128) {
    return bits == 2 ? kernel_for<2, DT, GU>(tail, gs128)
                     : (bits == 3 ? kernel_for<3, DT, GU>(tail, gs128) : kernel_for<4, DT, GU>(tail, gs128));
}

template <bool GU>
const void* kernel_for_dt(int dt, int bits, bool tail, bool gs128) {
    return dt == DT_BF16 ? kernel_for_bits<DT_BF16, GU>(bits, tail, gs128)
                         : kernel_for_bits<DT_F16, GU>(bits, tail, gs128);
}

}  // namespace

bool gemm_f16_supported(const GemmArgs& A) {
    // 16-byte activation pieces, whole octets before K, 16-byte aligned packed /
    // scale / zero bases (the loads' aligned pieces and the zero scan), windows of
    // 8 groups spanning whole weight blocks (group size a multiple of 32), tensors
    // within the 32-bit range of a buffer descriptor
    const auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const long lim = 0x7FFFFFFF;                 // buffer offsets and ranges are 32-bit
    const bool up_ok = !A.w2 || (al16(A.w2) && al16(A.s2) && al16(A.z2));
    return A.K % 8 == 0 && A.K >= 8 && A.gs % 32 == 0 && al16(A.x) && al16(A.w) && al16(A.s) && al16(A.z) && up_ok &&
           (long)A.M * A.K * 2 < lim && (long)A.N * A.wpr * 4 < lim && (long)A.N * A.G * 2 < lim;
}

hipError_t launch_gemm_f16(const GemmArgs& A, int dt, hipStream_t stream, bool gate_up) {
    const bool tail = A.K % BK != 0, gs128 = A.gs == 128;
    const void* f = gate_up ? kernel_for_dt<true>(dt, A.bits, tail, gs128)
                            : kernel_for_dt<false>(dt, A.bits, tail, gs128);
    const int lds = A.bits == 2 ? LDS_BYTES<2> : (A.bits == 3 ? LDS_BYTES<3> : LDS_BYTES<4>);
    hipError_t e = lds_limit_raise(f, lds);
    if (e != hipSuccess) return e;
    const int tn = gate_up ? BN / 2 : BN;
    const int tiles = ((A.M + BM - 1) / BM) * ((A.N + tn - 1) / tn);
    void* args[] = {const_cast<GemmArgs*>(&A)};
    return launch(f, dim3(tiles), dim3(THREADS), args, (size_t)lds, stream);
}

}  // namespace cbk
