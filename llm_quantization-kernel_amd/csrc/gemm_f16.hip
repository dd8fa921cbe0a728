// gemm_f16.hip -- fp16 prefill packed GEMM on gfx950: out[M,N] = act(x . W-hat^T + bias).
//
// Replaces cb_gemm_tc_kernel (Kernel/csrc/packed_gemm.cu:12-117) for fp16
// activations, with the reference's weight rounding W-hat = RN_fp16((q - z) * s)
// (packed_gemm.cu:56,60).
//
// Tile: 128 x 128 outputs per workgroup of six waves.  All global traffic is
// direct-to-LDS loads issued by two loader waves; the four compute waves read LDS
// only, so their waits are LDS counts the compiler tracks exactly.
//   activation loader (wave 4): the activation tile, 128 rows x 64 codes per stage,
//     into a ring of NSTAGE stages (16 instructions of 1 KB per stage, XOR-swizzled
//     16-byte pieces: piece p of row r at slot r * 8 + (p ^ ((r >> 1) & 7))),
//     NSTAGE - 1 stages ahead; one workgroup barrier publishes each stage.
//   weight loader (wave 5): the packed tile in blocks of WBLK stages (256 codes =
//     8 chunks of each of the 128 rows), double-buffered one block ahead.  A row's
//     block is fetched as the 16-byte-aligned pieces that cover it (its start has
//     phase (row address & 15) within the first), with an odd piece count per row
//     as the LDS pitch, so the compute lanes' reads of 32 rows are free of bank
//     conflicts.  Scales and zeros likewise: per row and tensor a 32-byte aligned
//     span holding the 8 groups of a window (gs / 32 blocks), double-buffered.
//     Aligned pieces never straddle a page, so a piece holding any valid byte is
//     readable; pieces wholly past a tensor's end re-read its last piece.
//   compute (waves 0-3, a 2 x 2 grid of 64 x 64 wave tiles): each wave reads its
//     activation operands and its columns' packed chunks from LDS and dequantizes
//     the chunks straight into the B operands of v_mfma_f32_32x32x16_f16; the
//     dequantized tile never touches LDS.
//
// Weight rounding: the codes of a pair are OR-ed into 0x6400 (1024 + q, exact),
// then (h - (1024 + z)) * s in packed fp16 when every zero point of the tile is an
// integer below 1024 in magnitude (the reference quantizer's; the weight loader
// scans the tile's zeros once): the difference is an exact integer and the product
// rounds once, exactly RN_fp16((q - z) * s).  Other zero points take the fp32
// product.  Codes at k >= K dequantize to zero, so the clamped activation reads and
// the tail of the last weight block contribute nothing.
//
// MFMA operand lane map (32x32x16): lane (r = lane & 31, h = lane >> 5) holds
// row / column r and 8 k-values of the step.  The k order within a stage is free
// as long as both operands use it: step ks of a stage gives lane half h the codes
// 32 h + 8 ks .. +7 (octet ks of chunk 2 s + h), so each compute lane needs one
// packed chunk and one (scale, zero) pair per column per stage.
#include "cbk_decode.hpp"
#include "cbk_device.hpp"
#include "cbk_kernels.hpp"

namespace cbk {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int NSTAGE = 3;                    // activation stages in LDS
constexpr int THREADS = 448;                 // 4 compute waves + 2 activation loaders + 1 weight loader
constexpr int TILE = BM * BK * 2;            // bytes of an activation stage (32 KB)
constexpr int APR = BK * 2 / 16;             // 16-byte pieces per activation row of a stage
constexpr int A_INSTR = TILE / 1024 / 2;     // instructions per activation loader per stage
constexpr int WBLK = 2;                      // stages per weight block (256 codes)
constexpr int SZG = 8;                       // groups per scale / zero window
constexpr int SZ_INSTR = 2 * BN * 2 / 64;    // window: [tensor][row] x two 16-byte pieces
constexpr int SZ_BUF = 2 * BN * 32;

// Weight block geometry: a row's block is 32 * BITS bytes at phase 0 (W4), 0 / 8
// (W2) or 0 / 4 / 8 / 12 (W3) within its first aligned piece.
template <int BITS> struct WGeo {
    static constexpr int PPR = BITS == 4 ? 9 : (BITS == 3 ? 7 : 5);   // pieces per row, odd
    static constexpr int PITCH = 16 * PPR;
    static constexpr int BUF = BN * PITCH;
    static constexpr int INSTR = BN * PPR / 64;
};

constexpr int A_OFF = 0;
constexpr int W_OFF = NSTAGE * TILE;
template <int BITS> constexpr int SZ_OFF = W_OFF + 2 * WGeo<BITS>::BUF;
template <int BITS> constexpr int FLAG_OFF = SZ_OFF<BITS> + 2 * SZ_BUF;   // tile zeros allow the fp16 form
template <int BITS> constexpr int LDS_BYTES = FLAG_OFF<BITS> + 16;

__device__ __forceinline__ int swz(int r) { return r & (APR - 1); }

template <int N>
__device__ __forceinline__ void vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (((N >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier without a memory fence: __syncthreads() would make the compiler
// wait for every in-flight load of the wave (vmcnt(0)), draining the prefetch.
// This only completes the wave's own LDS traffic (lgkmcnt(0)) before the barrier.
__device__ __forceinline__ void barrier_lds() {
    __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4));    // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
}

__device__ __forceinline__ void dma16(const void* g, char* lds) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds, 16, 0, 0);
}

// ------------------------------------------------------------------ activation loader
// Loader wave h moves instructions t = 8 h .. 8 h + 7 of each stage; lane l of
// instruction t moves slot q = 64 t + l: row q >> 3, logical piece (q & 7) ^ swz(row).
// The loads go through a buffer descriptor over the activations: the lane's offset
// (row clamped to M, piece) is fixed, the stage's column offset is a scalar, so a
// stage costs no VALU.  Pieces past K read on into the next row (or, past the
// tensor, zero), which meets zero weights -- except in the last stage, where pieces
// at k >= K read as zero (K % 8 == 0, so a piece is wholly inside or outside), so
// whatever the weight tile holds there contributes nothing.
struct ALoader {
    __amdgpu_buffer_rsrc_t rsrc;
    int voff[A_INSTR];
    int rowoff[A_INSTR];          // byte offset of the lane's row
    int pk[A_INSTR];              // k of the lane's piece within a stage
    int t0;                       // first instruction of this loader
};

__device__ __forceinline__ void a_setup(const GemmArgs& A, int m0, int half, int lane, ALoader& d) {
    d.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(A.x), (short)0, A.M * A.K * 2, 0x00020000);
    d.t0 = A_INSTR * half;
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i) {
        const int q = 64 * (d.t0 + i) + lane;
        const int r = q / APR, p = (q & (APR - 1)) ^ swz(r);
        d.rowoff[i] = min(m0 + r, A.M - 1) * A.K * 2;
        d.pk[i] = 8 * p;
        d.voff[i] = d.rowoff[i] + 16 * p;
    }
}

// A byte offset past every buffer descriptor's range: such loads return zero.
constexpr int OOR = 0x7FFFFFF0;

// Stage s into slot s % NSTAGE; a stage past the last is issued as the last one,
// so every iteration issues A_INSTR loads and the waits are constants.
__device__ __forceinline__ void issue_a(const GemmArgs& A, const ALoader& d, int s, int nst, char* lds) {
    char* dst = lds + A_OFF + (s % NSTAGE) * TILE + d.t0 * 1024;
    s = min(s, nst - 1);
    if (s == nst - 1 && A.K % BK != 0) {
#pragma unroll
        for (int i = 0; i < A_INSTR; ++i) {
            const int k = BK * s + d.pk[i];
            __builtin_amdgcn_raw_ptr_buffer_load_lds(d.rsrc, (lds_void*)(dst + i * 1024), 16,
                                                     k < A.K ? d.rowoff[i] + 2 * k : OOR, 0, 0, 0);
        }
    } else {
#pragma unroll
        for (int i = 0; i < A_INSTR; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(d.rsrc, (lds_void*)(dst + i * 1024), 16, d.voff[i], BK * 2 * s,
                                                     0, 0);
    }
}

// ------------------------------------------------------------------ weight loader
// Block j of the tile into buffer j & 1: lane l of instruction t moves piece
// q = 64 t + l, row q / PPR, piece q % PPR of the row's aligned span.  Scale /
// zero window w: instruction t < 4 the scales, else the zeros; lane l moves piece
// q & 1 of tile row (q >> 1) & 127's span, the 16 halves from floor8(col * G) + 8 w
// (floor8(col * G + 8 w), as 8 w is a multiple of 8).  Buffer descriptors over the
// packed words, scales and zeros: the lane's offsets are fixed and the block /
// window offset is a scalar; reads past a tensor return zero (they are never used).
template <int BITS>
struct WLoader {
    __amdgpu_buffer_rsrc_t wr, sr, zr;
    int woff[WGeo<BITS>::INSTR];
    int szoff[SZ_INSTR];
};

template <int BITS>
__device__ __forceinline__ void w_setup(const GemmArgs& A, int n0, int lane, WLoader<BITS>& d) {
    using G = WGeo<BITS>;
    d.wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(A.w), (short)0, A.N * A.wpr * 4, 0x00020000);
    d.sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(A.s), (short)0, A.N * A.G * 2, 0x00020000);
    d.zr = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(A.z), (short)0, A.N * A.G * 2, 0x00020000);
#pragma unroll
    for (int t = 0; t < G::INSTR; ++t) {
        const int q = 64 * t + lane;
        const int r = q / G::PPR, p = q - r * G::PPR;
        d.woff[t] = ((min(n0 + r, A.N - 1) * A.wpr * 4) & ~15) + 16 * p;
    }
#pragma unroll
    for (int t = 0; t < SZ_INSTR; ++t) {
        const int q = 64 * t + lane;
        const int r = (q >> 1) & (BN - 1), p = q & 1;
        d.szoff[t] = ((min(n0 + r, A.N - 1) * A.G) & ~7) * 2 + 16 * p;
    }
}

template <int BITS>
__device__ __forceinline__ void issue_w(const WLoader<BITS>& d, int j, char* lds) {
    using G = WGeo<BITS>;
    char* dst = lds + W_OFF + (j & 1) * G::BUF;
#pragma unroll
    for (int t = 0; t < G::INSTR; ++t)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(d.wr, (lds_void*)(dst + t * 1024), 16, d.woff[t], j * (32 * BITS), 0,
                                                 0);
}

template <int BITS>
__device__ __forceinline__ void issue_sz(const WLoader<BITS>& d, int w, char* lds) {
    char* dst = lds + SZ_OFF<BITS> + (w & 1) * SZ_BUF;
#pragma unroll
    for (int t = 0; t < SZ_INSTR; ++t)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(t < SZ_INSTR / 2 ? d.sr : d.zr, (lds_void*)(dst + t * 1024), 16,
                                                 d.szoff[t], 2 * SZG * w, 0, 0);
}

__device__ __forceinline__ _Float16 half_of(uint32_t v) {
    return __builtin_bit_cast(_Float16, (uint16_t)v);
}

// An fp16 zero point allows the packed-fp16 form: an integer below 1024 in magnitude.
__device__ __forceinline__ bool zero_is_small_int(uint32_t zbits) {
    const float zf = (float)half_of(zbits);
    return zf == __builtin_rintf(zf) && __builtin_fabsf(zf) < 1024.f;
}

// Whether every zero point of tile columns [n0, min(n0 + BN, N)) -- a contiguous
// range of the zeros tensor, whose start is 16-byte aligned -- allows the
// packed-fp16 form.
__device__ __forceinline__ bool scan_zeros(const GemmArgs& A, int n0, int lane) {
    const uint16_t* z = reinterpret_cast<const uint16_t*>(A.z);
    const long beg = (long)n0 * A.G, end = (long)min(n0 + BN, A.N) * A.G;   // beg % 8 == 0
    bool ok = true;
    for (long i = beg + 8 * lane; i < end; i += 8 * 64) {
        if (i + 8 <= end) {
            const u4 v = *reinterpret_cast<const u4*>(z + i);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                ok &= zero_is_small_int(v[j] & 0xFFFFu) & zero_is_small_int(v[j] >> 16);
        } else {
            for (long e = i; e < end; ++e) ok &= zero_is_small_int(z[e]);
        }
    }
    return __builtin_amdgcn_ballot_w64(!ok) == 0;
}

// ------------------------------------------------------------------ compute
// A compute wave owns a 128 x 32 slab of the tile: every row, columns
// 32 wn .. 32 wn + 31 (wn = wave), so each column is dequantized by exactly one
// wave.  Lane (r32 = lane & 31, hk = lane >> 5) holds column r32's B operand and
// the A operands of rows 32 a + r32 (a < 4).  Step ks of a stage gives lane half hk
// the codes 32 hk + 8 ks .. +7 (octet ks of chunk 2 s + hk), so a lane needs one
// packed chunk and one (scale, zero) pair per stage.

// The lane's two packed chunks of a stage and their scales and zeros as raw fp16 bits.
template <int BITS>
struct WStage {
    uint32_t w[2][BITS];
    uint32_t s[2], z[2];
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

// B operand of step ks: the lane's codes 64 hk + 8 ks .. +7 of its column (octet
// ks & 3 of its chunk ks >> 2).  FAST: every zero point of the tile is an integer
// below 1024 in magnitude.
template <int BITS, bool FAST>
__device__ __forceinline__ u4 dequant_octet(const WStage<BITS>& r, int ks, uint32_t g) {
    const int c = ks >> 2;
    const float zf = (float)half_of(r.z[c]);
    const _Float16 cz = (_Float16)(1024.f + zf);      // exact when FAST: an integer below 2048
    const _Float16 sh = half_of(r.s[c]);
    const h2 c2 = {cz, cz}, s2 = {sh, sh};
    const float sf = (float)sh;
    uint32_t h[4];
    Octet<BITS>::run(r.w[c], ks & 3, g, h);
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

// A operands of step ks of stage s: af[a] = row 32 a + r32, codes 64 hk + 8 ks .. +7.
__device__ __forceinline__ void read_a(const char* lds, int s, int ks, int aoff, int hk, int sw, u4 (&af)[4]) {
    const u4* at = reinterpret_cast<const u4*>(lds + A_OFF + (s % NSTAGE) * TILE);
    const int p = (8 * hk + ks) ^ sw;
#pragma unroll
    for (int a = 0; a < 4; ++a) af[a] = at[aoff + a * 32 * APR + p];     // 32 rows apart
}

// Per-lane constants of a compute wave's column (tile row wn * 32 + r32).
struct ColInfo {
    int woff;         // LDS byte of the row in a weight buffer (row * PITCH + phase)
    int soff;         // LDS byte of the row's scale span in a window buffer
    long cg;          // col * G
};

// The lane's chunks (4 s + 2 hk + c, c < 2: chunks 4 (s % WBLK) + 2 hk + c of block
// s / WBLK) and their (scale, zero) of stage s, as the weight loader filled its
// buffer and window.
template <int BITS>
__device__ __forceinline__ void read_w(const GemmArgs& A, const char* lds, int s, const ColInfo& ci, int hk,
                                       WStage<BITS>& r) {
    const int j = s / WBLK;
    const char* p = lds + W_OFF + (j & 1) * WGeo<BITS>::BUF + (4 * (s % WBLK) + 2 * hk) * (4 * BITS) + ci.woff;
    if constexpr (BITS == 4) {
        const u4 v0 = *reinterpret_cast<const u4*>(p), v1 = *reinterpret_cast<const u4*>(p + 16);
        r.w[0][0] = v0.x; r.w[0][1] = v0.y; r.w[0][2] = v0.z; r.w[0][3] = v0.w;
        r.w[1][0] = v1.x; r.w[1][1] = v1.y; r.w[1][2] = v1.z; r.w[1][3] = v1.w;
    } else if constexpr (BITS == 2) {
        const u4 v = *reinterpret_cast<const u4*>(p);
        r.w[0][0] = v.x; r.w[0][1] = v.y; r.w[1][0] = v.z; r.w[1][1] = v.w;
    } else {
        const u2 v0 = *reinterpret_cast<const u2*>(p), v1 = *reinterpret_cast<const u2*>(p + 8);
        const u2 v2 = *reinterpret_cast<const u2*>(p + 16);
        r.w[0][0] = v0.x; r.w[0][1] = v0.y; r.w[0][2] = v1.x;
        r.w[1][0] = v1.y; r.w[1][1] = v2.x; r.w[1][2] = v2.y;
    }
    const int w = (int)(fdiv((uint32_t)(j * 256), A.divG) >> 3);           // j / (gs / 32)
    const char* sb = lds + SZ_OFF<BITS> + (w & 1) * SZ_BUF;
    const long span = (ci.cg + SZG * w) & ~7L;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int gi = (int)fdiv((uint32_t)((4 * s + 2 * hk + c) * 32), A.divG);
        const uint16_t* q = reinterpret_cast<const uint16_t*>(sb + ci.soff) + (int)(ci.cg + gi - span);
        r.s[c] = q[0];
        r.z[c] = q[BN * 16];      // the zeros follow the scales' 128 rows x 32 bytes
    }
}

// One k-step: 4 MFMAs of 32 x 32 x 16 (rows 32 a .. of the slab, the lane's column).
__device__ __forceinline__ void mma_step(const u4 (&af)[4], const u4& bw, f16x (&acc)[4]) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
        acc[a] = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const h8*>(&af[a]),
                                                        *reinterpret_cast<const h8*>(&bw), acc[a], 0, 0, 0);
}

// One stage, as a software pipeline over its 8 k-steps: the A operands of step ks
// are read two steps ahead (a[ks & 3] of four rotating sets) and its B operand
// dequantized one step ahead, so each step's 4 MFMAs find their operands in
// registers while the dequant VALU of the next step and the LDS reads of the step
// after it go out between them.  On entry a[0], a[1] hold steps 0 and 1, bw step
// 0, wc the chunks of stage s.  NEXT: the wave meets barrier s + 1 after step 5 --
// every read of stage s's activation slot has been issued by then, and
// barrier_lds waits for them, so the loaders may refill it -- then reads steps 0
// and 1 of stage s + 1 and its chunks (wn), and dequantizes its step 0, leaving
// the entry state of stage s + 1.
template <int BITS, bool FAST, bool NEXT>
__device__ __forceinline__ void run_stage(const GemmArgs& A, const char* lds, int s, const ColInfo& ci, int hk,
                                          int sw, int aoff, uint32_t g, u4 (&a)[4][4], u4& bw,
                                          const WStage<BITS>& wc, WStage<BITS>& wn, f16x (&acc)[4]) {
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
        if (ks + 2 < 8) read_a(lds, s, ks + 2, aoff, hk, sw, a[(ks + 2) & 3]);
        else if (NEXT) read_a(lds, s + 1, ks - 6, aoff, hk, sw, a[(ks + 2) & 3]);
        if (NEXT && ks == 6) read_w<BITS>(A, lds, s + 1, ci, hk, wn);
        u4 bwn = bw;
        if (ks + 1 < 8) bwn = dequant_octet<BITS, FAST>(wc, ks + 1, g);
        else if (NEXT) bwn = dequant_octet<BITS, FAST>(wn, 0, g);
        mma_step(a[ks & 3], bw, acc);
        bw = bwn;
        if (NEXT && ks == 5) barrier_lds();       // stage s + 1 published
    }
}

// The compute waves' stages, unrolled by two so the chunk registers of stage s and
// stage s + 1 alternate without copies; the last stage is peeled.
template <int BITS, bool FAST>
__device__ __forceinline__ void compute_loop(const GemmArgs& A, const char* lds, int nst, const ColInfo& ci, int hk,
                                             int sw, int aoff, uint32_t g, f16x (&acc)[4]) {
    u4 a[4][4], bw;
    WStage<BITS> w0, w1;
    barrier_lds();                                // stage 0 published
    read_a(lds, 0, 0, aoff, hk, sw, a[0]);
    read_a(lds, 0, 1, aoff, hk, sw, a[1]);
    read_w<BITS>(A, lds, 0, ci, hk, w0);
    bw = dequant_octet<BITS, FAST>(w0, 0, g);
    int s = 0;
    for (; s + 2 < nst; s += 2) {
        run_stage<BITS, FAST, true>(A, lds, s, ci, hk, sw, aoff, g, a, bw, w0, w1, acc);
        run_stage<BITS, FAST, true>(A, lds, s + 1, ci, hk, sw, aoff, g, a, bw, w1, w0, acc);
    }
    if (s + 1 < nst) {
        run_stage<BITS, FAST, true>(A, lds, s, ci, hk, sw, aoff, g, a, bw, w0, w1, acc);
        run_stage<BITS, FAST, false>(A, lds, s + 1, ci, hk, sw, aoff, g, a, bw, w1, w0, acc);
    } else {
        run_stage<BITS, FAST, false>(A, lds, s, ci, hk, sw, aoff, g, a, bw, w0, w1, acc);
    }
}

template <int BITS>
__global__ void __launch_bounds__(THREADS) gemm_f16_kernel(const GemmArgs A) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int mtiles = (A.M + BM - 1) / BM;
    const int m0 = (blockIdx.x % mtiles) * BM, n0 = (blockIdx.x / mtiles) * BN;
    const int nst = (A.K + BK - 1) / BK;

    if (wave == 4 || wave == 5) {
        // activation loaders: stages s+1 .. s+NSTAGE-2 stay in flight while stage s is
        // published
        ALoader da;
        a_setup(A, m0, wave - 4, lane, da);
        for (int j = 0; j < NSTAGE - 1; ++j) issue_a(A, da, j, nst, lds);
        barrier_lds();                            // weight block 0 and the zero-point flag
        for (int s = 0; s < nst; ++s) {
            vmcnt<A_INSTR * (NSTAGE - 2)>();      // this loader's half of stage s landed
            barrier_lds();                        // publish stage s; every wave is past stage s-1
            issue_a(A, da, s + NSTAGE - 1, nst, lds);   // into the slot of stage s-1
        }
        vmcnt<0>();                               // the surplus stages land before the wave ends
        return;
    }
    if (wave == 6) {
        // weight loader: block j + 1 (and the scale window it starts) is issued at
        // the first barrier of block j and has landed before the first barrier of
        // block j + 1
        const int nblk = (nst + WBLK - 1) / WBLK, rp = A.gs >> 5;
        WLoader<BITS> dw;
        w_setup<BITS>(A, n0, lane, dw);
        issue_w<BITS>(dw, 0, lds);
        issue_sz<BITS>(dw, 0, lds);
        const bool fast = scan_zeros(A, n0, lane);
        if (lane == 0) *reinterpret_cast<int*>(lds + FLAG_OFF<BITS>) = fast;
        vmcnt<0>();
        barrier_lds();                            // weight block 0 and the zero-point flag
        for (int s = 0; s < nst; ++s) {
            if (s % WBLK == 0) vmcnt<0>();        // block s / WBLK landed: published by barrier s
            barrier_lds();                        // every wave is past stage s-1
            if (s % WBLK == 0) {
                const int j = s / WBLK + 1;       // the next block: its buffer held block j - 2
                if (j < nblk) {
                    issue_w<BITS>(dw, j, lds);
                    if (j % rp == 0) issue_sz<BITS>(dw, j / rp, lds);
                }
            }
        }
        vmcnt<0>();
        return;
    }

    // compute wave: the 128 x 32 slab at columns wn * 32 of the tile
    const int wn = wave;
    const int r32 = lane & 31;
    const int hk = lane >> 5;
    ColInfo ci;
    {
        const int r = wn * 32 + r32;
        const int col = min(n0 + r, A.N - 1);
        const uintptr_t row = reinterpret_cast<uintptr_t>(A.w) + (uintptr_t)col * A.wpr * 4;
        ci.woff = r * WGeo<BITS>::PITCH + (int)(row & 15);
        ci.soff = r * 32;
        ci.cg = (long)col * A.G;
    }
    const uint32_t g = magic_vreg();

    f16x acc[4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[a][v] = 0.f;

    const int aoff = r32 * APR;                   // u4 index of row r32 in a stage
    const int sw = swz(r32);                      // rows are 32-aligned + r32

    barrier_lds();                                // weight block 0 and the zero-point flag
    if (__builtin_amdgcn_readfirstlane(*reinterpret_cast<const int*>(lds + FLAG_OFF<BITS>)))
        compute_loop<BITS, true>(A, lds, nst, ci, hk, sw, aoff, g, acc);
    else
        compute_loop<BITS, false>(A, lds, nst, ci, hk, sw, aoff, g, acc);

    // D layout of a 32x32 block: lane (j = lane & 31, h = lane >> 5), register
    // 4q + r holds row 8q + 4h + r, column j
    const int n = n0 + wn * 32 + r32;
    if (n >= A.N) return;
    const float bias = A.b ? load_f<DT_F16>(A.b, n) : 0.f;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int m = m0 + 32 * a + 8 * (v >> 2) + 4 * hk + (v & 3);
            if (m < A.M) store_f<DT_F16>(A.out, (long)m * A.N + n, apply_act(acc[a][v] + bias, A.act));
        }
    }
}

template <int BITS>
const void* kernel_for() {
    return reinterpret_cast<const void*>(&gemm_f16_kernel<BITS>);
}

template <int BITS>
int lds_for() {
    return LDS_BYTES<BITS>;
}

}  // namespace

bool gemm_f16_supported(const GemmArgs& A) {
    // 16-byte activation pieces, whole octets before K, 16-byte aligned packed /
    // scale / zero bases (the loaders' aligned pieces and the zero scan), windows of
    // 8 groups spanning whole weight blocks (group size a multiple of 32), tensors
    // within the 32-bit range of a buffer descriptor
    const auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const long lim = 0x7FFFFFFF;                 // buffer offsets and ranges are 32-bit
    return A.K % 8 == 0 && A.K >= 8 && A.gs % 32 == 0 && al16(A.x) && al16(A.w) && al16(A.s) && al16(A.z) &&
           (long)A.M * A.K * 2 < lim && (long)A.N * A.wpr * 4 < lim && (long)A.N * A.G * 2 < lim;
}

hipError_t launch_gemm_f16(const GemmArgs& A, hipStream_t stream) {
    const void* f = A.bits == 2 ? kernel_for<2>() : (A.bits == 3 ? kernel_for<3>() : kernel_for<4>());
    const int lds = A.bits == 2 ? lds_for<2>() : (A.bits == 3 ? lds_for<3>() : lds_for<4>());
    hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    const int tiles = ((A.M + BM - 1) / BM) * ((A.N + BN - 1) / BN);
    void* args[] = {const_cast<GemmArgs*>(&A)};
    return launch(f, dim3(tiles), dim3(THREADS), args, (size_t)lds, stream);
}

}  // namespace cbk
