// gemm_f16.hip -- fp16 prefill packed GEMM on gfx950: out[M,N] = act(x . W-hat^T + bias).
//
// Replaces cb_gemm_tc_kernel (Kernel/csrc/packed_gemm.cu:12-117) for fp16
// activations, with the reference's weight rounding W-hat = RN_fp16((q - z) * s)
// (packed_gemm.cu:56,60).
//
// Tile: 128 x 128 outputs per workgroup of eight waves in two roles, one of each
// per SIMD:
//   consumers (waves 0-3): stream the activation tile HBM -> LDS with
//     direct-to-LDS loads AHEAD stages ahead (explicit vmcnt waits), and run a
//     2 x 2 grid of 64 x 64 wave tiles, each 2 x 2 blocks of
//     v_mfma_f32_32x32x16_f16 with fp32 accumulation -- the 32x32 instruction
//     keeps the matrix core busy from a single wave, where 16x16 ones stall on
//     issue;
//   producers (waves 4-7): load the packed words and (scale, zero) of a
//     (column, chunk) per thread into a 3-stage register ring (plain vector
//     loads: these waves issue no direct-to-LDS loads, so the compiler's waits
//     stay exact) and dequantize stage s+2 into LDS while the consumers multiply
//     stage s.
// K runs in stages of 64 codes (two 32-code chunks); one barrier per stage.  The
// consumers multiply stage s from registers while they read stage s+1's operands
// from LDS, so the LDS latency hides behind the matrix core.
//
// Activation stage: 128 rows x 64 codes, 16-byte pieces into an XOR-swizzled tile
// (piece p of row r at slot r*8 + (p ^ ((r >> 1) & 7))), so the MFMA operand reads
// of 16 consecutive rows hit 16 distinct groups of 4 banks.  The dequantized B
// tile uses the same layout, in natural k order:
//   fast path (integer zero point, as the reference quantizer produces): the
//   codes of a pair are OR-ed into 0x6400 (1024 + q, exact), then
//   (h - (1024 + z)) * s in packed fp16 -- the difference is an exact integer and
//   the product rounds once, exactly RN_fp16((q - z) * s);
//   other zero points: (q - z) * s in fp32, rounded to fp16 (the reference's
//   fp32 arithmetic).
// Codes at k >= K dequantize to zero, so the clamped activation reads past K
// contribute nothing.
//
// LDS: 4 activation stages (64 KB) + 3 B tiles (48 KB).
#include "cbk_decode.hpp"
#include "cbk_device.hpp"
#include "cbk_kernels.hpp"

namespace cbk {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int NSTAGE = 4;                    // activation buffers: stages s .. s+3 live
constexpr int AHEAD = 3;                     // activation stages issued ahead of the one computed
constexpr int THREADS = 512;                 // 4 consumer + 4 producer waves
constexpr int TILE = BM * BK * 2;            // bytes of an activation stage or a B tile (16 KB)
constexpr int NB = 3;                        // B tiles: stage s (in registers), s+1 (read), s+2 (written)
constexpr int A_OFF = 0;
constexpr int B_OFF = NSTAGE * TILE;
constexpr int LDS_BYTES = B_OFF + NB * TILE;
constexpr int A_ISSUE = 4;                   // activation loads per consumer wave per stage

// 16-byte slot of piece p (0..7) of tile row r: r * 8 + (p ^ swz(r))
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }

template <int N>
__device__ __forceinline__ void vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (((N >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier without a memory fence: __syncthreads() would make the compiler
// wait for every in-flight direct-to-LDS load (vmcnt(0)), draining the prefetch.
// The stage waits are explicit (wait_groups); this only completes the wave's own
// LDS writes (lgkmcnt(0)) before the barrier.
__device__ __forceinline__ void barrier_lds() {
    __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4));    // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
}


// Activation sources of a consumer wave (cw = 0..3), fixed for the whole K loop:
// slot q = 256 cw + 64 t + lane -> row q >> 3, logical piece (q & 7) ^ swz(row).
struct ASrc {
    const _Float16* a[A_ISSUE];   // activation row (clamped to M)
    int ak[A_ISSUE];              // k of the piece within a stage
};

__device__ __forceinline__ void a_setup(const GemmArgs& A, int m0, int cw, int lane, ASrc& d) {
    const _Float16* x = reinterpret_cast<const _Float16*>(A.x);
#pragma unroll
    for (int t = 0; t < A_ISSUE; ++t) {
        const int q = 256 * cw + 64 * t + lane;
        const int r = q >> 3, p = (q & 7) ^ swz(r);
        d.a[t] = x + (long)min(m0 + r, A.M - 1) * A.K;
        d.ak[t] = 8 * p;
    }
}

// Issue activation stage s into slot `buf` (this wave's quarter).  Pieces past K
// re-read a valid piece (their codes dequantize to zero); a stage past the last is
// issued as the last one, into a slot whose stage is consumed, so every iteration
// issues A_ISSUE loads and the waits are constants.
__device__ __forceinline__ void issue_a(const GemmArgs& A, const ASrc& d, int s, int buf, char* lds, int cw, int nst) {
    s = min(s, nst - 1);
    char* abase = lds + A_OFF + buf * TILE + 256 * cw * 16;
#pragma unroll
    for (int t = 0; t < A_ISSUE; ++t)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(d.a[t] + min(BK * s + d.ak[t], A.K - 8)),
                                         (lds_void*)(abase + 64 * t * 16), 16, 0, 0);
}

// Packed words and (scale, zero) of one (column, chunk) of a stage, in registers.
template <int BITS>
struct WRegs {
    uint32_t w[BITS];
    _Float16 s, z;
};

template <int BITS>
__device__ __forceinline__ void load_w(const GemmArgs& A, const uint32_t* wrow, const _Float16* srow,
                                       const _Float16* zrow, int s, int c, WRegs<BITS>& r) {
    const int chunk = min(2 * s + c, A.C - 1);
    const uint32_t* p = wrow + chunk * BITS;
#pragma unroll
    for (int d = 0; d < BITS; ++d) r.w[d] = p[d];
    const int g = (int)fdiv((uint32_t)(chunk * 32), A.divG);
    r.s = srow[g];
    r.z = zrow[g];
}

// ------------------------------------------------------------------ natural-order decode
// h[i] = (1024 + code 2i, 1024 + code 2i+1) as packed fp16 bit patterns (g = 0x64006400
// in a VGPR, so each pair is one v_and_or_b32 after its byte/bit placement).
template <int BITS> struct NatDecode;

template <> struct NatDecode<4> {
    static __device__ __forceinline__ void run(const uint32_t (&w)[4], uint32_t (&h)[16], uint32_t g) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t v = w[t] >> 4;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                // byte b of w (code 8t+2b in its low nibble) and of w >> 4 (code 8t+2b+1)
                const uint32_t sel = (uint32_t)b | (0x0Cu << 8) | ((4u + b) << 16) | (0x0Cu << 24);
                h[4 * t + b] = (__builtin_amdgcn_perm(v, w[t], sel) & 0x000F000Fu) | g;
            }
        }
    }
};

template <> struct NatDecode<2> {
    static __device__ __forceinline__ void run(const uint32_t (&w)[2], uint32_t (&h)[16], uint32_t g) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint32_t v0 = w[t], v2 = w[t] >> 2, v4 = w[t] >> 4, v6 = w[t] >> 6;
#pragma unroll
            for (int pr = 0; pr < 8; ++pr) {
                // codes 2pr, 2pr+1 of the word sit at bits 4pr and 4pr + 2
                const uint32_t b = (uint32_t)(pr >> 1);
                const uint32_t sel = b | (0x0Cu << 8) | ((4u + b) << 16) | (0x0Cu << 24);
                const uint32_t lo = (pr & 1) ? v4 : v0, hi = (pr & 1) ? v6 : v2;
                h[8 * t + pr] = (__builtin_amdgcn_perm(hi, lo, sel) & 0x00030003u) | g;
            }
        }
    }
};

template <> struct NatDecode<3> {
    static __device__ __forceinline__ void run(const uint32_t (&w)[3], uint32_t (&h)[16], uint32_t g) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            // codes 2i, 2i+1 at chunk bits 6i .. 6i+5
            const int bit = 6 * i, wi = bit >> 5, off = bit & 31;
            uint32_t a;
            if (off == 0) a = w[wi];
            else if (wi + 1 < 3) a = __builtin_amdgcn_alignbit(w[wi + 1], w[wi], off);
            else a = w[wi] >> off;
            const uint32_t pair = (a & 0x0000FFFFu) | ((a << 13) & 0xFFFF0000u);   // v_bfi
            h[i] = (pair & 0x00070007u) | g;
        }
    }
};

// Dequantize the (column n, chunk c) of stage s held in registers into B tile `bbuf`.
template <int BITS>
__device__ __forceinline__ void dequant(const GemmArgs& A, const WRegs<BITS>& r, int s, int n, int c, int bbuf,
                                        char* lds) {
    uint32_t h[16];
    NatDecode<BITS>::run(r.w, h, magic_vreg());
    uint32_t o[16];
    const float zf = (float)r.z;
    if (zf == __builtin_rintf(zf) && __builtin_fabsf(zf) < 1024.f) {
        const _Float16 cz = (_Float16)(1024.f + zf);          // exact: an integer below 2048
        const h2 c2 = {cz, cz}, s2 = {r.s, r.s};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const h2 v = (__builtin_bit_cast(h2, h[i]) - c2) * s2;
            o[i] = __builtin_bit_cast(uint32_t, v);
        }
    } else {
        const float sf = (float)r.s;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float lo = ((float)(h[i] & 0x3FFu) - zf) * sf;
            const float hi = ((float)((h[i] >> 16) & 0x3FFu) - zf) * sf;
            const h2 v = {(_Float16)lo, (_Float16)hi};
            o[i] = __builtin_bit_cast(uint32_t, v);
        }
    }
    const int k0 = BK * s + 32 * c;
    if (__builtin_expect(k0 + 32 > A.K, 0)) {                  // K % 8 == 0: pairs never straddle K
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (k0 + 2 * i >= A.K) o[i] = 0u;
    }
    u4* bt = reinterpret_cast<u4*>(lds + B_OFF + bbuf * TILE);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int p = 4 * c + j;
        bt[n * 8 + (p ^ swz(n))] = u4{o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]};
    }
}

template <int BITS>
__global__ void __launch_bounds__(THREADS) gemm_f16_kernel(const GemmArgs A) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool producer = wave >= 4;
    const int mtiles = (A.M + BM - 1) / BM;
    const int m0 = (blockIdx.x % mtiles) * BM, n0 = (blockIdx.x / mtiles) * BN;
    const int nst = (A.K + BK - 1) / BK;

    if (producer) {
        // thread (column n, chunk c) of every stage; a 3-stage register ring
        const int ptid = tid - 256, n = ptid & 127, c = ptid >> 7;
        const long col = (long)min(n0 + n, A.N - 1);
        const uint32_t* wrow = A.w + col * A.wpr;
        const _Float16* srow = reinterpret_cast<const _Float16*>(A.s) + col * A.G;
        const _Float16* zrow = reinterpret_cast<const _Float16*>(A.z) + col * A.G;
        // ring slot of stage t: t % 3; at iteration s stage s+2 is dequantized and
        // stage s+5 loaded into the slot it leaves, three iterations ahead (the loop
        // is unrolled by three so the slots are registers; every step issues its loads)
        WRegs<BITS> rr[3];
        load_w<BITS>(A, wrow, srow, zrow, 0, c, rr[0]);
        load_w<BITS>(A, wrow, srow, zrow, 1, c, rr[1]);
        load_w<BITS>(A, wrow, srow, zrow, 2, c, rr[2]);
        dequant<BITS>(A, rr[0], 0, n, c, 0, lds);
        load_w<BITS>(A, wrow, srow, zrow, 3, c, rr[0]);
        dequant<BITS>(A, rr[1], 1, n, c, 1, lds);
        load_w<BITS>(A, wrow, srow, zrow, 4, c, rr[1]);
        for (int s0 = 0; s0 < nst; s0 += 3) {
#pragma unroll
            for (int u = 0; u < 3; ++u) {
                const int s = s0 + u;
                if (s < nst) {
                    barrier_lds();                // B tiles s, s+1 ready; tile of s-1 free
                    if (s + 2 < nst) dequant<BITS>(A, rr[(u + 2) % 3], s + 2, n, c, (s + 2) % NB, lds);
                }
                load_w<BITS>(A, wrow, srow, zrow, s + 5, c, rr[(u + 2) % 3]);
            }
        }
        return;
    }

    // consumer: 32x32 block (a, b) of the wave tile at rows wm*64 + 32a, columns wn*64 + 32b
    const int wm = wave >> 1, wn = wave & 1;
    f16x acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.f;

    ASrc da;
    a_setup(A, m0, wave, lane, da);
    for (int j = 0; j < AHEAD; ++j) issue_a(A, da, j, j, lds, wave, nst);
    // operand lane map of v_mfma_f32_32x32x16_f16: lane (r = lane & 31, h = lane >> 5)
    // holds row / column r, k = 8h .. 8h+7 of the 16-code step
    const int r32 = lane & 31, hk = lane >> 5;
    int aoff[2], boff[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) aoff[a] = (wm * 64 + a * 32 + r32) * 8;
#pragma unroll
    for (int b = 0; b < 2; ++b) boff[b] = (wn * 64 + b * 32 + r32) * 8;
    const int sw = swz(r32);                      // rows / columns are 32-aligned + r32
    // operands of a stage: 4 steps of 16 codes x (2 A blocks, 2 B blocks)
    auto read_ops = [&](int st, u4 (&af)[4][2], u4 (&bf)[4][2]) {
        const u4* at = reinterpret_cast<const u4*>(lds + A_OFF + (st % NSTAGE) * TILE);
        const u4* bt = reinterpret_cast<const u4*>(lds + B_OFF + (st % NB) * TILE);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int p = (2 * ks + hk) ^ sw;
#pragma unroll
            for (int a = 0; a < 2; ++a) af[ks][a] = at[aoff[a] + p];
#pragma unroll
            for (int b = 0; b < 2; ++b) bf[ks][b] = bt[boff[b] + p];
        }
    };
    auto mfma_stage = [&](const u4 (&af)[4][2], const u4 (&bf)[4][2]) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const h8*>(&af[ks][a]),
                                                                       *reinterpret_cast<const h8*>(&bf[ks][b]),
                                                                       acc[a][b], 0, 0, 0);
    };
    // stage s's operands are read during iteration s-1 (stage 0's after the first
    // barrier); iteration s: barrier, read stage s+1, multiply stage s
    u4 fa[2][4][2], fb[2][4][2];
    vmcnt<(AHEAD - 1) * A_ISSUE>();              // activation stage 0 landed (this wave)
    for (int s = 0; s < nst; s += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int st = s + u;
            if (st < nst) {
                // this wave's activation stage st+1 landed (stage st+2 may still be in flight)
                vmcnt<A_ISSUE>();
                barrier_lds();                    // every wave's: activation st+1, B tiles st, st+1
                if (st == 0) read_ops(0, fa[0], fb[0]);
                issue_a(A, da, st + AHEAD, (st + AHEAD) % NSTAGE, lds, wave, nst);
                if (st + 1 < nst) read_ops(st + 1, fa[(u + 1) & 1], fb[(u + 1) & 1]);
                mfma_stage(fa[u], fb[u]);
            }
        }
    }

    // D layout of the 32x32 block: lane (j = lane & 31, h = lane >> 5), register
    // 4g + r holds row 8g + 4h + r, column j
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int n = n0 + wn * 64 + b * 32 + r32;
        if (n >= A.N) continue;
        const float bias = A.b ? load_f<DT_F16>(A.b, n) : 0.f;
#pragma unroll
        for (int a = 0; a < 2; ++a) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = m0 + wm * 64 + a * 32 + 8 * (v >> 2) + 4 * hk + (v & 3);
                if (m < A.M) store_f<DT_F16>(A.out, (long)m * A.N + n, apply_act(acc[a][b][v] + bias, A.act));
            }
        }
    }
}

template <int BITS>
const void* kernel_for() {
    return reinterpret_cast<const void*>(&gemm_f16_kernel<BITS>);
}

}  // namespace

bool gemm_f16_supported(const GemmArgs& A) {
    // 16-byte activation pieces, whole pairs before K, 4-byte scale/zero reads
    return A.K % 8 == 0 && A.K >= 8 && (reinterpret_cast<uintptr_t>(A.x) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(A.w) & 3) == 0;
}

hipError_t launch_gemm_f16(const GemmArgs& A, hipStream_t stream) {
    const void* f = A.bits == 2 ? kernel_for<2>() : (A.bits == 3 ? kernel_for<3>() : kernel_for<4>());
    const int lds = LDS_BYTES;
    hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    const int tiles = ((A.M + BM - 1) / BM) * ((A.N + BN - 1) / BN);
    void* args[] = {const_cast<GemmArgs*>(&A)};
    return launch(f, dim3(tiles), dim3(THREADS), args, (size_t)lds, stream);
}

}  // namespace cbk
