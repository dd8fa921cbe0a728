// gemv_batch.hip -- batched fp16 decode GEMV (batch rows 3..16) in one dispatch.
//
// Replaces cb_gemv_kernel (Kernel/csrc/packed_gemv.cu:83-163) for decode batches
// of 3..16 activation rows where the K-split streaming kernel (gemv_stream.hip) would
// need split-K partials and the reduce launch that cb_reduce_kernel (:166-180) stands
// for: plain, fused-QKV and fused gate-up modes, the epilogue of cb_epilogue (:54-81,
// cbk_device.hpp).  fp16 activations; group sizes that are multiples of 128, so a unit
// of 128 codes (4 chunks) lies in one group.
//
// A workgroup owns RW (1 .. 3) blocks of 16 virtual rows over all of K with
// NW = Q RW waves, Q = 16 / RW per block (16 waves; 15 for RW = 3), and takes K in
// phases of PH = NW units, so each wave serves NMY = RW units of a phase and the
// NW 64 threads convert the 4 PH chunks of up to 16 batch rows in one item each.
// Each phase's activations are loaded and converted once per workgroup -- to the
// in-place decode's operand order (x_k 2^-e(k) at half slot k, cbk_decode.hpp) with
// per unit and batch row the sums X = sum x and XB = 1024 sum x 2^-e -- into one of
// two LDS buffers, while the waves compute the previous phase from the other.  Wave w
// serves row block w % RW and every Q-th unit of each phase: lane (j = l & 15,
// kq = l >> 4) loads chunk 4 u + kq of its block's row j (requested D phases ahead,
// D = 4, 2, 1 for RW = 1, 2, 3, each slot right after it is consumed), decodes it in
// place into the B operand of four v_mfma_f32_16x16x32_f16 whose A operand holds the
// staged batch rows, and adds
//   acc[i][j] += s[j] (D[i][j] - XB[i] - z[j] X[i])
// (lane (j, kq) holds batch rows 4 kq .. 4 kq + 3 of row j).  The Q partial sums
// of a row meet in LDS and are added in a fixed order, so the result does not
// depend on wave timing; the epilogue follows.
#include "cbk_decode.hpp"
#include "cbk_device.hpp"
#include "cbk_kernels.hpp"

namespace cbk {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u3 __attribute__((ext_vector_type(3)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int RAW = 0x00020000;          // buffer descriptor word 3: raw 32-bit data
// A byte offset past every descriptor's range: such loads return zero.  Loads are
// issued unconditionally and the ones that must not contribute read here.
constexpr int OOR = 0x7FFFFF00;

// The offset as an opaque VGPR value, so the compiler keeps the select in front of
// the load instead of turning it into a branch around two loads.
__device__ __forceinline__ int vofs(bool ok, int off) {
    int v = ok ? off : OOR;
    asm("" : "+v"(v));
    return v;
}

template <int BITS>
__device__ __forceinline__ void load_chunk(__amdgpu_buffer_rsrc_t r, int off, uint32_t (&w)[BITS]) {
    if constexpr (BITS == 4) {
        const u4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (BITS == 3) {
        const u3 v = __builtin_amdgcn_raw_buffer_load_b96(r, off, 0, 0);
        w[0] = v.x; w[1] = v.y; w[2] = v.z;
    } else {
        const u2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
        w[0] = v.x; w[1] = v.y;
    }
}

struct ProjRes {
    __amdgpu_buffer_rsrc_t w, s, z;
};

__device__ __forceinline__ ProjRes proj_res(const Proj& p, int G) {
    ProjRes r;
    r.w = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(p.w), (short)0, p.n * p.wpr * 4, RAW);
    r.s = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.s), (short)0, p.n * G * 2, RAW);
    r.z = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.z), (short)0, p.n * G * 2, RAW);
    return r;
}

// Activation chunk ca (codes 32 ca ..) of batch row b as 16 words of fp16 pairs; a
// 16-byte piece lies wholly before or past K (K % 8 == 0) and reads as zero past
// it, or when `ok` is false.
__device__ __forceinline__ void load_x(__amdgpu_buffer_rsrc_t xr, bool ok, int b, int ca, int K, uint32_t (&x)[16]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int k = 32 * ca + 8 * i;
        const u4 v = __builtin_amdgcn_raw_buffer_load_b128(xr, vofs(ok && k < K, 2 * (b * K + k)), 0, 0);
        x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
    }
}

// The chunk in the decode's operand order: pair p = (x[kappa(2p)] 2^-e, x[kappa(2p+1)]
// 2^-e') (a power-of-two scale, exact unless the fp16 result is subnormal), with its
// sums B = 1024 sum 2^-e x and xs = sum x.
template <int BITS>
__device__ __forceinline__ void convert_x(const uint32_t (&x)[16], u4 (&X)[4], float& B, float& xs) {
    const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
    uint32_t o[16];
    float b = 0.f, t = 0.f;
#pragma unroll
    for (int p = 0; p < 16; ++p) {
        const int ka = Decode<BITS>::kappa(2 * p), kb = Decode<BITS>::kappa(2 * p + 1);
        const int ea = Decode<BITS>::expo(2 * p), eb = Decode<BITS>::expo(2 * p + 1);
        const uint32_t sel = (uint32_t)(2 * (ka & 1)) | ((uint32_t)(2 * (ka & 1) + 1) << 8) |
                             ((uint32_t)(4 + 2 * (kb & 1)) << 16) | ((uint32_t)(5 + 2 * (kb & 1)) << 24);
        const uint32_t raw = __builtin_amdgcn_perm(x[kb >> 1], x[ka >> 1], sel);
        const h2 sc = {(_Float16)(1.0f / (float)(1 << ea)), (_Float16)(1.0f / (float)(1 << eb))};
        const h2 v = __builtin_bit_cast(h2, raw) * sc;
        o[p] = __builtin_bit_cast(uint32_t, v);
        b = __builtin_amdgcn_fdot2(v, one, b, false);
        t = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, x[p]), one, t, false);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) X[q] = u4{o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]};
    B = 1024.f * b;
    xs = t;
}

// Units per phase (and waves) of a workgroup with rw row blocks.
__host__ __device__ constexpr int batch_phase(int rw) { return (16 / rw) * rw; }

// LDS of one phase buffer (PH units, 4 PH chunks): piece m of chunk c of batch row i
// at ((m 4 PH + c) MP + i) 16 with the odd stride MP = M | 1, so the 16-byte pieces
// that consecutive lanes write (consecutive c) and read (consecutive i) fall in
// distinct bank groups; then per unit and batch row the sums X (at XS[u 16 + i]) and XB.
__host__ __device__ constexpr int batch_stride(int M) { return M | 1; }
__host__ __device__ constexpr int batch_buf_bytes(int M, int ph) {
    return 256 * ph * batch_stride(M) + 2 * ph * 16 * 4;
}

// The lane's activation chunk of a phase: item t = tid (batch row t / NCH, chunk
// t % NCH, NCH = 4 PH), loaded, then converted into buffer `buf`.  The NW = PH waves
// hold 64 PH = 16 NCH items, one per batch row and chunk for M <= 16.
template <int PH>
__device__ __forceinline__ void x_issue(__amdgpu_buffer_rsrc_t xr, const GemvArgs& A, int phase, int tid,
                                        uint32_t (&xi)[16]) {
    constexpr int NCH = 4 * PH;
    const int i = tid / NCH, c = tid - i * NCH;
    const int cg = phase * NCH + c;
    load_x(xr, i < A.M && cg < A.C, i, cg, A.K, xi);
}

template <int BITS, int PH>
__device__ __forceinline__ void x_stage(const GemvArgs& A, int tid, const uint32_t (&xi)[16], char* buf) {
    constexpr int NCH = 4 * PH;
    const int M = A.M;
    const int i = tid / NCH, c = tid - i * NCH;
    if (i >= M) return;                           // whole quads leave together (NCH % 4 == 0)
    u4* Xl = reinterpret_cast<u4*>(buf);
    const int MP = batch_stride(M);
    float* XS = reinterpret_cast<float*>(buf + 64 * NCH * MP);
    float* XB = XS + 16 * PH;
    u4 X[4];
    float B, xs;
    convert_x<BITS>(xi, X, B, xs);
#pragma unroll
    for (int m = 0; m < 4; ++m) Xl[(m * NCH + c) * MP + i] = X[m];
    // the 4 chunks of a unit are 4 consecutive threads
    B += __shfl_xor(B, 1, 64);
    xs += __shfl_xor(xs, 1, 64);
    B += __shfl_xor(B, 2, 64);
    xs += __shfl_xor(xs, 2, 64);
    if ((c & 3) == 0) {
        XS[(c >> 2) * 16 + i] = xs;
        XB[(c >> 2) * 16 + i] = B;
    }
}

// Workgroup barrier that completes the wave's LDS traffic but not its global loads.
__device__ __forceinline__ void barrier_lds() {
    __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4));    // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
}

// One unit slot of a wave: the lane's chunk and its row's (scale, zero).
template <int BITS>
struct WSlot {
    uint32_t w[BITS];
    uint32_t s, z;
};

// Requests unit ul (phase-local) of `phase` for the lane's row r and chunk kq.
template <int BITS, int PH>
__device__ __forceinline__ void w_issue(const GemvArgs& A, const ProjRes& P, int wpr, int r, bool vin, int phase,
                                        int ul, int kq, WSlot<BITS>& ws) {
    const int U = (A.C + 3) >> 2;
    const int u = phase * PH + ul;
    const int c = 4 * u + kq;
    load_chunk<BITS>(P.w, vofs(vin && c < A.C, 4 * (r * wpr + c * BITS)), ws.w);
    // (scale, zero) of the unit's group through buffer loads (a generic-pointer load
    // would make every LDS access wait for all loads in flight)
    const int gu = (int)fdiv((uint32_t)u, A.divG);
    const int so = vofs(vin && u < U, 2 * (r * A.G + gu));
    ws.s = __builtin_amdgcn_raw_buffer_load_b16(P.s, so, 0, 0);
    ws.z = __builtin_amdgcn_raw_buffer_load_b16(P.z, so, 0, 0);
}

// Unit ul of the phase staged in `buf` against the slot's weights.
template <int BITS, int PH>
__device__ __forceinline__ void w_compute(const GemvArgs& A, const WSlot<BITS>& ws, const char* buf, int ul, int j,
                                          int kq, uint32_t g, f4& acc) {
    constexpr int NCH = 4 * PH;
    const int M = A.M;
    const u4* Xl = reinterpret_cast<const u4*>(buf);
    const int MP = batch_stride(M);
    const float* XS = reinterpret_cast<const float*>(buf + 64 * NCH * MP);
    const float* XB = XS + 16 * PH;
    const int ia = min(j, M - 1);                 // rows past M repeat a staged row (not stored)
    const int c = 4 * ul + kq;
    u4 a[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) a[m] = Xl[(m * NCH + c) * MP + ia];
    const f4 X4 = *reinterpret_cast<const f4*>(XS + ul * 16 + 4 * kq);
    const f4 XB4 = *reinterpret_cast<const f4*>(XB + ul * 16 + 4 * kq);
    uint32_t h[16];
    Decode<BITS>::run(ws.w, h, g);
    f4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const u4 bw = {h[4 * m], h[4 * m + 1], h[4 * m + 2], h[4 * m + 3]};
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const h8*>(&a[m]),
                                                   *reinterpret_cast<const h8*>(&bw), d, 0, 0, 0);
    }
    const float sc = (float)__builtin_bit_cast(_Float16, (uint16_t)ws.s);
    const float ze = (float)__builtin_bit_cast(_Float16, (uint16_t)ws.z);
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = fmaf(sc, fmaf(-ze, X4[q], d[q] - XB4[q]), acc[q]);
}

// Weight prefetch depth (phases in flight) and activation prefetch depth per RW, sized
// to the 128 VGPRs of a wave at four waves per SIMD.
__host__ __device__ constexpr int batch_wdepth(int rw) { return rw == 1 ? 4 : (rw == 2 ? 2 : 1); }
__host__ __device__ constexpr int batch_xdepth(int) { return 1; }

// RW row blocks: Q = 16 / RW waves per block, NW = PH = Q RW waves and units per
// phase, NMY = RW unit slots per wave (units qw + n Q).  Weights are requested D
// phases ahead into a ring of D slot sets, activations DX phases ahead.
template <int BITS, int MODE, int RW>
__device__ __forceinline__ void batch_body(const GemvArgs& A, char* lds) {
    constexpr int Q = 16 / RW;
    constexpr int PH = batch_phase(RW);
    constexpr int NW = PH;
    constexpr int NMY = RW;
    constexpr int NCH = 4 * PH;
    constexpr int RB = 16 * RW;
    constexpr int D = batch_wdepth(RW);
    constexpr int DX = batch_xdepth(RW);
    constexpr int UNROLL = D > 2 ? D : 2;          // D, DX in {1, 2, 4}: even and a multiple of both
    static_assert(UNROLL % 2 == 0 && UNROLL % D == 0 && UNROLL % DX == 0, "phase parity must be static");
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rb = wave % RW, qw = wave / RW;
    const int M = A.M;
    const int nph = (A.C + NCH - 1) / NCH;
    const int vbase = blockIdx.x * RB;
    const int j = lane & 15, kq = lane >> 4;
    const uint32_t g = magic_vreg();

    // the wave's 16 rows: virtual rows vbase + 16 rb + j, or for gate-up projection
    // rb & 1 of pair rows vbase / 2 + 16 (rb >> 1) + j (virtual rows 2 n + (rb & 1))
    int roff, vfirst;
    if constexpr (MODE == MODE_GATEUP) {
        vfirst = vbase + 32 * (rb >> 1) + (rb & 1);
        roff = 32 * (rb >> 1) + 2 * j + (rb & 1);
    } else {
        vfirst = vbase + 16 * rb;
        roff = 16 * rb + j;
    }
    const int vrow = vbase + roff;
    int proj, rfirst;
    vmap<MODE>(A, min(vfirst, A.V - 1), proj, rfirst);
    const int r = rfirst + j;
    const bool vin = vrow < A.V;

    ProjRes R[3];
    R[0] = proj_res(A.p[0], A.G);
    if constexpr (MODE == MODE_GATEUP) R[1] = proj_res(A.p[1], A.G);
    if constexpr (MODE == MODE_QKV) { R[1] = proj_res(A.p[1], A.G); R[2] = proj_res(A.p[2], A.G); }
    const ProjRes& P = proj == 0 ? R[0] : (proj == 1 ? R[1] : R[2]);
    const int wpr = CBK_SEL(A, proj, wpr);
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(A.x), (short)0, A.M * A.K * 2, RAW);

    char* const buf0 = lds;
    char* const buf1 = lds + batch_buf_bytes(M, PH);
    float* red = reinterpret_cast<float*>(lds + 2 * batch_buf_bytes(M, PH));

    // prologue: weights of phases 0 .. D - 1, activations of phases 0 .. DX (phase 0
    // staged).  Loads of phases past the last one read zeros (offsets out of range) and
    // are issued anyway, here and in the loop: unconditional loads leave no merge of old
    // and new register values, whose copy would wait for every load in flight.
    uint32_t xi[DX][16];
    WSlot<BITS> ws[D][NMY];
#pragma unroll
    for (int e = 0; e < DX; ++e) x_issue<PH>(xr, A, e, tid, xi[e]);
#pragma unroll
    for (int h = 0; h < D; ++h)
#pragma unroll
        for (int n = 0; n < NMY; ++n) w_issue<BITS, PH>(A, P, wpr, r, vin, h, qw + n * Q, kq, ws[h][n]);
    x_stage<BITS, PH>(A, tid, xi[0], buf0);
    x_issue<PH>(xr, A, DX, tid, xi[0]);
    barrier_lds();

    f4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int ph = 0; ph < nph; ph += UNROLL) {
#pragma unroll
        for (int h = 0; h < UNROLL; ++h) {
            const int phase = ph + h;
            if (phase >= nph) break;
            const char* cur = (h & 1) ? buf1 : buf0;           // phase parity = h parity (UNROLL even)
#pragma unroll
            for (int n = 0; n < NMY; ++n) {
                w_compute<BITS, PH>(A, ws[h % D][n], cur, qw + n * Q, j, kq, g, acc);
                asm volatile("" : "+v"(acc));       // the update stays ahead of the loads
                __builtin_amdgcn_sched_barrier(0);
                w_issue<BITS, PH>(A, P, wpr, r, vin, phase + D, qw + n * Q, kq, ws[h % D][n]);
            }
            // stage phase + 1 into the other buffer (last read in phase - 1), then request
            // phase + 1 + DX into the registers it frees
            if (phase + 1 < nph) x_stage<BITS, PH>(A, tid, xi[(h + 1) % DX], (h & 1) ? buf0 : buf1);
            x_issue<PH>(xr, A, phase + 1 + DX, tid, xi[(h + 1) % DX]);
            barrier_lds();
        }
    }

    // the Q partial sums of each row meet in LDS: red[(qw M + i) RB + roff]
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int i = 4 * kq + q;
        if (i < M) red[(qw * M + i) * RB + roff] = acc[q];
    }
    barrier_lds();
    for (int t = tid; t < M * RB; t += NW * 64) {
        const int b = t / RB, ro = t - b * RB;
        const int v = vbase + ro;
        if (v < A.V) {
            float mine = 0.f, partner = 0.f;
            for (int k = 0; k < Q; ++k) {
                mine += red[(k * M + b) * RB + ro];
                partner += red[(k * M + b) * RB + (ro ^ 1)];
            }
            epilogue<DT_F16, MODE>(A, b, v, mine, partner);
        }
    }
}

template <int MODE, int BITS, int RW>
__global__ void __launch_bounds__(1024) gemv_batch_kernel(const GemvArgs A) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    if constexpr (BITS != 0) {
        batch_body<BITS, MODE, RW>(A, lds);
    } else {
        // fused QKV with a width per projection: the host keeps each workgroup's rows
        // inside one projection, so the width is uniform per workgroup
        int proj, r;
        vmap<MODE>(A, (int)blockIdx.x * 16 * RW, proj, r);
        const int bits = CBK_SEL(A, proj, bits);
        if (bits == 2) batch_body<2, MODE, RW>(A, lds);
        else if (bits == 3) batch_body<3, MODE, RW>(A, lds);
        else batch_body<4, MODE, RW>(A, lds);
    }
}

template <int RW>
const void* batch_kernel(int mode, int bits, bool mixed) {
    if (mixed) return reinterpret_cast<const void*>(&gemv_batch_kernel<MODE_QKV, 0, RW>);
#define CBK_BATCH_BITS(M)                                                                            \
    (bits == 2 ? reinterpret_cast<const void*>(&gemv_batch_kernel<M, 2, RW>)                         \
               : (bits == 3 ? reinterpret_cast<const void*>(&gemv_batch_kernel<M, 3, RW>)            \
                            : reinterpret_cast<const void*>(&gemv_batch_kernel<M, 4, RW>)))
    if (mode == MODE_GATEUP) {
        // a gate row and its up row share the workgroup: an even number of row blocks
        if constexpr (RW % 2 == 0) return CBK_BATCH_BITS(MODE_GATEUP);
        return nullptr;
    }
    if (mode == MODE_QKV) return CBK_BATCH_BITS(MODE_QKV);
    return CBK_BATCH_BITS(MODE_GEMV);
#undef CBK_BATCH_BITS
}

}  // namespace

int batch_threads(int rw) { return 64 * batch_phase(rw); }

int batch_lds_bytes(int M, int rw) {
    const int ph = batch_phase(rw);
    return 2 * batch_buf_bytes(M, ph) + ph * M * 16 * 4;
}

const void* gemv_batch_kernel_for(int mode, int bits, bool mixed, int rw) {
    return rw == 1 ? batch_kernel<1>(mode, bits, mixed)
                   : (rw == 2 ? batch_kernel<2>(mode, bits, mixed) : batch_kernel<3>(mode, bits, mixed));
}

}  // namespace cbk
