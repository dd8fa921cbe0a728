// gemv_stream.hip -- decode GEMVs that stream packed rows through VGPRs.
//
// Replaces cb_gemv_kernel (Kernel/csrc/packed_gemv.cu:83-163) and, when the K
// range is split, the partial write that cb_reduce_kernel (:166-180) combines,
// for one or two activation rows (the decode step) in fp16 or bf16, or one fp32 row (as two
// fp16 operand rows), with any group size that is a multiple of 32.  Plain, fused-QKV and
// fused gate-up modes share the body; the
// outputs are finished per row (plain) or row pair (fused modes; finish, cbk_device.hpp).
//
// Job = (block of RB = RPW RW virtual rows, K split p).  A workgroup holds KS x RW
// waves: wave (ks, rw) takes rows RPW rw .. RPW rw + RPW - 1 of the block (RPW = 4,
// or 8 for the host's short-K plain GEMVs) over K slice ks of the split, 64 CPL chunks
// of 32 codes, lane l owning chunks l + 64 i (i < CPL) of the slice.  Per wave:
//   1. The thread's activation chunk is requested, then every packed
//      chunk of the wave's rows (one buffer load of BITS dwords per row and lane
//      chunk, 64 lanes = 64 consecutive chunks) and their (scale, zero) halves --
//      the whole of the wave's weights is in flight before any arithmetic.
//   2. Activations are converted to the operand order of the in-place decode
//      (cbk_decode.hpp): pair p = (x_a 2^-e_a, x_b 2^-e_b) for the codes kappa and
//      field offsets expo of the chunk's half slots, with the chunk's slot-offset
//      sum B = 1024 sum_p X_p and its plain sum sum_j x_j, into LDS; one barrier
//      publishes them to every wave of the workgroup.  bf16 chunks are first scaled
//      by a power of two 2^-c of their own (convert_x_bf16), so the fp16 operands
//      hold every bf16 value exactly; the chunk's terms are scaled back by 2^c.
//   3. Per row and chunk: the BITS words decode into 16 fp16 pairs 1024 + 2^e q by
//      one v_and_or_b32 each, 16 v_dot2_f32_f16 against the staged pairs give
//      sum x q + B, and acc += s * (dot - B - z * sum x)  (packed_gemv.cu:113-138
//      algebra: the zero point is applied per chunk against the activation sum).
//   4. Each 4 rows' lane sums meet by v_permlane32_swap, v_permlane16_swap and four
//      DPP row rotations (every lane of a 16-lane row ends with one row's total).
//   5. Row totals of the slices meet in LDS and are added in slice order (so the
//      result does not depend on wave timing); the finish stage runs per finish unit
//      (a row, or a row pair in the fused modes), or with P > 1 the fp32 partials are
//      written for the split-K combine.
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

constexpr int CPL = STREAM_CPL;          // chunks per lane of a slice
constexpr int SLICE = 64 * CPL;          // chunks per K slice
constexpr int RAW = 0x00020000;          // buffer descriptor word 3: raw 32-bit data
// A byte offset past every descriptor's range: such loads return zero.  Loads are
// issued unconditionally (a branch around a load makes the compiler wait for it at
// the join), and the ones that must not contribute read here.
constexpr int OOR = 0x7FFFFF00;


// The offset as an opaque VGPR value, so the compiler keeps the select in front of
// the load instead of turning it into a branch around two loads.
__device__ __forceinline__ int vofs(bool ok, int off) {
    int v = ok ? off : OOR;
    asm("" : "+v"(v));
    return v;
}

// One chunk's BITS words at byte offset `off` of the packed tensor (zero past its end).
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

// Descriptors of a projection's packed rows and of its scales and zeros (MB bytes each).
__device__ __forceinline__ ProjRes proj_res(const Src& p, int G, int MB = 2) {
    ProjRes r;
    r.w = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(p.w), (short)0, p.n * p.wpr * 4, RAW);
    r.s = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.s), (short)0, p.n * G * MB, RAW);
    r.z = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.z), (short)0, p.n * G * MB, RAW);
    return r;
}

// Activation chunk ca of batch row b as 16 words of fp16 pairs (x_2i, x_2i+1).  Each
// 16-byte piece holds 8 codes; K % 8 == 0, so a piece lies wholly before or past K,
// and pieces past K (and every piece when `ok` is false) read as zero.
__device__ __forceinline__ void load_x(__amdgpu_buffer_rsrc_t xr, bool ok, int b, int ca, int K, uint32_t (&x)[16]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int k = 32 * ca + 8 * i;
        const u4 v = __builtin_amdgcn_raw_buffer_load_b128(xr, vofs(ok && k < K, 2 * (b * K + k)), 0, 0);
        x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
    }
}

// Operand pairs of one chunk for the BITS decode, their slot-offset sum B and sum x.
template <int BITS>
__device__ __forceinline__ void convert_x(const uint32_t (&x)[16], u4 (&X)[4], float& B, float& xs) {
    const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
    uint32_t o[16];
    float b = 0.f, t = 0.f;
#pragma unroll
    for (int p = 0; p < 16; ++p) {
        const int ka = Decode<BITS>::kappa(2 * p), kb = Decode<BITS>::kappa(2 * p + 1);
        const int ea = Decode<BITS>::expo(2 * p), eb = Decode<BITS>::expo(2 * p + 1);
        // low half = x[ka] (half ka & 1 of word ka >> 1), high half = x[kb]
        const uint32_t sel = (uint32_t)(2 * (ka & 1)) | ((uint32_t)(2 * (ka & 1) + 1) << 8) |
                             ((uint32_t)(4 + 2 * (kb & 1)) << 16) | ((uint32_t)(5 + 2 * (kb & 1)) << 24);
        const uint32_t raw = __builtin_amdgcn_perm(x[kb >> 1], x[ka >> 1], sel);
        const h2 sc = {(_Float16)(1.0f / (float)(1 << ea)), (_Float16)(1.0f / (float)(1 << eb))};
        const h2 v = __builtin_bit_cast(h2, raw) * sc;      // power-of-two scale: exact unless subnormal
        o[p] = __builtin_bit_cast(uint32_t, v);
        b = __builtin_amdgcn_fdot2(v, one, b, false);
        t = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, x[p]), one, t, false);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) X[q] = u4{o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]};
    B = 1024.f * b;
    xs = t;
}

// bf16 activations.  The chunk is prescaled by 2^-c, c taken from its largest exponent so
// that its largest magnitude lands in [2^14, 2^15): times 2^-e (e <= 5) that stays inside
// fp16's range, and every element at least 2^-23 of the largest is a normal fp16 number
// after the scaling, where its 8 significant bits are exact (smaller ones lose bits only
// below 2^-34 of it).  X and B are the fp16 operands as in convert_x; xs = sum x 2^-c
// (fp32, formed from the operands) and f = 2^c scales the chunk's terms back.  Infinities and NaNs stay what they
// are; c >= -126 keeps f a normal float.
// The largest biased exponent of a bf16 chunk.
__device__ __forceinline__ int chunk_exp_bf16(const uint32_t (&x)[16]) {
    typedef uint16_t us2 __attribute__((ext_vector_type(2)));
    us2 m = {0, 0};
#pragma unroll
    for (int p = 0; p < 16; ++p) m = __builtin_elementwise_max(m, __builtin_bit_cast(us2, x[p] & 0x7F807F80u));
    return (int)(max(m.x, m.y) >> 7);
}

// The prescale exponent c for a largest biased exponent E.
__device__ __forceinline__ int prescale_bf16(int E) { return max(E - (127 + 14), -126); }

// The chunk's operands at a given prescale exponent c.
template <int BITS>
__device__ __forceinline__ void convert_x_bf16_at(const uint32_t (&x)[16], int c, u4 (&X)[4], float& B, float& xs) {
    const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
    uint32_t o[16];
    float b = 0.f, t = 0.f;
#pragma unroll
    for (int p = 0; p < 16; ++p) {
        const int ka = Decode<BITS>::kappa(2 * p), kb = Decode<BITS>::kappa(2 * p + 1);
        const int ea = Decode<BITS>::expo(2 * p), eb = Decode<BITS>::expo(2 * p + 1);
        const uint32_t wa = x[ka >> 1], wb = x[kb >> 1];
        const float xa = __uint_as_float((ka & 1) ? (wa & 0xFFFF0000u) : (wa << 16));
        const float xb = __uint_as_float((kb & 1) ? (wb & 0xFFFF0000u) : (wb << 16));
        const h2 v = {(_Float16)__builtin_ldexpf(xa, -c - ea), (_Float16)__builtin_ldexpf(xb, -c - eb)};
        o[p] = __builtin_bit_cast(uint32_t, v);
        b = __builtin_amdgcn_fdot2(v, one, b, false);
        // sum x 2^-c from the operands: v 2^e (exact powers of two in fp16, exact products)
        const h2 up = {(_Float16)(float)(1 << ea), (_Float16)(float)(1 << eb)};
        t = __builtin_amdgcn_fdot2(v, up, t, false);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) X[q] = u4{o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]};
    B = 1024.f * b;
    xs = t;
}

template <int BITS>
__device__ __forceinline__ void convert_x_bf16(const uint32_t (&x)[16], u4 (&X)[4], float& B, float& xs, float& f) {
    const int c = prescale_bf16(chunk_exp_bf16(x));
    convert_x_bf16_at<BITS>(x, c, X, B, xs);
    f = __builtin_ldexpf(1.0f, c);
}

// fp32 activations.  Activation chunk ca of batch row b as 32 fp32 words (8 pieces of 16
// bytes; K % 8 == 0, so a piece lies wholly before or past K).
__device__ __forceinline__ void load_x32(__amdgpu_buffer_rsrc_t xr, bool ok, int b, int ca, int K,
                                         uint32_t (&x)[32]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int k = 32 * ca + 4 * i;
        const u4 v = __builtin_amdgcn_raw_buffer_load_b128(xr, vofs(ok && k < K, 4 * (b * K + k)), 0, 0);
        x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
    }
}

// An fp32 chunk as two fp16 operand rows.  The chunk is prescaled by 2^-c as a bf16 chunk is
// (its largest magnitude into [2^14, 2^15)); each slot-scaled value v = x 2^(-c-e) is split
// into hi = RN_fp16(v) and lo = RN_fp16(v - hi) (v - hi is exact in fp32), so hi + lo holds v
// to 2^-22 of the chunk's largest value (subnormal lo parts lose bits only below 2^-39 of it).
// Both rows meet the same decoded weights; their terms add before the scale 2^c.  The
// weights' pairs 1024 + 2^e q lose their 1024 first (exact in fp16), so the dot products
// carry no 1024 sum x term whose cancellation would cost fp32 bits: B = 0.  convert_x_f32_at
// takes the prescale exponent c (the batched kernel shares one per 128-code unit).
__device__ __forceinline__ int chunk_exp_f32(const uint32_t (&x)[32]) {
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) m = max(m, x[i] & 0x7F800000u);
    return (int)(m >> 23);
}

template <int BITS>
__device__ __forceinline__ void convert_x_f32_at(const uint32_t (&x)[32], int c, u4 (&Xh)[4], u4 (&Xl)[4],
                                                 float& xsh, float& xsl) {
    uint32_t oh[16], ol[16];
    float th = 0.f, tl = 0.f;
#pragma unroll
    for (int p = 0; p < 16; ++p) {
        const int ka = Decode<BITS>::kappa(2 * p), kb = Decode<BITS>::kappa(2 * p + 1);
        const int ea = Decode<BITS>::expo(2 * p), eb = Decode<BITS>::expo(2 * p + 1);
        const float va = __builtin_ldexpf(__uint_as_float(x[ka]), -c - ea);
        const float vb = __builtin_ldexpf(__uint_as_float(x[kb]), -c - eb);
        const h2 hi = {(_Float16)va, (_Float16)vb};
        const h2 lo = {(_Float16)(va - (float)hi.x), (_Float16)(vb - (float)hi.y)};
        oh[p] = __builtin_bit_cast(uint32_t, hi);
        ol[p] = __builtin_bit_cast(uint32_t, lo);
        const h2 up = {(_Float16)(float)(1 << ea), (_Float16)(float)(1 << eb)};
        th = __builtin_amdgcn_fdot2(hi, up, th, false);
        tl = __builtin_amdgcn_fdot2(lo, up, tl, false);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        Xh[q] = u4{oh[4 * q], oh[4 * q + 1], oh[4 * q + 2], oh[4 * q + 3]};
        Xl[q] = u4{ol[4 * q], ol[4 * q + 1], ol[4 * q + 2], ol[4 * q + 3]};
    }
    xsh = th;
    xsl = tl;
}

template <int BITS>
__device__ __forceinline__ void convert_x_f32(const uint32_t (&x)[32], u4 (&Xh)[4], u4 (&Xl)[4], float& Bh,
                                              float& xsh, float& Bl, float& xsl, float& f) {
    const int c = prescale_bf16(chunk_exp_f32(x));
    convert_x_f32_at<BITS>(x, c, Xh, Xl, xsh, xsl);
    Bh = 0.f;
    Bl = 0.f;
    f = __builtin_ldexpf(1.0f, c);
}

// Bytes staged per chunk and operand row after its 64 bytes of operand pairs: (B, sum x),
// and for bf16 and fp32 also 2^c (a 16-byte entry).  fp32 stages two operand rows (hi, lo)
// per batch row.
template <int DT> constexpr int XB_BYTES = DT == DT_F16 ? 8 : 16;
template <int DT> constexpr int SROWS = DT == DT_F32 ? 2 : 1;

// A (scale, zero) half of the activations' dtype as a float.
template <int DT>
__device__ __forceinline__ float meta_f(uint32_t bits) {
    if constexpr (DT == DT_BF16) return __uint_as_float(bits << 16);
    else if constexpr (DT == DT_F32) return __uint_as_float(bits);
    else return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

// sum x q + B of one row's chunk: its 16 decoded pairs against one batch row's
// staged operands.
__device__ __forceinline__ float pairs_dot(const uint32_t (&h)[16], const u4 (&X)[4]) {
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        // vector elements are copied to scalars first: clang's __builtin_bit_cast of an
        // ext-vector element lvalue reads the vector's first element
        const uint32_t x0 = X[q].x, x1 = X[q].y, x2 = X[q].z, x3 = X[q].w;
        d0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, h[4 * q + 0]), __builtin_bit_cast(h2, x0), d0, false);
        d1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, h[4 * q + 1]), __builtin_bit_cast(h2, x1), d1, false);
        d0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, h[4 * q + 2]), __builtin_bit_cast(h2, x2), d0, false);
        d1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, h[4 * q + 3]), __builtin_bit_cast(h2, x3), d1, false);
    }
    return d0 + d1;
}

template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Lane sums of 4 rows -> every lane of 16-lane row i holds the total of wave row
// srow(i): rows (0, 2, 1, 3) for lane rows (0, 1, 2, 3).
__device__ __forceinline__ float reduce4(const float (&a)[4]) {
    const auto p01 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[0]), __float_as_uint(a[1]), false, false);
    const auto p23 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[2]), __float_as_uint(a[3]), false, false);
    const float s01 = __uint_as_float(p01[0]) + __uint_as_float(p01[1]);   // lanes 0-31 row 0, 32-63 row 1
    const float s23 = __uint_as_float(p23[0]) + __uint_as_float(p23[1]);   // lanes 0-31 row 2, 32-63 row 3
    const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(s01), __float_as_uint(s23), false, false);
    float s = __uint_as_float(q[0]) + __uint_as_float(q[1]);
    s = dpp_add<0x128>(s);     // row_ror:8
    s = dpp_add<0x124>(s);     // row_ror:4
    s = dpp_add<0x122>(s);     // row_ror:2
    s = dpp_add<0x121>(s);     // row_ror:1
    return s;
}

__device__ __forceinline__ int lane_row(int lane) { return ((lane >> 5) & 1) | (((lane >> 4) & 1) << 1); }

template <int BITS, int MODE, int MB, int RPW, int DT>
__device__ __forceinline__ void stream_body(const GemvArgs& A, char* lds) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int KS = A.st_ks, RW = A.st_rw, RB = RPW * A.st_rw;
    const int NCH = KS * SLICE;
    const int ks = (int)fdiv((uint32_t)wave, A.divRW);
    const int rw = wave - ks * RW;
    const int blk = (int)fdiv(blockIdx.x, A.divP);     // job = blk * P + p (split fastest)
    const int p = blockIdx.x - blk * A.P;
    // split p covers chunks [C p / P, C (p + 1) / P)  (packed_gemv.cu:94-95)
    const int c0 = (int)fdiv((uint32_t)(A.C * p), A.divP);
    const int c1 = (int)fdiv((uint32_t)(A.C * (p + 1)), A.divP);
    const int nrange = c1 - c0;
    const int vbase = blk * RB;
    const int v0 = vbase + RPW * rw;
    const uint32_t g = magic_vreg();

    // 1a. the thread's activation chunk of every batch row (job chunk tid; the host
    // keeps RW >= CPL, so the 64 KS RW threads cover the KS * SLICE staged chunks);
    // batch rows past M read as zero
    constexpr int XE = DT == DT_F32 ? 4 : 2;           // bytes of an activation / scale / zero
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(A.x), (short)0, A.M * A.K * XE, RAW);
    uint32_t xa[MB][DT == DT_F32 ? 32 : 16];
#pragma unroll
    for (int b = 0; b < MB; ++b) {
        if constexpr (DT == DT_F32) load_x32(xr, tid < nrange && b < A.M, b, c0 + tid, A.K, xa[b]);
        else load_x(xr, tid < nrange && b < A.M, b, c0 + tid, A.K, xa[b]);
    }

    // 1b. the wave's packed chunks and their (scale, zero) halves
    int gi[CPL];
    bool cin[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = ks * SLICE + lane + 64 * i;
        cin[i] = c < nrange;
        gi[i] = (int)fdiv((uint32_t)(c0 + c), A.divGS);       // group of the chunk
    }
    // The wave's RPW rows, resolved once: v0 is a multiple of RPW, so gate-up rows alternate
    // gate / up from an even row, and fused QKV rows lie in one projection (the host keeps
    // the Q and K widths multiples of RPW).  A per-row map would put a chain of scalar
    // branches between the row loads.
    int proj0, r0;
    vmap<MODE>(A, min(v0, A.V - 1), proj0, r0);
    const Src S0 = MODE == MODE_QKV ? src_of(A, proj0) : A.src[0];
    ProjRes R[2];
    R[0] = proj_res(S0, A.G, XE);
    if constexpr (MODE == MODE_GATEUP) R[1] = proj_res(A.src[1], A.G, XE);
    uint32_t w[RPW][CPL][BITS];
    uint32_t sz[RPW][CPL][2];
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
        const int v = v0 + j;
        const bool vin = v < A.V;
        const int r = MODE == MODE_GATEUP ? r0 + (j >> 1) : r0 + j;
        const ProjRes& P = MODE == MODE_GATEUP ? R[j & 1] : R[0];
        const int wpr = MODE == MODE_GATEUP ? A.src[j & 1].wpr : S0.wpr;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = ks * SLICE + lane + 64 * i;
            const bool ok = vin && cin[i];
            const int so = vofs(ok, XE * (r * A.G + gi[i]));
            load_chunk<BITS>(P.w, vofs(ok, 4 * (r * wpr + (c0 + c) * BITS)), w[j][i]);
            if constexpr (DT == DT_F32) {
                sz[j][i][0] = __builtin_amdgcn_raw_buffer_load_b32(P.s, so, 0, 0);
                sz[j][i][1] = __builtin_amdgcn_raw_buffer_load_b32(P.z, so, 0, 0);
            } else {
                sz[j][i][0] = __builtin_amdgcn_raw_buffer_load_b16(P.s, so, 0, 0);
                sz[j][i][1] = __builtin_amdgcn_raw_buffer_load_b16(P.z, so, 0, 0);
            }
        }
        // rows are issued in the order they are consumed, so row j's arithmetic
        // waits for its own loads only
        __builtin_amdgcn_sched_barrier(0);
    }

    // 2. activations -> LDS: piece q of chunk c of operand row b at ((b * 4 + q) NCH + c) * 16,
    // (B, sum x[, 2^c]) at 64 MB SR NCH + XB (b NCH + c); chunks past the split read as zero
    // (they meet no weights).  Operand row b is batch row b, or for fp32 half b & 1 (hi, lo)
    // of batch row b >> 1.
    constexpr int XBB = XB_BYTES<DT>;
    constexpr int SR = SROWS<DT>;                       // staged operand rows per batch row
    u4* Xl = reinterpret_cast<u4*>(lds);
    char* XBl = lds + 64 * MB * SR * NCH;
    float* red = reinterpret_cast<float*>(lds + (64 + XBB) * MB * SR * NCH);
    if (tid < NCH) {
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            u4 X[4];
            float B, xs;
            if constexpr (DT == DT_F32) {
                u4 Xo[4];
                float Bo, xso, f;
                convert_x_f32<BITS>(xa[b], X, Xo, B, xs, Bo, xso, f);
                *reinterpret_cast<float4*>(XBl + XBB * ((2 * b) * NCH + tid)) = make_float4(B, xs, f, 0.f);
                *reinterpret_cast<float4*>(XBl + XBB * ((2 * b + 1) * NCH + tid)) = make_float4(Bo, xso, f, 0.f);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    Xl[((2 * b) * 4 + q) * NCH + tid] = X[q];
                    Xl[((2 * b + 1) * 4 + q) * NCH + tid] = Xo[q];
                }
                continue;
            } else if constexpr (DT == DT_BF16) {
                float f;
                convert_x_bf16<BITS>(xa[b], X, B, xs, f);
                *reinterpret_cast<float4*>(XBl + XBB * (b * NCH + tid)) = make_float4(B, xs, f, 0.f);
            } else {
                convert_x<BITS>(xa[b], X, B, xs);
                *reinterpret_cast<float2*>(XBl + XBB * (b * NCH + tid)) = make_float2(B, xs);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) Xl[(b * 4 + q) * NCH + tid] = X[q];
        }
    }
    lds_barrier();

    // 3. rows: each chunk is decoded once and meets every batch row's activations
    u4 X[MB * SR][CPL][4];
    float2 XB[MB * SR][CPL];
    float XF[MB * SR][CPL];              // 2^c of a bf16 or fp32 chunk
#pragma unroll
    for (int b = 0; b < MB * SR; ++b) {
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = ks * SLICE + lane + 64 * i;
#pragma unroll
            for (int q = 0; q < 4; ++q) X[b][i][q] = Xl[(b * 4 + q) * NCH + c];
            if constexpr (DT != DT_F16) {
                const float4 e = *reinterpret_cast<const float4*>(XBl + XBB * (b * NCH + c));
                XB[b][i] = make_float2(e.x, e.y);
                XF[b][i] = e.z;
            } else {
                XB[b][i] = *reinterpret_cast<const float2*>(XBl + XBB * (b * NCH + c));
                XF[b][i] = 1.f;
            }
        }
    }
    float acc[MB][RPW];
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
#pragma unroll
        for (int b = 0; b < MB; ++b) acc[b][j] = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            uint32_t h[16];
            Decode<BITS>::run(w[j][i], h, g);
            if constexpr (DT == DT_F32) {
                const h2 off = {(_Float16)1024.f, (_Float16)1024.f};
#pragma unroll
                for (int q = 0; q < 16; ++q) h[q] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, h[q]) - off);
            }
            const float s = meta_f<DT>(sz[j][i][0]);
            const float z = meta_f<DT>(sz[j][i][1]);
#pragma unroll
            for (int b = 0; b < MB; ++b) {
                // operand row SR b (fp32: hi), then for fp32 its lo row
                float t = pairs_dot(h, X[SR * b][i]) - fmaf(z, XB[SR * b][i].y, XB[SR * b][i].x);
#pragma unroll
                for (int r = 1; r < SR; ++r) {
                    const int sr = SR * b + r;
                    t += pairs_dot(h, X[sr][i]) - fmaf(z, XB[sr][i].y, XB[sr][i].x);
                }
                acc[b][j] = fmaf(s, DT == DT_F16 ? t : t * XF[SR * b][i], acc[b][j]);
            }
        }
    }

    // 4. row totals of the wave, per batch row, 4 rows at a time
#pragma unroll
    for (int b = 0; b < MB; ++b) {
#pragma unroll
        for (int q = 0; q < RPW / 4; ++q) {
            const float a4[4] = {acc[b][4 * q], acc[b][4 * q + 1], acc[b][4 * q + 2], acc[b][4 * q + 3]};
            const float tot = reduce4(a4);
            if ((lane & 15) == 0) red[(ks * MB + b) * RB + RPW * rw + 4 * q + lane_row(lane)] = tot;
        }
    }
    lds_barrier();
}

// 5. slices in order, then the finish stage (or the split's partials), a finish unit per
//    thread: MB RB / U <= 16 RW units against 64 KS RW threads, so one pass.  Kept out of
//    stream_body, so the mixed-width kernel carries one copy of it, not one per width.
// 6. with P > 1 and arrival counters, the last split of the block combines.
template <int MODE, int MB, int RPW, int DT>
__device__ __forceinline__ void stream_tail(const GemvArgs& A, char* lds) {
    const int tid = threadIdx.x;
    const int KS = A.st_ks, RB = RPW * A.st_rw;
    const int NCH = KS * SLICE;
    const int blk = (int)fdiv(blockIdx.x, A.divP);
    const int p = blockIdx.x - blk * A.P;
    const int vbase = blk * RB;
    const float* red = reinterpret_cast<const float*>(lds + (64 + XB_BYTES<DT>) * MB * SROWS<DT> * NCH);
    constexpr int U = FINISH_ROWS<MODE>;
    const int NU = RB / U;
    if (tid < MB * NU) {
        const int b = MB == 1 ? 0 : (tid >= NU ? 1 : 0);
        const int row = U * (tid - b * NU);
        const int v = vbase + row;
        if (b < A.M && v < A.V) {
            float y0 = 0.f, y1 = 0.f;
            for (int k = 0; k < KS; ++k) {
                y0 += red[(k * MB + b) * RB + row];
                if constexpr (U == 2) y1 += red[(k * MB + b) * RB + row + 1];
            }
            const bool two = U == 2 && v + 1 < A.V;
            if (A.P == 1) finish<DT, MODE>(A, b, v, y0, y1, two);
            else put_unit(A, p, b, v, y0, y1, two);
        }
    }
    if (A.P > 1 && A.split_cnt &&
        split_arrive(A, blk, reinterpret_cast<int*>(const_cast<float*>(red))))
        split_finish<DT, MODE>(A, vbase, RB, 64 * KS * A.st_rw);
}

// ------------------------------------------------------------------ batch rows 3..16
// (fp32: 2..8, each batch row staged as two fp16 operand rows, hi and lo, so the 16 MFMA
// batch rows hold 8 batch rows; a lane adds its hi and lo rows' totals at the end)
// Job = (block of RB = 16 RW virtual rows, K split p over 128-code units).  A
// workgroup holds KS x RW waves: wave (ks, rw) takes 16 rows of the block over K
// slice ks, BSU (4 or 8) units; lane (j = l & 15, kq = l >> 4) owns chunk 4 u + kq of row j
// for each unit u of the slice, so one buffer load per unit moves 16 rows x 4
// consecutive chunks.  The decoded chunk is the B operand of four
// v_mfma_f32_16x16x32_f16 whose A operand holds the M activation rows staged in
// the decode's operand order:
//   D[i][j] = sum_k x[i][k] (B(k) + q[j][k]) over the unit,
//   acc[i][j] += s[j] (D[i][j] - XB[i] - z[j] X[i])
// with X = sum x and XB = sum x B(k) over the unit (a unit is one group: the host
// requires g % 128 == 0).  The MFMA sums over k, so no cross-lane reduction is
// needed; lane (j, kq) holds batch rows 4 kq .. 4 kq + 3 of row j.  Gate-up rows
// alternate between the waves of a workgroup (even waves gate, odd waves up, the
// same 16 pair rows), so every wave's rows lie in one projection and its buffer
// descriptors stay uniform.

template <int BITS, int MODE, int BSU, int DT>
__device__ __forceinline__ void bstream_body(const GemvArgs& A, char* lds) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int KS = A.st_ks, RW = A.st_rw, RB = 16 * A.st_rw, M = A.M;
    const int NU = KS * BSU, NCH = 4 * NU;
    const int nthr = 64 * KS * RW;
    const int ks = (int)fdiv((uint32_t)wave, A.divRW);
    const int rw = wave - ks * RW;
    const int blk = (int)fdiv(blockIdx.x, A.divP);     // job = blk * P + p (split fastest)
    const int p = blockIdx.x - blk * A.P;
    // split p covers units [U p / P, U (p + 1) / P) of the row's U = ceil(C / 4)
    const int U = (A.C + 3) >> 2;
    const int u0 = (int)fdiv((uint32_t)(U * p), A.divP);
    const int u1 = (int)fdiv((uint32_t)(U * (p + 1)), A.divP);
    const int c0 = 4 * u0;                        // first chunk of the split
    const int nrange = min(4 * u1, A.C) - c0;     // its chunks
    const int vbase = blk * RB;
    const int j = lane & 15, kq = lane >> 4;
    const uint32_t g = magic_vreg();

    // the wave's 16 rows: virtual rows vbase + 16 rw + j, or for gate-up projection
    // rw & 1 of pair rows vbase / 2 + 16 (rw >> 1) + j (virtual rows 2 n + (rw & 1))
    int roff, vfirst;
    if constexpr (MODE == MODE_GATEUP) {
        vfirst = vbase + 32 * (rw >> 1) + (rw & 1);
        roff = 32 * (rw >> 1) + 2 * j + (rw & 1);
    } else {
        vfirst = vbase + 16 * rw;
        roff = 16 * rw + j;
    }
    const int vrow = vbase + roff;
    int proj, rfirst;
    vmap<MODE>(A, min(vfirst, A.V - 1), proj, rfirst);
    const int r = rfirst + j;                     // the lane's row in its projection
    const bool vin = vrow < A.V;

    // 1a. the thread's activation items t = tid + e * nthr, e < 2: (job chunk c, batch row
    // i) = (t mod NCH, t / NCH); the host keeps NCH * M <= 2 * nthr, so these are all of
    // them, and they are requested before the weights so that the staging waits for
    // them only
    constexpr int XE = DT == DT_F32 ? 4 : 2;           // bytes of an activation / scale / zero
    constexpr int OPR = DT == DT_F32 ? 2 : 1;          // operand rows per batch row (fp32: hi, lo)
    const int MR = OPR * M;                            // staged operand rows (<= 16)
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(A.x), (short)0, A.M * A.K * XE, RAW);
    uint32_t xa[2][DT == DT_F32 ? 32 : 16];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int t = tid + e * nthr, i = t / NCH, c = t - i * NCH;
        if constexpr (DT == DT_F32) load_x32(xr, i < M && c < nrange, i, c0 + c, A.K, xa[e]);
        else load_x(xr, i < M && c < nrange, i, c0 + c, A.K, xa[e]);
    }

    // 1b. the wave's packed chunks and the (scale, zero) of each unit's group
    // the wave's projection, selected once (by masks: no branches in front of the loads)
    const Src S = MODE == MODE_GEMV ? A.src[0] : src_of(A, proj);
    const ProjRes P = proj_res(S, A.G, XE);
    const int wpr = S.wpr;
    // the (scale, zero) of unit 4 e + kq's group of row j: BSU / 4 2-byte gathers each per
    // wave (lanes of a row then share them by ds_bpermute), rather than one per unit
    static_assert(BSU % 4 == 0, "whole units per lane quarter");
    uint32_t s_own[BSU / 4], z_own[BSU / 4];
#pragma unroll
    for (int e = 0; e < BSU / 4; ++e) {
        const int ul = ks * BSU + 4 * e + kq;
        const int gu = (int)fdiv((uint32_t)(u0 + ul), A.divG);   // the unit's group
        const int so = vofs(vin && 4 * ul < nrange, XE * (r * A.G + gu));
        if constexpr (DT == DT_F32) {
            s_own[e] = __builtin_amdgcn_raw_buffer_load_b32(P.s, so, 0, 0);
            z_own[e] = __builtin_amdgcn_raw_buffer_load_b32(P.z, so, 0, 0);
        } else {
            s_own[e] = __builtin_amdgcn_raw_buffer_load_b16(P.s, so, 0, 0);
            z_own[e] = __builtin_amdgcn_raw_buffer_load_b16(P.z, so, 0, 0);
        }
    }
    uint32_t w[BSU][BITS];
#pragma unroll
    for (int u = 0; u < BSU; ++u) {
        const int c = 4 * (ks * BSU + u) + kq;
        const bool ok = vin && c < nrange;
        load_chunk<BITS>(P.w, vofs(ok, 4 * (r * wpr + (c0 + c) * BITS)), w[u]);
        __builtin_amdgcn_sched_barrier(0);        // units issued in the order they are consumed
    }

    // 2. activations -> LDS: piece m of chunk c of operand row o at ((m NCH + c) MR + o) * 16;
    // per unit and operand row its sums X (at XSu[u * 16 + o]) and XB (XBu[u * 16 + o]), and
    // for bf16 and fp32 the unit's prescale 2^c (XFu[u * 16 + o]; the four chunks of a unit
    // share c, from their largest exponent, since the MFMA sums over the unit).  Operand row o
    // is batch row o, or for fp32 half o & 1 (hi, lo) of batch row o >> 1, whose decoded
    // pairs lose their 1024 (XB = 0).
    u4* Xl = reinterpret_cast<u4*>(lds);
    float* XSu = reinterpret_cast<float*>(lds + 64 * NCH * MR);
    float* XBu = XSu + 16 * NU;
    float* XFu = XBu + 16 * NU;
    float* red = XBu + (DT != DT_F16 ? 32 : 16) * NU;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int t = tid + e * nthr, i = t / NCH, c = t - i * NCH;
        if (t >= NCH * M) break;                  // whole quads of threads leave together (NCH % 4 == 0)
        if constexpr (DT == DT_F32) {
            int E = chunk_exp_f32(xa[e]);
            E = max(E, __shfl_xor(E, 1, 64));
            E = max(E, __shfl_xor(E, 2, 64));
            const int cu = prescale_bf16(E);
            u4 Xh[4], Xo[4];
            float xsh, xso;
            convert_x_f32_at<BITS>(xa[e], cu, Xh, Xo, xsh, xso);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                Xl[(m * NCH + c) * MR + 2 * i] = Xh[m];
                Xl[(m * NCH + c) * MR + 2 * i + 1] = Xo[m];
            }
            xsh += __shfl_xor(xsh, 1, 64);
            xso += __shfl_xor(xso, 1, 64);
            xsh += __shfl_xor(xsh, 2, 64);
            xso += __shfl_xor(xso, 2, 64);
            if ((c & 3) == 0) {
                const float f = __builtin_ldexpf(1.0f, cu);
                XSu[(c >> 2) * 16 + 2 * i] = xsh;
                XSu[(c >> 2) * 16 + 2 * i + 1] = xso;
                XBu[(c >> 2) * 16 + 2 * i] = 0.f;
                XBu[(c >> 2) * 16 + 2 * i + 1] = 0.f;
                XFu[(c >> 2) * 16 + 2 * i] = f;
                XFu[(c >> 2) * 16 + 2 * i + 1] = f;
            }
        } else {
            u4 X[4];
            float B, xs;
            int cu = 0;
            if constexpr (DT == DT_BF16) {
                int E = chunk_exp_bf16(xa[e]);
                E = max(E, __shfl_xor(E, 1, 64));
                E = max(E, __shfl_xor(E, 2, 64));
                cu = prescale_bf16(E);
                convert_x_bf16_at<BITS>(xa[e], cu, X, B, xs);
            } else {
                convert_x<BITS>(xa[e], X, B, xs);
            }
#pragma unroll
            for (int m = 0; m < 4; ++m) Xl[(m * NCH + c) * M + i] = X[m];
            // the 4 chunks of a unit are 4 consecutive threads (NCH % 4 == 0)
            B += __shfl_xor(B, 1, 64);
            xs += __shfl_xor(xs, 1, 64);
            B += __shfl_xor(B, 2, 64);
            xs += __shfl_xor(xs, 2, 64);
            if ((c & 3) == 0) {
                XSu[(c >> 2) * 16 + i] = xs;
                XBu[(c >> 2) * 16 + i] = B;
                if constexpr (DT == DT_BF16) XFu[(c >> 2) * 16 + i] = __builtin_ldexpf(1.0f, cu);
            }
        }
    }
    lds_barrier();

    // 3. units: A operands of operand row min(j, MR - 1) (rows past MR repeat a staged row;
    // their D rows are not stored)
    const int ia = min(j, MR - 1);
    f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < BSU; ++u) {
        const int uj = ks * BSU + u;              // job-local unit
        const int c = 4 * uj + kq;
        u4 a[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) a[m] = Xl[(m * NCH + c) * MR + ia];
        const f4 X4 = *reinterpret_cast<const f4*>(XSu + uj * 16 + 4 * kq);
        const f4 XB4 = *reinterpret_cast<const f4*>(XBu + uj * 16 + 4 * kq);
        uint32_t h[16];
        Decode<BITS>::run(w[u], h, g);
        if constexpr (DT == DT_F32) {
            const h2 off = {(_Float16)1024.f, (_Float16)1024.f};
#pragma unroll
            for (int q = 0; q < 16; ++q) h[q] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, h[q]) - off);
        }
        f4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const u4 bw = {h[4 * m], h[4 * m + 1], h[4 * m + 2], h[4 * m + 3]};
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const h8*>(&a[m]),
                                                       *reinterpret_cast<const h8*>(&bw), d, 0, 0, 0);
        }
        // unit u's scale and zero sit in lane (j, u % 4), set u / 4
        const uint32_t su = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (j + 16 * (u & 3)), (int)s_own[u >> 2]);
        const uint32_t zu = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (j + 16 * (u & 3)), (int)z_own[u >> 2]);
        const float sc = meta_f<DT>(su);
        const float ze = meta_f<DT>(zu);
        if constexpr (DT != DT_F16) {
            const f4 F4 = *reinterpret_cast<const f4*>(XFu + uj * 16 + 4 * kq);
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[q] = fmaf(sc, fmaf(-ze, X4[q], d[q] - XB4[q]) * F4[q], acc[q]);
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[q] = fmaf(sc, fmaf(-ze, X4[q], d[q] - XB4[q]), acc[q]);
        }
    }

    // 4. row totals per slice: lane (j, kq) holds operand rows 4 kq + q of row j (fp32: the
    // hi and lo rows of batch rows 2 kq and 2 kq + 1)
    if constexpr (DT == DT_F32) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int i = 2 * kq + h;
            if (i < M) red[(ks * M + i) * RB + roff] = acc[2 * h] + acc[2 * h + 1];
        }
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = 4 * kq + q;
            if (i < M) red[(ks * M + i) * RB + roff] = acc[q];
        }
    }
    lds_barrier();
}

// 5. slices in order, then the finish stage (or the split's partials), a finish unit per
//    thread; out of bstream_body, so the mixed-width kernel carries one copy.  Unit t is
//    (batch row t / NFU, row pair or row t % NFU), NFU = 16 RW / FU: the batch row is a
//    shift and the invariant division by RW.
// 6. with P > 1 and arrival counters, the last split of the block combines.
template <int MODE, int BSU, int DT>
__device__ __forceinline__ void bstream_tail(const GemvArgs& A, char* lds) {
    const int tid = threadIdx.x;
    const int KS = A.st_ks, RB = 16 * A.st_rw, M = A.M;
    const int NU = KS * BSU, NCH = 4 * NU;
    const int nthr = 64 * KS * A.st_rw;
    const int blk = (int)fdiv(blockIdx.x, A.divP);
    const int p = blockIdx.x - blk * A.P;
    const int vbase = blk * RB;
    constexpr int OPR = DT == DT_F32 ? 2 : 1;
    float* red = reinterpret_cast<float*>(lds + 64 * NCH * M * OPR) + (DT != DT_F16 ? 48 : 32) * NU;
    constexpr int FU = FINISH_ROWS<MODE>;
    constexpr int LOG = FU == 2 ? 3 : 4;          // log2(16 / FU)
    const int NFU = RB / FU;
    for (int t = tid; t < M * NFU; t += nthr) {
        const int b = (int)fdiv((uint32_t)(t >> LOG), A.divRW), ro = FU * (t - b * NFU);
        const int v = vbase + ro;
        if (v < A.V) {
            float y0 = 0.f, y1 = 0.f;
            for (int k = 0; k < KS; ++k) {
                y0 += red[(k * M + b) * RB + ro];
                if constexpr (FU == 2) y1 += red[(k * M + b) * RB + ro + 1];
            }
            const bool two = FU == 2 && v + 1 < A.V;
            if (A.P == 1) finish<DT, MODE>(A, b, v, y0, y1, two);
            else put_unit(A, p, b, v, y0, y1, two);
        }
    }
    if (A.P > 1 && A.split_cnt && split_arrive(A, blk, reinterpret_cast<int*>(red)))
        split_finish<DT, MODE>(A, vbase, RB, nthr);
}

// bf16 and fp32 with 8-unit slices: 768 threads at most, so 170 VGPRs (the per-unit
// prescale does not fit 128 next to eight units of streamed chunks); the planner keeps such
// workgroups to 12 waves.
template <int MODE, int BITS, int BSU, int DT>
__global__ void __launch_bounds__(DT != DT_F16 && BSU == 8 ? 768 : 1024) gemv_bstream_kernel(const GemvArgs A) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    if constexpr (BITS != 0) {
        bstream_body<BITS, MODE, BSU, DT>(A, lds);
    } else {
        int proj, r;
        vmap<MODE>(A, (int)fdiv(blockIdx.x, A.divP) * 16 * A.st_rw, proj, r);
        const int bits = bits_of(A, proj);
        if (bits == 2) bstream_body<2, MODE, BSU, DT>(A, lds);
        else if (bits == 3) bstream_body<3, MODE, BSU, DT>(A, lds);
        else bstream_body<4, MODE, BSU, DT>(A, lds);
    }
    bstream_tail<MODE, BSU, DT>(A, lds);
}

// BITS = 0: fused QKV with a width per projection; the host keeps each
// workgroup's rows inside one projection, so the width is uniform per workgroup.
// MB batch rows (1 or 2; rows past M are zero).  Wider batches stage MB copies of
// the activations, which at K = 11008 leaves one workgroup per CU; they take the
// batch-rows MFMA kernel instead.  RPW rows per wave (4, or 8 for the host's short-K
// batch-1 plan: half the waves for the same rows per workgroup).
template <int MODE, int BITS, int MB, int RPW, int DT>
__global__ void __launch_bounds__(1024) gemv_stream_kernel(const GemvArgs A) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    if constexpr (BITS != 0) {
        stream_body<BITS, MODE, MB, RPW, DT>(A, lds);
    } else {
        int proj, r;
        vmap<MODE>(A, (int)fdiv(blockIdx.x, A.divP) * RPW * A.st_rw, proj, r);
        const int bits = bits_of(A, proj);
        if (bits == 2) stream_body<2, MODE, MB, RPW, DT>(A, lds);
        else if (bits == 3) stream_body<3, MODE, MB, RPW, DT>(A, lds);
        else stream_body<4, MODE, MB, RPW, DT>(A, lds);
    }
    stream_tail<MODE, MB, RPW, DT>(A, lds);
}

template <int MB, int RPW, int DT>
const void* stream_kernel(int mode, int bits, bool mixed) {
    if (mixed) return reinterpret_cast<const void*>(&gemv_stream_kernel<MODE_QKV, 0, MB, RPW, DT>);
#define CBK_STREAM_K(M)                                                                            \
    (bits == 2 ? reinterpret_cast<const void*>(&gemv_stream_kernel<M, 2, MB, RPW, DT>)             \
               : (bits == 3 ? reinterpret_cast<const void*>(&gemv_stream_kernel<M, 3, MB, RPW, DT>)\
                            : reinterpret_cast<const void*>(&gemv_stream_kernel<M, 4, MB, RPW, DT>)))
    if (mode == MODE_QKV) return CBK_STREAM_K(MODE_QKV);
    if (mode == MODE_GATEUP) return CBK_STREAM_K(MODE_GATEUP);
    return CBK_STREAM_K(MODE_GEMV);
#undef CBK_STREAM_K
}

template <int BSU, int DT>
const void* bstream_kernel(int mode, int bits, bool mixed) {
    if (mixed) return reinterpret_cast<const void*>(&gemv_bstream_kernel<MODE_QKV, 0, BSU, DT>);
#define CBK_BSTREAM_K(M)                                                                           \
    (bits == 2 ? reinterpret_cast<const void*>(&gemv_bstream_kernel<M, 2, BSU, DT>)                \
               : (bits == 3 ? reinterpret_cast<const void*>(&gemv_bstream_kernel<M, 3, BSU, DT>)   \
                            : reinterpret_cast<const void*>(&gemv_bstream_kernel<M, 4, BSU, DT>)))
    if (mode == MODE_QKV) return CBK_BSTREAM_K(MODE_QKV);
    if (mode == MODE_GATEUP) return CBK_BSTREAM_K(MODE_GATEUP);
    return CBK_BSTREAM_K(MODE_GEMV);
#undef CBK_BSTREAM_K
}

}  // namespace

template <int DT>
const void* stream_kernel_dt(int mode, int bits, bool mixed, int mb, int rpw) {
    if constexpr (DT != DT_F32)                        // fp32 streams at batch 1 only
        if (mb > 1) return stream_kernel<2, STREAM_RPW, DT>(mode, bits, mixed);
    if (rpw == STREAM_RPW_WIDE && mode == MODE_GEMV && !mixed) {     // the host plans 8 rows for plain GEMVs only
        constexpr int W = STREAM_RPW_WIDE;
        return bits == 2 ? reinterpret_cast<const void*>(&gemv_stream_kernel<MODE_GEMV, 2, 1, W, DT>)
                         : (bits == 3 ? reinterpret_cast<const void*>(&gemv_stream_kernel<MODE_GEMV, 3, 1, W, DT>)
                                      : reinterpret_cast<const void*>(&gemv_stream_kernel<MODE_GEMV, 4, 1, W, DT>));
    }
    return stream_kernel<1, STREAM_RPW, DT>(mode, bits, mixed);
}

const void* gemv_stream_kernel_for(int mode, int bits, bool mixed, int mb, int rpw, int dt) {
    return dt == DT_BF16 ? stream_kernel_dt<DT_BF16>(mode, bits, mixed, mb, rpw)
                         : (dt == DT_F32 ? stream_kernel_dt<DT_F32>(mode, bits, mixed, mb, rpw)
                                         : stream_kernel_dt<DT_F16>(mode, bits, mixed, mb, rpw));
}

const void* gemv_bstream_kernel_for(int mode, int bits, bool mixed, int bsu, int dt) {
    if (dt == DT_BF16)
        return bsu == 8 ? bstream_kernel<8, DT_BF16>(mode, bits, mixed) : bstream_kernel<4, DT_BF16>(mode, bits, mixed);
    if (dt == DT_F32)
        return bsu == 8 ? bstream_kernel<8, DT_F32>(mode, bits, mixed) : bstream_kernel<4, DT_F32>(mode, bits, mixed);
    return bsu == 8 ? bstream_kernel<8, DT_F16>(mode, bits, mixed) : bstream_kernel<4, DT_F16>(mode, bits, mixed);
}


}  // namespace cbk
