// abi.cpp -- the extern "C" entry points of libcrispybits_hip.so (include/crispybits_hip.h).
//
// Replaces the reference's host glue: argument checks of host_utils.h:49-93,
// launch planning of packed_gemv.cu:182-238 / packed_gemm.cu:158-203, and the
// module exports of bindings.cpp:32-40.  Every check runs before the first HIP
// call, so invalid arguments are reported without touching a device.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "crispybits_hip.h"
#include "cbk_kernels.hpp"

using namespace cbk;

namespace {

// Measurement timer: while armed, each launch gets its own start/stop event pair
// recorded by the dispatch itself (hipExtLaunchKernel), so the durations exclude
// host overhead and the gaps between launches.
struct Timer {
    std::mutex mu;
    bool armed = false;
    int used = 0;
    std::vector<hipEvent_t> ev;    // 2 per launch slot
} g_timer;

}  // namespace

namespace cbk {

hipError_t launch(const void* f, dim3 grid, dim3 block, void** args, size_t lds, hipStream_t stream) {
    hipEvent_t start = nullptr, stop = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_timer.mu);
        if (g_timer.armed && 2 * (g_timer.used + 1) <= (int)g_timer.ev.size()) {
            start = g_timer.ev[2 * g_timer.used];
            stop = g_timer.ev[2 * g_timer.used + 1];
            ++g_timer.used;
        }
    }
    if (start) return hipExtLaunchKernel(f, grid, block, args, lds, stream, start, stop, 0);
    return hipLaunchKernel(f, grid, block, args, lds, stream);
}

}  // namespace cbk

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(CBK_EHIP, "%s: %s", what, hipGetErrorString(e));
}

// Switches to `device` for the duration of a call (the reference's CUDAGuard).
struct DeviceGuard {
    int prev = -1;
    hipError_t err = hipSuccess;
    explicit DeviceGuard(int device) {
        err = hipGetDevice(&prev);
        if (err == hipSuccess && prev != device) err = hipSetDevice(device);
        else if (err != hipSuccess) prev = -1;
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

constexpr int MAX_DEVICES = 64;
int g_cu[MAX_DEVICES];
std::once_flag g_cu_once[MAX_DEVICES];

int cu_count(int device) {
    if (device < 0 || device >= MAX_DEVICES) return 0;
    std::call_once(g_cu_once[device], [device] {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) v = 0;
        g_cu[device] = v;
    });
    return g_cu[device];
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Split-K partial sums of the allocation-free decode entry point (cbk_packed_gemv_noalloc):
// a file-scope device array, one copy per GPU, held until the process ends.  Host code
// never passes `scratch` itself (on the host it names a stand-in, not device memory): it
// looks up each device's address once, with that device current, and passes that.
constexpr int64_t NOALLOC_PARTIAL_FLOATS = CBK_NOALLOC_PARTIAL_FLOATS;
static __device__ __align__(256) float scratch[NOALLOC_PARTIAL_FLOATS];
float* g_scratch[MAX_DEVICES];
hipError_t g_scratch_err[MAX_DEVICES];
std::once_flag g_scratch_once[MAX_DEVICES];

// This device's copy of `scratch`; the caller has made `device` current.
hipError_t scratch_for(int device, float** out) {
    if (device < 0 || device >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::call_once(g_scratch_once[device], [device] {
        void* p = nullptr;
        g_scratch_err[device] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch[device] = g_scratch_err[device] == hipSuccess ? static_cast<float*>(p) : nullptr;
    });
    *out = g_scratch[device];
    return g_scratch_err[device];
}

// Arrival counters of the in-dispatch split-K combine (split_arrive, cbk_device.hpp):
// one word per row block of a call, zero between calls (the combining workgroup resets
// its word).  A file-scope device array, one copy per GPU, cut into windows.  A window
// has one holder for good:
//  * a stream, for its eager calls -- calls on one stream run in order, so one window
//    serves all of them;
//  * a graph capture -- the captured launches keep the window's address and may be
//    replayed at any time on any stream, so the window is never handed to eager calls
//    or to another capture.
// A window is never taken from its holder (a stream may still have split calls in
// flight).  A call that finds no window of its own and no free one, or whose row blocks
// outnumber a window's counters, takes the combine launch instead: correct, one launch
// more.  One graph must not be replayed while another replay of it runs.
constexpr int SPLIT_WINDOWS = 256;
constexpr int SPLIT_COUNTERS = 4096;
static __device__ __align__(256) uint32_t split_counters[SPLIT_WINDOWS * SPLIT_COUNTERS];

struct SplitWindows {
    std::mutex mu;
    uint32_t* base = nullptr;
    hipError_t err = hipSuccess;
    bool init = false;
    int used = 0;                                   // windows [0, used) have holders
    bool by_capture[SPLIT_WINDOWS];
    hipStream_t stream[SPLIT_WINDOWS];              // holder stream (eager windows)
    unsigned long long capture[SPLIT_WINDOWS];      // holder capture id (capture windows)
};
SplitWindows g_split[MAX_DEVICES];

// The counter window of this call on `device` (made current by the caller), or nullptr.
uint32_t* split_window(int device, hipStream_t stream) {
    if (device < 0 || device >= MAX_DEVICES) return nullptr;
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    unsigned long long id = 0;
    if (hipStreamGetCaptureInfo(stream, &st, &id) != hipSuccess) return nullptr;
    const bool cap = st == hipStreamCaptureStatusActive;
    SplitWindows& W = g_split[device];
    std::lock_guard<std::mutex> lk(W.mu);
    if (!W.init) {
        void* p = nullptr;
        W.err = hipGetSymbolAddress(&p, HIP_SYMBOL(split_counters));
        W.base = W.err == hipSuccess ? static_cast<uint32_t*>(p) : nullptr;
        W.init = true;
    }
    if (!W.base) return nullptr;
    int slot = -1;
    for (int i = 0; i < W.used && slot < 0; ++i)
        if (W.by_capture[i] == cap && (cap ? W.capture[i] == id : W.stream[i] == stream)) slot = i;
    if (slot < 0) {
        if (W.used == SPLIT_WINDOWS) return nullptr;
        slot = W.used++;
        W.by_capture[slot] = cap;
        W.stream[slot] = cap ? nullptr : stream;
        W.capture[slot] = cap ? id : 0;
    }
    return W.base + (size_t)slot * SPLIT_COUNTERS;
}

constexpr int MFMA_TILE = 16;          // virtual rows per decode job tile (the policy's tile_n)
constexpr int LDS_BUDGET = 160 * 1024; // dynamic LDS per decode workgroup (gfx950: 160 KB per CU)
constexpr int ANY_FILL_WAVES = 4096;   // waves the fp32 matrix-core decode aims for
constexpr int ANY_MIN_CHUNKS = 4;      // ... keeping at least this many chunks per wave

bool valid_dtype(int dt) { return dt == CBK_F16 || dt == CBK_BF16 || dt == CBK_F32; }

int check_weight(const int32_t* packed, const void* scales, const void* zeros, int64_t n, int bits,
                 int group_size, const char* name) {
    if (!packed || !scales || !zeros) return fail(CBK_EINVAL, "%s: packed/scales/zeros must be non-null", name);
    if (n <= 0) return fail(CBK_EINVAL, "%s: out_features must be positive", name);
    if (n > (1 << 30)) return fail(CBK_EINVAL, "%s: out_features too large", name);
    if (bits != 2 && bits != 3 && bits != 4) return fail(CBK_EINVAL, "%s: bits must be 2/3/4", name);
    if (group_size <= 0 || group_size % 32 != 0)
        return fail(CBK_EINVAL, "%s: group_size must be a positive multiple of 32", name);
    const uintptr_t align = bits == 4 ? 16 : (bits == 2 ? 8 : 4);
    if (reinterpret_cast<uintptr_t>(packed) % align != 0)
        return fail(CBK_EINVAL, "%s: packed storage must be %d-byte aligned for vector loads", name, (int)align);
    return CBK_OK;
}

int check_x(const void* x, int dtype, int64_t M, int64_t K) {
    if (!valid_dtype(dtype)) return fail(CBK_EINVAL, "x must be fp16/bf16/fp32");
    if (M < 0) return fail(CBK_EINVAL, "x must be [B,K] with B >= 0");
    if (K <= 0 || K > (1 << 24)) return fail(CBK_EINVAL, "in_features must be in [1, 2^24]");
    if (M > 0 && !x) return fail(CBK_EINVAL, "x must be non-null");
    if (M > (1 << 24)) return fail(CBK_EINVAL, "too many rows in x");
    return CBK_OK;
}

// ----------------------------------------------------------------------------- decode plan
// Plan of the fp32 matrix-core decode (gemv_any.hip): jobs of 16 virtual rows x 16 batch
// rows x one K split (the requested one), one workgroup each.  The CUs are filled with
// waves rather than extra splits -- a split needs a partial buffer the caller sized for
// its own split_k: a job's workgroup takes enough waves (1..16) that the launch holds
// about ANY_FILL_WAVES waves (four per SIMD of the 256-CU parts), while every wave keeps
// at least ANY_MIN_CHUNKS chunks of its split.  rho is not used: the kernel is not
// persistent.
struct AnyPlan {
    int P = 1, ntiles = 0, mtiles = 0, waves = 1;
    int64_t jobs = 0;
};

AnyPlan plan_any(int64_t M, int64_t V, int64_t K, int split_k) {
    AnyPlan pl;
    const int64_t C = ceil_div(K, 32);
    pl.ntiles = (int)ceil_div(V, 16);
    pl.mtiles = (int)ceil_div(std::max<int64_t>(M, 1), 16);
    pl.P = (int)std::max<int64_t>(1, std::min<int64_t>(split_k, C));
    pl.jobs = (int64_t)pl.ntiles * pl.mtiles * pl.P;
    const int64_t chunks = ceil_div(C, pl.P);
    int64_t w = ceil_div(ANY_FILL_WAVES, pl.jobs);
    w = std::min<int64_t>(w, std::max<int64_t>(1, chunks / ANY_MIN_CHUNKS));
    pl.waves = (int)std::max<int64_t>(1, std::min<int64_t>(w, ANY_MAX_THREADS / 64));
    return pl;
}

// Streaming plan (gemv_stream.hip), batch 1 or 2: fp16 or bf16 x (fp32 x at batch 1) with 16-byte pieces, any group
// size that is a multiple of 32, 32-bit byte offsets into every tensor, and for
// mixed-width QKV workgroups that stay inside one projection.  The K range of a
// split is cut into slices of 64 * STREAM_CPL chunks (one wave each, within the launch bound);
// rows go rpw to a wave, RW row groups to a workgroup.  A plain GEMV at batch 1 with
// at most two slices (K <= 4096 at one split) takes 8 rows a wave in two row groups:
// the same 16 rows per workgroup from half the waves (4096^2 W3: 4.5 -> 4.1 us per
// call; fused QKV measured 3 % slower that way and keeps 4).
struct StreamPlan {
    bool ok = false;
    int P = 1, ks = 1, rw = 2, rpw = STREAM_RPW, mb = 1, grid = 0, lds = 0;
};

// Bytes the streaming kernel stages per chunk and batch row: 64 of operand pairs, then
// (B, sum x), and for bf16 the chunk's power-of-two prescale as well; fp32 stages two such
// operand rows (hi, lo) per batch row.
int stream_chunk_bytes(int dtype) { return dtype == CBK_F32 ? 160 : (dtype == CBK_BF16 ? 80 : 72); }

// Slices a streaming job may hold: one wave each within the launch bound (16 waves),
// and the staged activations per chunk and batch row plus the row-sum area (at most
// 16 slices x 2 rows x 16 rows x 4 bytes) in the LDS.
int stream_max_slices(int mb, int dtype) {
    const int waves = 16 / STREAM_CPL;
    const int lds = (LDS_BUDGET - 16 * 2 * 16 * 4) / (64 * STREAM_CPL * stream_chunk_bytes(dtype) * mb);
    return std::max(1, std::min(waves, lds));
}

// K splits of the streaming kernel: the requested split, raised until a split's
// chunks fit `max_slices` slices of 64 * STREAM_CPL.
int stream_splits(int64_t C, int split_k, int max_slices) {
    const int64_t slice = 64 * STREAM_CPL;
    int64_t P = std::max<int64_t>(1, std::min<int64_t>(split_k, C));
    while (ceil_div(ceil_div(C, P), slice) > max_slices && P < C) ++P;
    return (int)P;
}

StreamPlan plan_stream(const GemvArgs& A, int dtype, int mode, bool mixed, int split_k) {
    StreamPlan sp;
    const int64_t lim = INT32_MAX;
    // fp32 x streams at batch 1 (two fp16 operand rows); at batch 2 the batched kernel, which
    // stages the four operand rows once per workgroup and takes the products on MFMAs, is as
    // fast or faster at every shape (W3 4096^2 / 4096 -> 11008 / 11008 -> 4096: 6.74 / 12.37 /
    // 14.60 us against 6.89 / 16.90 / 14.75 on a 512-thread build of this kernel)
    const int xe = dtype == CBK_F32 ? 4 : 2;
    bool ok = A.M >= 1 && A.M <= (dtype == CBK_F32 ? 1 : 2) && valid_dtype(dtype) && A.gs % 32 == 0 &&
              A.K % 8 == 0 && reinterpret_cast<uintptr_t>(A.x) % 16 == 0 && (int64_t)A.M * A.K * xe < lim;
    for (int i = 0; i < 3; ++i)
        ok = ok && (int64_t)A.src[i].n * A.src[i].wpr * 4 < lim && (int64_t)A.src[i].n * A.G * xe < lim;
    if (!ok) return sp;
    sp.mb = A.M;
    const int max_waves = 16;                           // the kernel's launch bound: 1024 threads
    const int64_t slice = 64 * STREAM_CPL;
    sp.P = stream_splits(A.C, split_k, stream_max_slices(sp.mb, dtype));
    if ((int64_t)A.C * sp.P >= (1ll << 32)) return sp;     // split bounds C p / P in 32 bits
    sp.ks = (int)ceil_div(ceil_div(A.C, sp.P), slice);
    if (sp.ks * STREAM_CPL > max_waves) return sp;
    sp.rw = sp.ks <= 2 ? 4 : 2;
    sp.rw = std::max(STREAM_CPL, std::min(sp.rw, max_waves / sp.ks));
    if (sp.mb == 1 && sp.ks <= 2 && mode == CBK_MODE_GEMV && !mixed) {
        sp.rpw = STREAM_RPW_WIDE;
        sp.rw = std::max(STREAM_CPL, sp.rw / 2);
    }
    const int rb = sp.rpw * sp.rw;
    if (mixed && (A.src[0].n % rb != 0 || A.src[1].n % rb != 0)) return sp;
    // a wave's rows lie in one projection (the kernel resolves them once per wave)
    if (mode == CBK_MODE_QKV && (A.src[0].n % sp.rpw != 0 || A.src[1].n % sp.rpw != 0)) return sp;
    const int64_t grid = ceil_div(A.V, rb) * sp.P;
    if (grid >= lim) return sp;
    sp.grid = (int)grid;
    sp.lds = (int)(sp.ks * slice * stream_chunk_bytes(dtype) * sp.mb + (int64_t)sp.ks * sp.mb * rb * 4);
    sp.ok = true;
    return sp;
}

// Batched streaming plan (gemv_stream.hip, bstream), batch 3..16 for fp16 or bf16 x and
// 2..8 for fp32 x, with 16-byte pieces, group sizes that are multiples of 128 (a unit of 128 codes is one
// group), 32-bit offsets, and rows that keep every 16-row tile inside one projection
// (fused QKV: Q and K widths multiples of 16; mixed widths: of the workgroup's rows).
// K is split over units; a split's units are cut into slices of bsu units (one wave
// each, at most 16 waves): 4 where that needs no split, else 8.  The split grows until
// the staged activations (64 bytes per chunk and batch row), the unit sums and the row
// sums fit the LDS; the splits of a row block combine inside the dispatch
// (split_arrive), so a split costs no second launch.
struct BStreamPlan {
    bool ok = false;
    bool filled = false;         // chosen by bstream_fill
    int P = 1, ks = 1, rw = 1, bsu = 4, grid = 0, lds = 0;
};

// LDS of a batched streaming workgroup: the staged activations (xr operand rows per batch
// row: 2 for fp32, hi and lo), two per-unit sums (three for bf16 and fp32: the per-unit
// prescale) for 16 operand rows, and the row totals.
int64_t bstream_lds(int64_t ks, int64_t M, int64_t rw, int bsu, bool bf, int xr = 1) {
    const int64_t nu = ks * bsu;
    return 64 * 4 * nu * M * xr + (bf ? 3 : 2) * 16 * nu * 4 + 4 * ks * M * 16 * rw;
}

// Row groups: enough threads to stage the activations two items per thread (4 bsu M
// items over 64 threads per wave), and for gate-up an even count (one wave per
// projection of 16 pair rows).
int bstream_rw(int64_t M, int bsu, bool gateup) {
    int rw = (int)std::max<int64_t>(1, ceil_div(M * bsu, 32));
    if (gateup) rw = (rw + 1) & ~1;
    return rw;
}

// Waves a batched streaming workgroup may hold: 16, or 12 for bf16 and fp32 (`bf`: a per-unit
// prescale) with 8-unit slices (that kernel is built for 768 threads, so it has 170 VGPRs).
int bstream_max_waves(int bsu, bool bf) { return bf && bsu == 8 ? 12 : 16; }

// K splits of the batched streaming kernel for slices of bsu units.
int bstream_splits(int64_t C, int64_t M, int split_k, int rw, int bsu, bool bf, int xr = 1) {
    const int64_t U = ceil_div(C, 4);
    int64_t P = std::max<int64_t>(1, std::min<int64_t>(split_k, U));
    while (P < U) {
        const int64_t ks = ceil_div(ceil_div(U, P), bsu);
        if (ks * rw <= bstream_max_waves(bsu, bf) && bstream_lds(ks, M, rw, bsu, bf, xr) <= LDS_BUDGET) break;
        ++P;
    }
    return (int)P;
}

// The plan (P, bsu, rw) of the batched streaming kernel, checked against what the kernel
// assumes: a wave per slice and row group within 16 waves, every activation item staged
// by at most two threads, an even number of row groups for gate-up, the LDS, one
// projection per workgroup for mixed widths, 32-bit indices, and with P > 1 a counter
// per row block in one window (the splits combine in the dispatch).
BStreamPlan bstream_make(const GemvArgs& A, int mode, bool mixed, int P, int bsu, int rw, bool bf, int xr = 1) {
    BStreamPlan bp;
    const int64_t U = ceil_div(A.C, 4);
    if (P < 1 || P > U || (int64_t)U * P >= (1ll << 32)) return bp;
    if (rw < bstream_rw(A.M, bsu, mode == CBK_MODE_GATEUP) || (mode == CBK_MODE_GATEUP && rw % 2)) return bp;
    bp.P = P;
    bp.bsu = bsu;
    bp.rw = rw;
    bp.ks = (int)ceil_div(ceil_div(U, P), bsu);
    if (bp.ks * rw > bstream_max_waves(bsu, bf)) return bp;
    bp.lds = (int)bstream_lds(bp.ks, A.M, rw, bsu, bf, xr);
    if (bp.lds > LDS_BUDGET) return bp;
    const int rb = 16 * rw;
    if (mixed && (A.src[0].n % rb != 0 || A.src[1].n % rb != 0)) return bp;
    const int64_t blocks = ceil_div(A.V, rb);
    if (P > 1 && blocks > SPLIT_COUNTERS) return bp;
    if (blocks * P >= INT32_MAX) return bp;
    bp.grid = (int)(blocks * P);
    bp.ok = true;
    return bp;
}

// A batched call whose unsplit plan would leave half the CUs without a workgroup, or that
// needs K splits anyway, takes the plan with P in [P0, P0 + 3] whose workgroup count is
// closest to one per CU (then the fewest splits, the shorter slices, the fewest row
// groups): each CU then converts only its split's activations.  Measured on W3 at the
// Llama-2-7B shapes (us per call): 11008 -> 4096 batch 8 15.4 (whole-K batch kernel) ->
// 13.6 (P = 2, 8-unit slices, 2 row groups), batch 16 18.1 -> 16.3 (P = 4, 4 row
// groups); 4096^2 batch 16 10.1 -> 8.9 (P = 2).  The target is a constant -- the CU count
// of every gfx950 part -- so cbk_gemv_partial_floats can bound P without a device.
constexpr int BSTREAM_CU_TARGET = 256;
constexpr int BSTREAM_FILL_SPLITS = 4;

BStreamPlan bstream_fill(const GemvArgs& A, int mode, bool mixed, int P0, bool bf, int xr = 1) {
    BStreamPlan best;
    int64_t best_key = INT64_MAX;
    for (int P = P0; P < P0 + BSTREAM_FILL_SPLITS; ++P) {
        for (int bsu : {4, 8}) {
            for (int rw = 1; rw <= 16; ++rw) {
                const BStreamPlan c = bstream_make(A, mode, mixed, P, bsu, rw, bf, xr);
                if (!c.ok) continue;
                const int64_t dist = std::abs((int64_t)c.grid - BSTREAM_CU_TARGET);
                const int64_t key = ((dist * 64 + (P - P0)) * 2 + (bsu == 8)) * 32 + rw;
                if (key < best_key) {
                    best_key = key;
                    best = c;
                }
            }
        }
    }
    return best;
}

// The unsplit-first plan before any widening for the CU count: 4-unit slices with the
// fewest splits that fit, or 8-unit slices where those need fewer splits.
BStreamPlan bstream_base(int64_t M, int64_t C, int split_k, bool gateup, bool bf, int xr = 1) {
    BStreamPlan bp;
    bp.bsu = 4;
    bp.rw = bstream_rw(M, 4, gateup);
    bp.P = bstream_splits(C, M, split_k, bp.rw, 4, bf, xr);
    if (bp.P > std::max(split_k, 1)) {           // 4-unit slices would add a split: try 8
        const int rw8 = bstream_rw(M, 8, gateup);
        const int p8 = bstream_splits(C, M, split_k, rw8, 8, bf, xr);
        if (p8 < bp.P) {
            bp.bsu = 8;
            bp.rw = rw8;
            bp.P = p8;
        }
    }
    return bp;
}

// Whether a call with this base plan takes bstream_fill's plan.
bool bstream_fills(const BStreamPlan& base, int64_t V) {
    return base.P > 1 || ceil_div(V, 16 * base.rw) * base.P * 2 <= BSTREAM_CU_TARGET;
}

BStreamPlan plan_bstream(const GemvArgs& A, int dtype, int mode, bool mixed, int split_k, int cus) {
    BStreamPlan bp;
    const int64_t lim = INT32_MAX;
    // bf16 with 8-unit slices runs a 768-thread build of the kernel (its per-unit prescale
    // does not fit 128 VGPRs next to eight units of chunks; 170 hold it), so its plans keep to
    // 12 waves (bstream_max_waves).  W3 11008 -> 4096 batch 8: 22.7 us on the 1024-thread
    // build, which spilled, 19.3 on 4-unit slices, 14.8 on the 768-thread build (fp16 13.8).
    // fp32 x stages two fp16 operand rows (hi, lo) per batch row (16 operand rows at most: batch
    // 2..8) with a per-unit prescale like bf16's.
    const bool bf = dtype != CBK_F16;
    const int xr = dtype == CBK_F32 ? 2 : 1, xe = dtype == CBK_F32 ? 4 : 2;
    const int mmin = dtype == CBK_F32 ? 2 : 3;         // below: the batch-1/2 streaming kernel
    bool ok = A.M >= mmin && A.M * xr <= 16 && valid_dtype(dtype) && A.gs % 128 == 0 && A.K % 8 == 0 &&
              reinterpret_cast<uintptr_t>(A.x) % 16 == 0 && (int64_t)A.M * A.K * xe < lim;
    for (int i = 0; i < 3; ++i)
        ok = ok && (int64_t)A.src[i].n * A.src[i].wpr * 4 < lim && (int64_t)A.src[i].n * A.G * xe < lim;
    if (mode == CBK_MODE_QKV) ok = ok && A.src[0].n % 16 == 0 && A.src[1].n % 16 == 0;
    if (!ok) return bp;
    const bool gateup = mode == CBK_MODE_GATEUP;
    const int64_t U = ceil_div(A.C, 4);
    bp = bstream_base(A.M, A.C, split_k, gateup, bf, xr);
    if (bstream_fills(bp, A.V)) {
        BStreamPlan fill = bstream_fill(A, mode, mixed, std::max(split_k, 1), bf, xr);
        if (fill.ok) {
            fill.filled = true;
            return fill;
        }
    }
    // Every workgroup converts all of its split's activations, so at many rows the
    // activation work, not the weight stream, sets the time: plain GEMVs whose 16-row
    // blocks would give each CU 2.5 or more workgroups take 8-unit slices and the
    // fewest workgroups that still cover the CUs (W3 4096 -> 11008: batch 8 13.2 -> 11.1
    // us, batch 16 18.8 -> 14.5), and gate-up takes 8-unit slices (batch 4 20.4 -> 15.6).
    if (bp.P == 1 && cus > 0) {
        const int64_t U8 = ceil_div(U, 8);
        const int mw = bstream_max_waves(8, bf);
        if (mode == CBK_MODE_GEMV && !mixed && ceil_div(A.V, 16) >= (5 * (int64_t)cus) / 2) {
            int rw = (int)std::max<int64_t>(bstream_rw(A.M, 8, false), ceil_div(ceil_div(A.V, 16), cus));
            if (U8 * rw <= mw && bstream_lds(U8, A.M, rw, 8, bf, xr) <= LDS_BUDGET) {
                bp.bsu = 8;
                bp.rw = rw;
            }
        } else if (gateup) {
            const int rw = bstream_rw(A.M, 8, true);
            if (U8 * rw <= mw && bstream_lds(U8, A.M, rw, 8, bf, xr) <= LDS_BUDGET) {
                bp.bsu = 8;
                bp.rw = rw;
            }
        }
    }
    return bstream_make(A, mode, mixed, bp.P, bp.bsu, bp.rw, bf, xr);
}

// Kernels (per device) whose dynamic-LDS limit has been raised to the whole budget.  The
// limit is set once, to LDS_BUDGET, and never lowered, so launches of one kernel with
// different LDS sizes from several threads cannot undercut each other.
std::mutex g_attr_mu;
std::vector<std::pair<int, const void*>> g_lds_raised;

hipError_t ensure_lds(const void* f, int bytes) {
    if (bytes <= 64 * 1024) return hipSuccess;
    if (bytes > LDS_BUDGET) return hipErrorInvalidValue;
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const std::pair<int, const void*> key(dev, f);
    std::lock_guard<std::mutex> lk(g_attr_mu);
    if (std::find(g_lds_raised.begin(), g_lds_raised.end(), key) != g_lds_raised.end()) return hipSuccess;
    e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BUDGET);
    if (e == hipSuccess) g_lds_raised.push_back(key);
    return e;
}

// The launch a decode call makes: kernel family, the kernel, its grid, workgroup size,
// dynamic LDS and K splits.  plan_decode also fills the plan fields of A the kernels read.
struct DecodeLaunch {
    int family = 0;              // CBK_KERNEL_*
    const void* f = nullptr;     // kernel address
    int grid = 0, block = 0, lds = 0, P = 1;
};

DecodeLaunch plan_decode(GemvArgs& A, int dtype, int mode, bool mixed, int split_k, int rho, int cus) {
    (void)rho;
    DecodeLaunch L;
    // batch 1 and 2: the streaming kernel
    const StreamPlan sp = plan_stream(A, dtype, mode, mixed, split_k);
    if (sp.ok) {
        A.P = sp.P;
        A.st_ks = sp.ks;
        A.st_rw = sp.rw;
        A.divP = make_fastdiv((uint32_t)A.P);
        A.divRW = make_fastdiv((uint32_t)A.st_rw);
        A.divGS = make_fastdiv((uint32_t)(A.gs / 32));
        L.family = CBK_KERNEL_STREAM;
        L.f = gemv_stream_kernel_for(mode, A.bits[0], mixed, sp.mb, sp.rpw, dtype);
        L.grid = sp.grid;
        L.block = 64 * sp.ks * sp.rw;
        L.lds = sp.lds;
        L.P = sp.P;
        return L;
    }
    // batch 3..16: the K-split streaming kernel (unsplit, or splits that combine in the
    // dispatch)
    const BStreamPlan bp = plan_bstream(A, dtype, mode, mixed, split_k, cus);
    if (bp.ok) {
        A.P = bp.P;
        A.st_ks = bp.ks;
        A.st_rw = bp.rw;
        A.divP = make_fastdiv((uint32_t)A.P);
        A.divRW = make_fastdiv((uint32_t)A.st_rw);
        A.divG = make_fastdiv((uint32_t)(A.gs / 128));
        L.family = CBK_KERNEL_BSTREAM;
        L.f = gemv_bstream_kernel_for(mode, A.bits[0], mixed, bp.bsu, dtype);
        L.grid = bp.grid;
        L.block = 64 * bp.ks * bp.rw;
        L.lds = bp.lds;
        L.P = bp.P;
        return L;
    }
    // everything else: the fp32 matrix-core kernel
    const AnyPlan pl = plan_any(A.M, A.V, A.K, split_k);
    A.P = pl.P;
    A.ntiles = pl.ntiles;
    A.mtiles = pl.mtiles;
    A.jobs = (int)std::min<int64_t>(pl.jobs, INT32_MAX);
    A.divP = make_fastdiv((uint32_t)A.P);
    A.divT = make_fastdiv((uint32_t)std::max(A.ntiles, 1));
    A.divGS = make_fastdiv((uint32_t)(A.gs / 32));
    A.st_xvec = (A.K % 8 == 0) && (reinterpret_cast<uintptr_t>(A.x) % 16 == 0);
    L.family = CBK_KERNEL_GENERIC;
    L.f = gemv_any_kernel_for(dtype, mode);
    L.grid = A.jobs;
    L.block = 64 * pl.waves;
    L.lds = 0;
    L.P = pl.P;
    return L;
}

// Whether the launch's K splits can combine inside the dispatch (the streaming kernels
// and the fp32 matrix-core kernel, with a counter per row block in one window) rather
// than in a combine launch.
bool combines_in_dispatch(const DecodeLaunch& L) {
    return L.P > 1 &&
           (L.family == CBK_KERNEL_STREAM || L.family == CBK_KERNEL_BSTREAM || L.family == CBK_KERNEL_GENERIC) &&
           L.grid / L.P <= SPLIT_COUNTERS;
}

// Common body of the three decode entry points.
int run_decode(GemvArgs& A, int dtype, int mode, bool mixed, int split_k, int rho, float* partial, int device,
               void* stream) {
    DeviceGuard guard(device);
    if (guard.err != hipSuccess) return hip_fail(guard.err, "set device");
    const int cus = cu_count(device);
    if (cus <= 0) return fail(CBK_EHIP, "cannot query the compute-unit count of device %d", device);
    const DecodeLaunch L = plan_decode(A, dtype, mode, mixed, split_k, rho, cus);
    if (L.family == CBK_KERNEL_GENERIC && (int64_t)A.ntiles * A.mtiles * A.P >= (1ll << 31))
        return fail(CBK_EINVAL, "packed_gemv: problem too large for 32-bit job indexing");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    A.split_cnt = nullptr;
    if (A.P > 1) {
        if (!partial) return fail(CBK_EINVAL, "split-K needs a partial buffer (cbk_gemv_partial_floats)");
        A.partial = partial;
        if (combines_in_dispatch(L)) A.split_cnt = split_window(device, s);
    } else {
        A.partial = nullptr;
    }
    hipError_t e = ensure_lds(L.f, L.lds);
    if (e != hipSuccess) return hip_fail(e, "packed_gemv: LDS attribute");
    void* args[] = {&A};
    e = launch(L.f, dim3(L.grid), dim3(L.block), args, (size_t)L.lds, s);
    if (e != hipSuccess) return hip_fail(e, "packed_gemv: launch");
    if (A.P > 1 && !A.split_cnt) {
        e = launch_gemv_combine(A, dtype, mode, s);
        if (e != hipSuccess) return hip_fail(e, "packed_gemv: combine launch");
    }
    return CBK_OK;
}

// Projection i of a decode call: its weight side and its output side.
void set_proj(GemvArgs& A, int i, const int32_t* w, const void* s, const void* z, const void* b, void* out,
              int64_t n, int bits, int64_t K) {
    Src& S = A.src[i];
    S.w = reinterpret_cast<const uint32_t*>(w);
    S.s = s;
    S.z = z;
    S.n = (int)n;
    S.wpr = (int)(ceil_div(K, 32) * bits);
    A.bits[i] = bits;
    Dst& D = A.dst[i];
    D.y = out;
    D.bias = b;
    D.ld = (int)n;
    D.pad_ = 0;
}

// Projections 1 and 2 of a single-projection call repeat projection 0.
void repeat_proj0(GemvArgs& A) {
    A.src[1] = A.src[2] = A.src[0];
    A.dst[1] = A.dst[2] = A.dst[0];
    A.bits[1] = A.bits[2] = A.bits[0];
}

GemvArgs base_args(const void* x, int64_t M, int64_t K, int gs) {
    GemvArgs A;
    std::memset(&A, 0, sizeof(A));
    A.x = x;
    A.M = (int)M;
    A.K = (int)K;
    A.C = (int)ceil_div(K, 32);
    A.G = (int)ceil_div(K, gs);
    A.gs = gs;
    A.divHD = make_fastdiv(1);
    return A;
}

int qkv_common(const void* x, int dtype, int64_t M, int64_t K, const int32_t* wq, const void* sq, const void* zq,
               const void* bq, int64_t nq, const int32_t* wk, const void* sk, const void* zk, const void* bk,
               int64_t nk, const int32_t* wv, const void* sv, const void* zv, const void* bv, int64_t nv,
               const float* rope_cos, const float* rope_sin, int head_dim, int perm_hd, int bits_q, int bits_k,
               int bits_v, int group_size, int split_k, int rho, float* partial, void* out_q, void* out_k,
               void* out_v, int device, void* stream) {
    int rc = check_x(x, dtype, M, K);
    if (rc) return rc;
    if ((rc = check_weight(wq, sq, zq, nq, bits_q, group_size, "fused_qkv(q)"))) return rc;
    if ((rc = check_weight(wk, sk, zk, nk, bits_k, group_size, "fused_qkv(k)"))) return rc;
    if ((rc = check_weight(wv, sv, zv, nv, bits_v, group_size, "fused_qkv(v)"))) return rc;
    if (split_k < 1) return fail(CBK_EINVAL, "split_k must be >= 1");
    if (!out_q || !out_k || !out_v) return fail(CBK_EINVAL, "fused_qkv: outputs must be non-null");
    if (perm_hd < 0 || head_dim < 0) return fail(CBK_EINVAL, "head_dim must be >= 0");
    if (perm_hd > 0) {
        if (perm_hd % 2) return fail(CBK_EINVAL, "perm head_dim must be even");
        if (nq % perm_hd || nk % perm_hd) return fail(CBK_EINVAL, "Q/K widths must be multiples of head_dim");
    }
    const bool rope = rope_cos != nullptr;
    if (rope) {
        if (!rope_sin) return fail(CBK_EINVAL, "cos/sin shape mismatch");
        if (!(perm_hd > 0 && perm_hd == head_dim))
            return fail(CBK_EINVAL,
                        "fused RoPE needs Q/K weights stored pair-interleaved with the same head_dim "
                        "(ops.permute_for_rope / install_bitmap(fuse_rope=True))");
    }
    if (M == 0) return CBK_OK;
    GemvArgs A = base_args(x, M, K, group_size);
    set_proj(A, 0, wq, sq, zq, bq, out_q, nq, bits_q, K);
    set_proj(A, 1, wk, sk, zk, bk, out_k, nk, bits_k, K);
    set_proj(A, 2, wv, sv, zv, bv, out_v, nv, bits_v, K);
    A.V = (int)(nq + nk + nv);
    A.perm_hd = perm_hd;
    A.divHD = make_fastdiv((uint32_t)(perm_hd > 0 ? perm_hd : 1));
    if (rope) {
        A.rope_cos = rope_cos;
        A.rope_sin = rope_sin;
        A.head_dim = head_dim;
    }
    const bool mixed = !(bits_q == bits_k && bits_k == bits_v);
    return run_decode(A, dtype, CBK_MODE_QKV, mixed, split_k, rho, partial, device, stream);
}

}  // namespace

namespace cbk {
hipError_t lds_limit_raise(const void* f, int bytes) { return ensure_lds(f, bytes); }
}  // namespace cbk

extern "C" {

const char* cbk_last_error(void) { return g_err.c_str(); }

int cbk_abi_version(void) { return 1; }

int cbk_sm_count(int device, int* out) {
    if (!out) return fail(CBK_EINVAL, "out must be non-null");
    const int c = cu_count(device);
    if (c <= 0) return fail(CBK_EHIP, "cannot query the compute-unit count of device %d", device);
    *out = c;
    return CBK_OK;
}

int cbk_tile_n(void) { return MFMA_TILE; }

int cbk_max_rho(int device, int bits, int mode, int* out) {
    if (!out) return fail(CBK_EINVAL, "out must be non-null");
    if (bits != 2 && bits != 3 && bits != 4) return fail(CBK_EINVAL, "bits must be 2/3/4");
    if (mode < 0 || mode > 2) return fail(CBK_EINVAL, "kind must be 'gemv', 'qkv' or 'gate_up'");
    DeviceGuard guard(device);
    if (guard.err != hipSuccess) return hip_fail(guard.err, "set device");
    const int cus = cu_count(device);
    if (cus <= 0) return fail(CBK_EHIP, "cannot query the compute-unit count of device %d", device);
    // the kernel, workgroup size and LDS of an fp16 batch-1 call at the Llama-2-7B widths of
    // this kind (K = 4096; N = 4096, 3 x 4096 or 2 x 11008), unsplit
    const uintptr_t base = (uintptr_t)1 << 20;
    const void* a = reinterpret_cast<const void*>(base);
    const int64_t n = mode == CBK_MODE_GATEUP ? 11008 : 4096;
    GemvArgs A = base_args(a, 1, 4096, 128);
    for (int i = 0; i < 3; ++i)
        set_proj(A, i, reinterpret_cast<const int32_t*>(base), a, a, nullptr, nullptr, n, bits, 4096);
    A.V = (int)(mode == CBK_MODE_QKV ? 3 * n : (mode == CBK_MODE_GATEUP ? 2 * n : n));
    const DecodeLaunch L = plan_decode(A, CBK_F16, mode, false, 1, 1, cus);
    const void* f = L.f;
    int blocks = 0;
    hipError_t e = ensure_lds(f, L.lds);
    if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, f, L.block, (size_t)L.lds);
    if (e != hipSuccess) return hip_fail(e, "max_rho: occupancy query");
    *out = std::max(blocks, 1);
    return CBK_OK;
}

int64_t cbk_gemv_partial_floats(int dtype, int64_t M, int64_t V, int64_t K, int group_size, int split_k) {
    if (M <= 0 || V <= 0 || K <= 0 || group_size <= 0 || split_k < 1) return 0;
    int P = plan_any(M, V, K, split_k).P;
    if (M <= 2) P = std::max(P, stream_splits(ceil_div(K, 32), split_k, stream_max_slices((int)M, dtype)));
    const int xr = dtype == CBK_F32 ? 2 : 1;
    if (M >= (dtype == CBK_F32 ? 2 : 3) && M * xr <= 16) {  // 4-unit slices split at least as often as 8-unit ones; gate-up rows
        const int64_t C = ceil_div(K, 32);
        const bool bf = dtype != CBK_F16;
        P = std::max(P, bstream_splits(C, M, split_k, bstream_rw(M, 4, true), 4, bf, xr));
        for (bool gateup : {false, true})     // bstream_fill takes at most P0 + 3 splits
            if (bstream_fills(bstream_base(M, C, split_k, gateup, bf, xr), V))
                P = std::max<int64_t>(P, std::min<int64_t>(ceil_div(C, 4), split_k + BSTREAM_FILL_SPLITS - 1));
    }
    return P > 1 ? (int64_t)P * M * V : 0;
}

int cbk_packed_gemv(const void* x, int dtype, int64_t M, int64_t K, const int32_t* packed, const void* scales,
                    const void* zeros, const void* bias, int64_t N, int bits, int group_size, int split_k, int rho,
                    int act, int32_t* workspace, float* partial, void* out, int device, void* stream) {
    (void)workspace;
    int rc = check_x(x, dtype, M, K);
    if (rc) return rc;
    if ((rc = check_weight(packed, scales, zeros, N, bits, group_size, "packed_gemv"))) return rc;
    if (split_k < 1) return fail(CBK_EINVAL, "split_k must be >= 1");
    if (act < 0 || act > 2) return fail(CBK_EINVAL, "act must be 0 (none), 1 (relu) or 2 (silu)");
    if (!out) return fail(CBK_EINVAL, "packed_gemv: out must be non-null");
    if (M == 0) return CBK_OK;
    GemvArgs A = base_args(x, M, K, group_size);
    set_proj(A, 0, packed, scales, zeros, bias, out, N, bits, K);
    repeat_proj0(A);
    A.V = (int)N;
    A.act = act;
    return run_decode(A, dtype, CBK_MODE_GEMV, false, split_k, rho, partial, device, stream);
}

int cbk_decode_plan(int dtype, int64_t M, int64_t K, int group_size, int64_t n0, int64_t n1, int64_t n2, int bits0,
                    int bits1, int bits2, int mode, int split_k, int rho, int device, int32_t* out) {
    if (!out) return fail(CBK_EINVAL, "decode_plan: out must be non-null");
    if (!valid_dtype(dtype)) return fail(CBK_EINVAL, "x must be fp16/bf16/fp32");
    if (M < 1 || K <= 0 || K > (1 << 24) || M > (1 << 24)) return fail(CBK_EINVAL, "decode_plan: bad shape");
    if (mode < 0 || mode > 2) return fail(CBK_EINVAL, "decode_plan: mode must be 0 (gemv), 1 (qkv) or 2 (gate_up)");
    if (group_size <= 0 || group_size % 32 != 0)
        return fail(CBK_EINVAL, "group_size must be a positive multiple of 32");
    if (split_k < 1) return fail(CBK_EINVAL, "split_k must be >= 1");
    const int64_t ns[3] = {n0, mode == CBK_MODE_QKV ? n1 : n0, mode == CBK_MODE_QKV ? n2 : n0};
    const int bs[3] = {bits0, mode == CBK_MODE_QKV ? bits1 : bits0, mode == CBK_MODE_QKV ? bits2 : bits0};
    for (int i = 0; i < 3; ++i) {
        if (ns[i] <= 0 || ns[i] > (1 << 29)) return fail(CBK_EINVAL, "decode_plan: bad out_features");
        if (bs[i] != 2 && bs[i] != 3 && bs[i] != 4) return fail(CBK_EINVAL, "bits must be 2/3/4");
    }
    const int cus = cu_count(device);
    if (cus <= 0) return fail(CBK_EHIP, "cannot query the compute-unit count of device %d", device);
    // the plan of tensors as torch allocates them: every base 256-byte aligned
    const uintptr_t base = (uintptr_t)1 << 20;
    const void* a = reinterpret_cast<const void*>(base);
    GemvArgs A = base_args(a, M, K, group_size);
    for (int i = 0; i < 3; ++i)
        set_proj(A, i, reinterpret_cast<const int32_t*>(base), a, a, nullptr, nullptr, ns[i], bs[i], K);
    A.V = (int)(mode == CBK_MODE_QKV ? ns[0] + ns[1] + ns[2] : (mode == CBK_MODE_GATEUP ? 2 * ns[0] : ns[0]));
    const bool mixed = mode == CBK_MODE_QKV && !(bs[0] == bs[1] && bs[1] == bs[2]);
    const DecodeLaunch L = plan_decode(A, dtype, mode, mixed, split_k, rho, cus);
    out[0] = L.family;
    out[1] = L.P;
    out[2] = L.grid;
    out[3] = L.block;
    out[4] = L.lds;
    out[5] = L.P > 1 && !combines_in_dispatch(L) ? 2 : 1;   // launches per call (a reduce launch combines)
    return CBK_OK;
}

int cbk_packed_gemv_noalloc(const void* x, int dtype, int64_t M, int64_t K, const int32_t* packed,
                            const void* scales, const void* zeros, const void* bias, int64_t N, int bits,
                            int group_size, int split_k, int rho, int act, void* out, int device, void* stream) {
    int rc = check_x(x, dtype, M, K);
    if (rc) return rc;
    if ((rc = check_weight(packed, scales, zeros, N, bits, group_size, "packed_gemv_noalloc"))) return rc;
    if (split_k < 1) return fail(CBK_EINVAL, "split_k must be >= 1");
    if (act < 0 || act > 2) return fail(CBK_EINVAL, "act must be 0 (none), 1 (relu) or 2 (silu)");
    if (!out) return fail(CBK_EINVAL, "packed_gemv_noalloc: out must be non-null");
    const int64_t need = cbk_gemv_partial_floats(dtype, M, N, K, group_size, split_k);
    if (need > NOALLOC_PARTIAL_FLOATS)
        return fail(CBK_EINVAL,
                    "packed_gemv_noalloc: split-K partial sums need %lld floats, above the %lld-float device "
                    "scratch (use cbk_packed_gemv with a caller buffer, or a smaller split_k or batch)",
                    (long long)need, (long long)NOALLOC_PARTIAL_FLOATS);
    if (M == 0) return CBK_OK;
    DeviceGuard guard(device);
    if (guard.err != hipSuccess) return hip_fail(guard.err, "set device");
    float* part = nullptr;
    const hipError_t e = scratch_for(device, &part);
    if (e != hipSuccess) return hip_fail(e, "packed_gemv_noalloc: scratch address");
    GemvArgs A = base_args(x, M, K, group_size);
    set_proj(A, 0, packed, scales, zeros, bias, out, N, bits, K);
    repeat_proj0(A);
    A.V = (int)N;
    A.act = act;
    return run_decode(A, dtype, CBK_MODE_GEMV, false, split_k, rho, need > 0 ? part : nullptr, device, stream);
}

int cbk_fused_gate_up(const void* x, int dtype, int64_t M, int64_t K, const int32_t* wg, const void* sg,
                      const void* zg, const int32_t* wu, const void* su, const void* zu, int64_t N, int bits,
                      int group_size, int split_k, int rho, int32_t* workspace, float* partial, void* out,
                      int device, void* stream) {
    (void)workspace;
    int rc = check_x(x, dtype, M, K);
    if (rc) return rc;
    if ((rc = check_weight(wg, sg, zg, N, bits, group_size, "fused_gate_up(gate)"))) return rc;
    if ((rc = check_weight(wu, su, zu, N, bits, group_size, "fused_gate_up(up)"))) return rc;
    if (split_k < 1) return fail(CBK_EINVAL, "split_k must be >= 1");
    if (!out) return fail(CBK_EINVAL, "fused_gate_up: out must be non-null");
    if (2 * N > (1 << 30)) return fail(CBK_EINVAL, "fused_gate_up: out_features too large");
    if (M == 0) return CBK_OK;
    GemvArgs A = base_args(x, M, K, group_size);
    set_proj(A, 0, wg, sg, zg, nullptr, out, N, bits, K);
    set_proj(A, 1, wu, su, zu, nullptr, out, N, bits, K);
    A.src[2] = A.src[0];
    A.dst[2] = A.dst[0];
    A.bits[2] = A.bits[0];
    A.V = (int)(2 * N);
    return run_decode(A, dtype, CBK_MODE_GATEUP, false, split_k, rho, partial, device, stream);
}

int cbk_fused_qkv(const void* x, int dtype, int64_t M, int64_t K, const int32_t* wq, const void* sq, const void* zq,
                  const void* bq, int64_t nq, const int32_t* wk, const void* sk, const void* zk, const void* bk,
                  int64_t nk, const int32_t* wv, const void* sv, const void* zv, const void* bv, int64_t nv,
                  const float* rope_cos, const float* rope_sin, int head_dim, int perm_hd, int bits, int group_size,
                  int split_k, int rho, int32_t* workspace, float* partial, void* out_q, void* out_k, void* out_v,
                  int device, void* stream) {
    (void)workspace;
    return qkv_common(x, dtype, M, K, wq, sq, zq, bq, nq, wk, sk, zk, bk, nk, wv, sv, zv, bv, nv, rope_cos, rope_sin,
                      head_dim, perm_hd, bits, bits, bits, group_size, split_k, rho, partial, out_q, out_k, out_v,
                      device, stream);
}

int cbk_fused_qkv_mixed(const void* x, int dtype, int64_t M, int64_t K, const int32_t* wq, const void* sq,
                        const void* zq, const void* bq, int64_t nq, const int32_t* wk, const void* sk, const void* zk,
                        const void* bk, int64_t nk, const int32_t* wv, const void* sv, const void* zv, const void* bv,
                        int64_t nv, const float* rope_cos, const float* rope_sin, int head_dim, int perm_hd,
                        int bits_q, int bits_k, int bits_v, int group_size, int split_k, int rho, int32_t* workspace,
                        float* partial, void* out_q, void* out_k, void* out_v, int device, void* stream) {
    (void)workspace;
    return qkv_common(x, dtype, M, K, wq, sq, zq, bq, nq, wk, sk, zk, bk, nk, wv, sv, zv, bv, nv, rope_cos, rope_sin,
                      head_dim, perm_hd, bits_q, bits_k, bits_v, group_size, split_k, rho, partial, out_q, out_k,
                      out_v, device, stream);
}

int cbk_packed_gemm(const void* x, int dtype, int64_t M, int64_t K, const int32_t* packed, const void* scales,
                    const void* zeros, const void* bias, int64_t N, int bits, int group_size, int act,
                    int use_matrix_cores, void* out, int device, void* stream) {
    int rc = check_x(x, dtype, M, K);
    if (rc) return rc;
    if ((rc = check_weight(packed, scales, zeros, N, bits, group_size, "packed_gemm"))) return rc;
    if (act < 0 || act > 2) return fail(CBK_EINVAL, "act must be 0 (none), 1 (relu) or 2 (silu)");
    if (!out) return fail(CBK_EINVAL, "packed_gemm: out must be non-null");
    if (M == 0) return CBK_OK;
    DeviceGuard guard(device);
    if (guard.err != hipSuccess) return hip_fail(guard.err, "set device");
    GemmArgs A{};
    A.x = x;
    A.w = reinterpret_cast<const uint32_t*>(packed);
    A.s = scales;
    A.z = zeros;
    A.b = bias;
    A.out = out;
    A.M = (int)M;
    A.N = (int)N;
    A.K = (int)K;
    A.C = (int)ceil_div(K, 32);
    A.G = (int)ceil_div(K, group_size);
    A.gs = group_size;
    A.wpr = (int)(A.C * bits);
    A.bits = bits;
    A.act = act;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    A.divG = make_fastdiv((uint32_t)group_size);
    A.xvec = (K % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0);
    const bool mc = use_matrix_cores && (dtype == CBK_F16 || dtype == CBK_BF16);
    hipError_t e;
    if (mc && gemm_f16_supported(A)) e = launch_gemm_f16(A, dtype, s);
    else e = mc ? launch_gemm_mfma(A, dtype, s) : launch_gemm_f32(A, dtype, s);
    if (e != hipSuccess) return hip_fail(e, "packed_gemm: launch");
    return CBK_OK;
}

int cbk_packed_gemm_gate_up(const void* x, int dtype, int64_t M, int64_t K, const int32_t* packed_gate,
                            const void* scales_gate, const void* zeros_gate, const int32_t* packed_up,
                            const void* scales_up, const void* zeros_up, int64_t N, int bits, int group_size,
                            void* out, int device, void* stream) {
    int rc = check_x(x, dtype, M, K);
    if (rc) return rc;
    if ((rc = check_weight(packed_gate, scales_gate, zeros_gate, N, bits, group_size, "packed_gemm_gate_up(gate)")))
        return rc;
    if ((rc = check_weight(packed_up, scales_up, zeros_up, N, bits, group_size, "packed_gemm_gate_up(up)")))
        return rc;
    if (!out) return fail(CBK_EINVAL, "packed_gemm_gate_up: out must be non-null");
    if (dtype != CBK_F16 && dtype != CBK_BF16)
        return fail(CBK_ENOTSUP, "packed_gemm_gate_up: x must be fp16 or bf16 (the 16-bit matrix cores)");
    GemmArgs A{};
    A.x = x;
    A.w = reinterpret_cast<const uint32_t*>(packed_gate);
    A.s = scales_gate;
    A.z = zeros_gate;
    A.w2 = reinterpret_cast<const uint32_t*>(packed_up);
    A.s2 = scales_up;
    A.z2 = zeros_up;
    A.out = out;
    A.M = (int)M;
    A.N = (int)N;
    A.K = (int)K;
    A.C = (int)ceil_div(K, 32);
    A.G = (int)ceil_div(K, group_size);
    A.gs = group_size;
    A.wpr = (int)(A.C * bits);
    A.bits = bits;
    A.act = ACT_SILU;
    A.divG = make_fastdiv((uint32_t)group_size);
    A.xvec = (K % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0);
    if (!gemm_f16_supported(A))
        return fail(CBK_ENOTSUP, "packed_gemm_gate_up: needs K %% 8 == 0 and 16-byte aligned x, packed, scales "
                                 "and zeros");
    if (M == 0) return CBK_OK;
    DeviceGuard guard(device);
    if (guard.err != hipSuccess) return hip_fail(guard.err, "set device");
    const hipError_t e = launch_gemm_f16(A, dtype, reinterpret_cast<hipStream_t>(stream), true);
    if (e != hipSuccess) return hip_fail(e, "packed_gemm_gate_up: launch");
    return CBK_OK;
}

int cbk_quantize_pack(const void* w, int dtype, int64_t N, int64_t K, int bits, int group_size, int scheme,
                      int32_t* packed, void* scales, void* zeros, int meta_dtype, int device, void* stream) {
    if (!valid_dtype(dtype)) return fail(CBK_EINVAL, "quantize_pack: weights must be fp16/bf16/fp32");
    if (!valid_dtype(meta_dtype)) return fail(CBK_EINVAL, "quantize_pack: scales/zeros must be fp16/bf16/fp32");
    if (bits != 2 && bits != 3 && bits != 4) return fail(CBK_EINVAL, "quantize_pack: bits must be 2/3/4");
    if (group_size <= 0 || group_size % 32 != 0)
        return fail(CBK_EINVAL, "quantize_pack: group_size must be a positive multiple of 32");
    if (scheme != 0 && scheme != 1) return fail(CBK_EINVAL, "quantize_pack: scheme must be 0 (kernel) or 1 (affine)");
    if (N < 0 || K <= 0 || N > (1 << 30) || K > (1 << 24)) return fail(CBK_EINVAL, "quantize_pack: bad shape");
    if (N == 0) return CBK_OK;
    if (!w || !packed || !scales || !zeros) return fail(CBK_EINVAL, "quantize_pack: pointers must be non-null");
    if ((int64_t)N * ceil_div(K, group_size) >= (1ll << 31)) return fail(CBK_EINVAL, "quantize_pack: too many groups");
    DeviceGuard guard(device);
    if (guard.err != hipSuccess) return hip_fail(guard.err, "set device");
    QuantArgs A;
    A.w = w;
    A.packed = reinterpret_cast<uint32_t*>(packed);
    A.scales = scales;
    A.zeros = zeros;
    A.N = (int)N;
    A.K = (int)K;
    A.G = (int)ceil_div(K, group_size);
    A.gs = group_size;
    A.bits = bits;
    A.wpr = (int)(ceil_div(K, 32) * bits);
    A.scheme = scheme;
    const hipError_t e = launch_quant_pack(A, dtype, meta_dtype, cu_count(device), reinterpret_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "quantize_pack: launch");
    return CBK_OK;
}

int cbk_unpack_codes(const int32_t* packed, int64_t N, int64_t K, int bits, int32_t* codes, int device,
                     void* stream) {
    if (!packed || !codes) return fail(CBK_EINVAL, "unpack_codes: pointers must be non-null");
    if (bits != 2 && bits != 3 && bits != 4) return fail(CBK_EINVAL, "unpack_codes: bits must be 2/3/4");
    if (N < 0 || K <= 0 || N > (1 << 30) || K > (1 << 24)) return fail(CBK_EINVAL, "unpack_codes: bad shape");
    if (N == 0) return CBK_OK;
    DeviceGuard guard(device);
    if (guard.err != hipSuccess) return hip_fail(guard.err, "set device");
    const hipError_t e = launch_unpack(reinterpret_cast<const uint32_t*>(packed), (int)N, (int)K, bits, codes,
                                       reinterpret_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "unpack_codes: launch");
    return CBK_OK;
}

int cbk_stream_probe(const void* src, int64_t bytes, int unroll, int block, int store, uint32_t* sink,
                     int device, void* stream) {
    if (!src || !sink) return fail(CBK_EINVAL, "stream_probe: pointers must be non-null");
    if (bytes <= 0 || bytes > (1ll << 30)) return fail(CBK_EINVAL, "stream_probe: bytes must be in [1, 2^30]");
    if (unroll != 1 && unroll != 2 && unroll != 4 && unroll != 8 && unroll != 16)
        return fail(CBK_EINVAL, "stream_probe: unroll must be 1, 2, 4, 8 or 16");
    if (block < 64 || block > 1024 || block % 64 != 0)
        return fail(CBK_EINVAL, "stream_probe: block must be a multiple of 64 in [64, 1024]");
    if (store != 0 && store != 1) return fail(CBK_EINVAL, "stream_probe: store must be 0 or 1");
    DeviceGuard guard(device);
    if (guard.err != hipSuccess) return hip_fail(guard.err, "set device");
    const hipError_t e = launch_stream_probe(src, (uint32_t)bytes, unroll, block, store != 0, sink,
                                             reinterpret_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "stream_probe: launch");
    return CBK_OK;
}

int cbk_timer_start(int capacity) {
    if (capacity <= 0 || capacity > (1 << 20)) return fail(CBK_EINVAL, "timer capacity must be in [1, 2^20]");
    std::lock_guard<std::mutex> lk(g_timer.mu);
    if (g_timer.armed) return fail(CBK_EINVAL, "timer already armed");
    while ((int)g_timer.ev.size() < 2 * capacity) {
        hipEvent_t e;
        const hipError_t err = hipEventCreate(&e);
        if (err != hipSuccess) return hip_fail(err, "timer: event create");
        g_timer.ev.push_back(e);
    }
    g_timer.used = 0;
    g_timer.armed = true;
    return CBK_OK;
}

int cbk_timer_stop(double* total_ms, int* launches, double* durations_ms, int max_durations) {
    std::lock_guard<std::mutex> lk(g_timer.mu);
    if (!g_timer.armed) return fail(CBK_EINVAL, "timer not armed");
    g_timer.armed = false;
    double total = 0.0;
    for (int i = 0; i < g_timer.used; ++i) {
        hipError_t err = hipEventSynchronize(g_timer.ev[2 * i + 1]);
        if (err != hipSuccess) return hip_fail(err, "timer: synchronize");
        float ms = 0.f;
        err = hipEventElapsedTime(&ms, g_timer.ev[2 * i], g_timer.ev[2 * i + 1]);
        if (err != hipSuccess) return hip_fail(err, "timer: elapsed");
        total += ms;
        if (durations_ms && i < max_durations) durations_ms[i] = ms;
    }
    if (total_ms) *total_ms = total;
    if (launches) *launches = g_timer.used;
    return CBK_OK;
}

}  // extern "C"
