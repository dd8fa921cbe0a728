// probe.hip -- a streaming kernel: the floor for moving a decode call's bytes in one launch.
//
// Not part of any op.  It reads `bytes` of device memory once, as 16-byte pieces: thread t
// of the grid issues its U loads (pieces t, t + T, ..., T threads in the grid, so a wave
// moves 1 KB contiguous per instruction) before it uses any of them and XORs them.  With
// STORE = false it keeps nothing (it stores only when the XOR hits a constant, which keeps
// the loads alive and practically never happens); with STORE = true each workgroup's
// first thread writes the workgroup's XOR (a wave reduction, an LDS exchange and one
// store, like a decode workgroup's results) to sink[workgroup % 1024].  The benchmark
// times it on the same byte counts as the decode GEMVs, over the same rotation of
// distinct buffers, to show how much of a GEMV's time one launch needs for its bytes
// alone on this GPU.
#include "cbk_kernels.hpp"

namespace cbk {
namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));
constexpr int RAW = 0x00020000;           // buffer descriptor word 3: raw 32-bit data
constexpr uint32_t SENTINEL = 0x9E3779B9u;

template <int U, bool STORE>
__global__ void __launch_bounds__(1024) stream_probe_kernel(const void* src, uint32_t bytes, uint32_t* sink) {
    __shared__ uint32_t part[16];
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(src), (short)0, (int)bytes, RAW);
    const uint32_t T = gridDim.x * blockDim.x;
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    u4 v[U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
        // pieces past `bytes` lie outside the descriptor's range and read as zero; the
        // host bounds the grid so these offsets stay below 2^32
        v[i] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(16u * (t + (uint32_t)i * T)), 0, 0);
    }
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < U; ++i) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if constexpr (STORE) {
        for (int o = 32; o > 0; o >>= 1) x ^= (uint32_t)__shfl_xor((int)x, o, 64);
        if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = x;
        __syncthreads();
        if (threadIdx.x == 0) {
            for (uint32_t w = 1; w < blockDim.x / 64; ++w) x ^= part[w];
            sink[blockIdx.x & 1023] = x;
        }
    } else {
        if (x == SENTINEL) sink[0] = x;
    }
}

template <int U>
const void* probe_kernel(bool store) {
    return store ? reinterpret_cast<const void*>(&stream_probe_kernel<U, true>)
                 : reinterpret_cast<const void*>(&stream_probe_kernel<U, false>);
}

}  // namespace

hipError_t launch_stream_probe(const void* src, uint32_t bytes, int unroll, int block, bool store, uint32_t* sink,
                               hipStream_t stream) {
    const uint32_t pieces = (bytes + 15u) / 16u;
    const uint32_t per_block = (uint32_t)block * (uint32_t)unroll;
    const dim3 grid((pieces + per_block - 1) / per_block);
    void* args[] = {const_cast<void**>(&src), &bytes, &sink};
    const void* f = unroll == 1 ? probe_kernel<1>(store)
                  : unroll == 2 ? probe_kernel<2>(store)
                  : unroll == 4 ? probe_kernel<4>(store)
                  : unroll == 8 ? probe_kernel<8>(store)
                                : probe_kernel<16>(store);
    return launch(f, grid, dim3(block), args, 0, stream);
}

}  // namespace cbk
