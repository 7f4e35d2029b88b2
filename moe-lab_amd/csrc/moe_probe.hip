// Read-bandwidth probe of the timing harness's contention guard: a plain stream of 16-byte loads over a buffer, the
// access pattern of the expert kernels' weight streams, with nothing else in the loop. Each workgroup folds the words
// it reads with XOR into one sink word (so no load can be dropped; the XOR of the sink is the XOR of the buffer).
#include "moe_common.h"
#include "moe_internal.h"

namespace moe {

constexpr int PROBE_THREADS = 256;
constexpr int PROBE_UNROLL = 4;   // 16-byte loads in flight per thread and iteration

// grid MOE_PROBE_SINK workgroups; workgroup b reads the 16-byte chunks b * 1024 + j (+ k * grid * 1024), j < 1024: each
// iteration one contiguous 16 KB block per workgroup, the blocks of consecutive workgroups adjacent
__global__ void __launch_bounds__(PROBE_THREADS) k_probe_read(const uint4* __restrict__ src, size_t nchunks,
                                                              uint32_t* __restrict__ sink) {
    constexpr size_t BLOCK = (size_t)PROBE_THREADS * PROBE_UNROLL;
    uint32_t acc = 0;
    for (size_t base = (size_t)blockIdx.x * BLOCK; base < nchunks; base += (size_t)gridDim.x * BLOCK) {
        uint4 v[PROBE_UNROLL];
#pragma unroll
        for (int u = 0; u < PROBE_UNROLL; ++u) {
            const size_t c = base + (size_t)u * PROBE_THREADS + threadIdx.x;
            v[u] = c < nchunks ? src[c] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < PROBE_UNROLL; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    __shared__ uint32_t part[PROBE_THREADS / 64];
    for (int s = 32; s >= 1; s >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, s, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t r = 0;
        for (int w = 0; w < PROBE_THREADS / 64; ++w) r ^= part[w];
        sink[blockIdx.x] = r;
    }
}

int launch_probe_read(const void* src, size_t nbytes, uint32_t* sink, hipStream_t st) {
    k_probe_read<<<MOE_PROBE_SINK, PROBE_THREADS, 0, st>>>((const uint4*)src, nbytes / 16, sink);
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

}  // namespace moe
