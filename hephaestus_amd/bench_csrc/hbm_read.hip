// hbm_read.hip - measurement kernels for bench.py (libhephbench.so), not
// part of the FP8 linear library: a plain streaming read of a device
// buffer, the denominator for "fraction of the achievable read rate".
//
// Every thread loads four 16-byte pieces per trip, one workgroup-width
// apart (each load instruction of a wave covers 1 KB of consecutive
// bytes), and folds them into one XOR that is stored per workgroup so the
// loads cannot be removed. Launched with `blocks` workgroups of 256
// threads; the buffer must be a multiple of 16 bytes.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__global__ __launch_bounds__(256) void read_kernel(const uint4* __restrict__ p, size_t n16,
                                                   uint32_t* __restrict__ sink)
{
    const size_t tile = (size_t)blockDim.x * 4;
    const size_t stride = tile * gridDim.x;
    uint32_t acc = 0;
    for (size_t base = (size_t)blockIdx.x * tile; base < n16; base += stride) {
        uint4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const size_t i = base + (size_t)k * blockDim.x + threadIdx.x;
            v[k] = i < n16 ? p[i] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    // one word per workgroup (only its value depends on the loads)
    acc = __reduce_or_sync(0xffffffffffffffffull, acc);
    if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16) at p with `blocks` 256-thread
// workgroups on `stream`; sink holds at least `blocks` words. Returns 0 or
// the hipError_t of the launch.
int heph_bench_read(const void* p, size_t bytes, int blocks, void* sink, void* stream)
{
    if (!p || !sink || blocks < 1 || bytes % 16) return (int)hipErrorInvalidValue;
    read_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint4*>(p), bytes / 16, static_cast<uint32_t*>(sink));
    return (int)hipGetLastError();
}

}  // extern "C"
