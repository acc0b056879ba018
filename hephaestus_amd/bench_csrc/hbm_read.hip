// hbm_read.hip - measurement kernels for bench.py (libhephbench.so), not
// part of the FP8 linear library: a plain streaming read of a device
// buffer, the denominator for "fraction of the achievable read rate", and
// an FP8 MFMA loop with no memory traffic, the denominator for "fraction of
// the achievable MFMA rate" (the shader clock settles lower under sustained
// MFMA load than the clock the published peak assumes).
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

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Every wave: `iters` rounds of 8 independent v_mfma_f32_16x16x128_f8f6f4
// (8 accumulator chains), then one store per thread so the work stays live.
// The operands are four sets of pseudo-random E4M3 codes (bytes & 0x77: no
// NaN, magnitudes up to 240) that successive MFMAs cycle through, so the
// multipliers switch as they do on real data (the power draw, and with it
// the clock the chip sustains, depends on that). 65536 flops per MFMA.
__device__ __forceinline__ uint32_t mix32(uint32_t x)
{
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return x;
}

__global__ __launch_bounds__(256) void mfma_loop_kernel(int iters, float* __restrict__ sink)
{
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    i32x8 a[4], b[4];
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            a[v][k] = (int)(mix32(t * 64u + v * 16u + k) & 0x77777777u);
            b[v][k] = (int)(mix32(t * 64u + v * 16u + 8u + k) & 0x77777777u);
        }
    f32x4 acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = f32x4{0, 0, 0, 0};
    for (int i = 0; i < iters; i += 4) {       // iters % 4 == 0
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int c = 0; c < 8; ++c)
                acc[c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                    a[c & 3], b[(c + u) & 3], acc[c], 0, 0, 0, 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) s += (acc[c][0] + acc[c][1]) + (acc[c][2] + acc[c][3]);
    sink[t] = s;
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

// `blocks` workgroups of 256 threads of mfma_loop_kernel, `iters` rounds
// (a multiple of 4) each (blocks * 4 waves * iters * 8 MFMAs * 65536 flops); sink holds
// blocks * 256 floats. Returns 0 or the hipError_t of the launch.
int heph_bench_mfma(int blocks, int iters, void* sink, void* stream)
{
    if (!sink || blocks < 1 || iters < 4 || iters % 4) return (int)hipErrorInvalidValue;
    mfma_loop_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
        iters, static_cast<float*>(sink));
    return (int)hipGetLastError();
}

}  // extern "C"
