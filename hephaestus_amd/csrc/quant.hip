// quant.hip - dynamic E4M3 activation quantization (gfx950).
//
// Restates the reference quantizer (src/hephaestus/kernels.mojo:136-193 and
// :214-267): per group, scale = amax/448 (1.0 below 1e-12), codes =
// e4m3(x * (1/scale)). The reference reduces one whole row with a 256-thread
// LDS tree; here a 1x128 group is 16 lanes x 8 bf16 reduced with cross-lane
// max, so one wave quantizes four groups with one 16-byte load per lane and
// no LDS or barrier. The amax is taken on the bf16 magnitude bits (NaN
// skipped, as the reference's `v > local` test does). The per-token form (group = K) keeps one workgroup per
// row.
#include "heph_kernels.h"

namespace heph {

// One 16-lane team per 128-wide group; groups are contiguous in memory
// because K % 128 == 0, so the flat group index g covers x[g*128, g*128+128)
// and its scale lands at scales[g] ([M, K/128] row-major).
__global__ __launch_bounds__(256) void quant_g128_kernel(
    const uint16_t* __restrict__ x, uint8_t* __restrict__ q,
    float* __restrict__ scales, long n_groups)
{
    const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long g = t >> 4;
    const int  j = threadIdx.x & 15;
    const bool live = g < n_groups;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (live) v = ldg16u(x + g * kChunk + j * 8);
    uint32_t mb = absmax_bits8(v);
    for (int o = 1; o < 16; o <<= 1) mb = max(mb, shfl_xor_u(mb, o));
    if (__builtin_amdgcn_ballot_w64(mb > 0x7F80u) != 0) {    // a group holds NaN
        mb = absmax_bits8_skip_nan(v);
        for (int o = 1; o < 16; o <<= 1) mb = max(mb, shfl_xor_u(mb, o));
    }
    float s, inv;
    group_scale(bf16_bits_f32(mb), s, inv);
    if (live) {
        *reinterpret_cast<uint2*>(q + g * kChunk + j * 8) = quant8(v, inv);
        if (j == 0) scales[g] = s;
    }
}

// Per-token (group = K): one 256-thread workgroup per row.
__global__ __launch_bounds__(256) void quant_row_kernel(
    const uint16_t* __restrict__ x, uint8_t* __restrict__ q,
    float* __restrict__ scales, int K)
{
    __shared__ uint32_t red[4];
    const int row = blockIdx.x;
    const uint16_t* xr = x + (size_t)row * K;
    uint8_t* qr = q + (size_t)row * K;
    uint32_t m = 0;
    for (int k = threadIdx.x * 8; k < K; k += 256 * 8) m = absmax_bits8_skip_nan(ldg16u(xr + k), m);
    for (int o = 32; o >= 1; o >>= 1) m = max(m, shfl_xor_u(m, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = max(max(red[0], red[1]), max(red[2], red[3]));
    float s, inv;
    group_scale(bf16_bits_f32(m), s, inv);
    if (threadIdx.x == 0) scales[row] = s;
    for (int k = threadIdx.x * 8; k < K; k += 256 * 8)
        *reinterpret_cast<uint2*>(qr + k) = quant8(ldg16u(xr + k), inv);
}

hipError_t launch_quant(const uint16_t* x, uint8_t* q, float* scales, int M,
                        int K, int group_k, hipStream_t stream, const LaunchTiming& t)
{
    if (group_k == kChunk) {
        const long n_groups = (long)M * (K / kChunk);
        const long threads = n_groups * 16;
        const unsigned blocks = (unsigned)((threads + 255) / 256);
        return launch(quant_g128_kernel, dim3(blocks), dim3(256), 0, stream, t, x, q, scales,
                      n_groups);
    }
    return launch(quant_row_kernel, dim3(M), dim3(256), 0, stream, t, x, q, scales, K);
}

}  // namespace heph
