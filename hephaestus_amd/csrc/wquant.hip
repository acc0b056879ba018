// wquant.hip - bf16 weight [N,K] -> E4M3 codes + 128x128 block scales.
//
// Produces the weight / weight_scale_inv format from a bf16 checkpoint
// tensor on the GPU. The arithmetic follows the reference's offline weight
// quantizer (scripts/stage_tiny_fp8_from_bf16.py:59-71: s = amax/448, 1.0
// when amax is 0 or s < 1e-12, codes = e4m3(w / s) by division) applied per
// 128x128 block instead of per row. One 256-thread workgroup per block:
// each thread reads eight 16-byte pieces, the block amax is reduced with
// cross-lane max and LDS, and the codes are written 8 bytes at a time.
#include "heph_kernels.h"

namespace heph {

__global__ __launch_bounds__(256) void wquant_block_kernel(
    const uint16_t* __restrict__ w, uint8_t* __restrict__ q,
    float* __restrict__ scale_inv, int N, int K)
{
    __shared__ uint32_t red[4];
    const int KB = K / kChunk;
    const int bn = blockIdx.y, bk = blockIdx.x;
    const int tid = threadIdx.x;
    // 128 rows x 16 pieces of 8 elements; thread t takes pieces t + 256*r.
    const int col = (tid & 15) * 8;
    uint4 v[8];
    bool ok[8];
    uint32_t mb = 0;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const int row = bn * kChunk + (tid >> 4) + 16 * r;
        ok[r] = row < N;
        v[r] = ok[r] ? ldg16u(w + (size_t)row * K + bk * kChunk + col) : make_uint4(0, 0, 0, 0);
        mb = absmax_bits8(v[r], mb);
    }
    for (int o = 32; o >= 1; o >>= 1) mb = max(mb, shfl_xor_u(mb, o));
    if ((tid & 63) == 0) red[tid >> 6] = mb;
    __syncthreads();
    // numpy's max propagates NaN: a block holding NaN has a NaN amax, fails
    // `amax > 0` and takes s = 1 (as NaN bits sort above every other
    // magnitude, the integer max carries it through)
    const float m = bf16_bits_f32(max(max(red[0], red[1]), max(red[2], red[3])));
    float s = m > 0.0f ? __fdiv_rn(m, kE4M3Max) : 1.0f;
    if (s < 1e-12f) s = 1.0f;
    if (tid == 0) scale_inv[(size_t)bn * KB + bk] = s;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        if (!ok[r]) continue;
        const int row = bn * kChunk + (tid >> 4) + 16 * r;
        const uint4 x = v[r];
        uint2 c;
        c.x = pack4_e4m3(__fdiv_rn(bf16lo(x.x), s), __fdiv_rn(bf16hi(x.x), s),
                         __fdiv_rn(bf16lo(x.y), s), __fdiv_rn(bf16hi(x.y), s));
        c.y = pack4_e4m3(__fdiv_rn(bf16lo(x.z), s), __fdiv_rn(bf16hi(x.z), s),
                         __fdiv_rn(bf16lo(x.w), s), __fdiv_rn(bf16hi(x.w), s));
        *reinterpret_cast<uint2*>(q + (size_t)row * K + bk * kChunk + col) = c;
    }
}

hipError_t launch_wquant(const uint16_t* w, uint8_t* q, float* scale_inv, int N, int K,
                         hipStream_t stream)
{
    const dim3 grid(K / kChunk, (N + kChunk - 1) / kChunk);
    wquant_block_kernel<<<grid, 256, 0, stream>>>(w, q, scale_inv, N, K);
    return hipGetLastError();
}

}  // namespace heph
