// producers.hip - the ops that feed an FP8 linear, quantizing their own
// output (gfx950): RMSNorm + activation quantization and SwiGLU +
// activation quantization, for rows of a prefill (or decode) batch.
//
// In the reference every FP8 linear quantizes its bf16 input in a separate
// launch (quantize_act_rows_fp8, src/hephaestus/kernels.mojo:270-287, called
// from linear_fp8 at :449-450) right after the op that produced that input
// (rms_norm, forward.mojo:45-81; silu_mul, kernels.mojo:1243-1278); the
// reference's own notes blame its FP8 GEMM gap on that extra launch and the
// extra pass over the activations. Here the producer writes the E4M3 codes
// and scales itself, bit for bit what heph_rmsnorm (heph_silu_mul) followed
// by heph_fp8_quant_act write, and the linear runs with
// HEPH_FLAG_SKIP_QUANT: one launch and one read of the bf16 activations
// fewer per linear, and the normalized (activated) bf16 row is never
// written.
#include "../../include/hephdecode.h"
#include "heph_kernels.h"

namespace heph {

namespace {

// Longest row the fused ops hold in LDS as bf16 (32 KB).
constexpr int kProdMaxCols = 16384;

__device__ __forceinline__ float f32b(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ float rbf16(float f) { return f32b(f32_to_bf16(f)); }

// Quantizes one row held as bf16 in LDS (yrow, cols elements) into codes
// q[cols] and scales s[cols / group_k], as quant_g128_kernel (group 128:
// 16-lane teams over 8 elements each, amax on bf16 magnitude bits, NaN
// skipped) or quant_row_kernel (group cols) do. Every thread of the
// 256-thread workgroup calls it after the row is in LDS.
__device__ __forceinline__ void quant_row_from_lds(const uint16_t* yrow, int cols, int group_k,
                                                   uint8_t* q, float* s)
{
    const int t = threadIdx.x;
    if (group_k == kChunk) {
        const int G = cols / kChunk, team = t >> 4, j = t & 15;
        for (int g0 = 0; g0 < G; g0 += 16) {
            const int g = g0 + team;
            const bool live = g < G;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (live) v = *reinterpret_cast<const uint4*>(yrow + g * kChunk + j * 8);
            uint32_t mb = absmax_bits8(v);
            for (int o = 1; o < 16; o <<= 1) mb = max(mb, shfl_xor_u(mb, o));
            if (__builtin_amdgcn_ballot_w64(mb > 0x7F80u) != 0) {
                mb = absmax_bits8_skip_nan(v);
                for (int o = 1; o < 16; o <<= 1) mb = max(mb, shfl_xor_u(mb, o));
            }
            float sc, inv;
            group_scale(bf16_bits_f32(mb), sc, inv);
            if (live) {
                *reinterpret_cast<uint2*>(q + g * kChunk + j * 8) = quant8(v, inv);
                if (j == 0) s[g] = sc;
            }
        }
        return;
    }
    __shared__ uint32_t red[4];
    uint32_t m = 0;
    for (int k = t * 8; k < cols; k += 256 * 8)
        m = absmax_bits8_skip_nan(*reinterpret_cast<const uint4*>(yrow + k), m);
    for (int o = 32; o >= 1; o >>= 1) m = max(m, shfl_xor_u(m, o));
    if ((t & 63) == 0) red[t >> 6] = m;
    __syncthreads();
    m = max(max(red[0], red[1]), max(red[2], red[3]));
    float sc, inv;
    group_scale(bf16_bits_f32(m), sc, inv);
    if (t == 0) s[0] = sc;
    for (int k = t * 8; k < cols; k += 256 * 8)
        *reinterpret_cast<uint2*>(q + k) = quant8(*reinterpret_cast<const uint4*>(yrow + k), inv);
}

// One 256-thread workgroup per row. The norm is heph_rmsnorm's: thread t
// owns elements t, t + 256, ... and sums their squares in that order (fma),
// the 256 sums fold as fold256_wave0 does, and y = bf16(gamma * bf16(x * r)).
// y goes to LDS instead of global memory (dynamic, 2 * cols bytes, so that
// short rows leave room for more workgroups per CU); then the row is
// quantized.
template <int PER>
__global__ __launch_bounds__(256) void rmsnorm_quant_kernel(uint8_t* q, float* scales,
                                                            const uint16_t* in,
                                                            const uint16_t* gamma, int cols,
                                                            float eps, int group_k)
{
    __shared__ float red[256];
    __shared__ float res;
    extern __shared__ __attribute__((aligned(16))) uint16_t yrow[];
    const uint16_t* x = in + (size_t)blockIdx.x * cols;
    const int t = threadIdx.x;
    if constexpr (PER > 0) {
        float v[PER], g[PER];
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int i = t + e * 256;
            v[e] = i < cols ? f32b(x[i]) : 0.0f;
            g[e] = i < cols ? f32b(gamma[i]) : 0.0f;
        }
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < PER; ++e)
            if (t + e * 256 < cols) ss = __builtin_fmaf(v[e], v[e], ss);
        const float r = rms_inv(fold256_wave0(ss, red, &res), cols, eps);
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int i = t + e * 256;
            if (i < cols) yrow[i] = f32_to_bf16(g[e] * rbf16(v[e] * r));
        }
    } else {
        float ss = 0.0f;
        for (int i = t; i < cols; i += 256) {
            const float v = f32b(x[i]);
            ss = __builtin_fmaf(v, v, ss);
        }
        const float r = rms_inv(fold256_wave0(ss, red, &res), cols, eps);
        for (int i = t; i < cols; i += 256)
            yrow[i] = f32_to_bf16(f32b(gamma[i]) * rbf16(f32b(x[i]) * r));
    }
    __syncthreads();
    quant_row_from_lds(yrow, cols, group_k, q + (size_t)blockIdx.x * cols,
                       scales + (size_t)blockIdx.x * (cols / group_k));
}

__device__ __forceinline__ uint4 swiglu8(const uint4& g, const uint4& u)
{
    const uint32_t gd[4] = {g.x, g.y, g.z, g.w}, ud[4] = {u.x, u.y, u.z, u.w};
    uint32_t r[4];
#pragma unroll
    for (int d = 0; d < 4; ++d)
        r[d] = swiglu_bits((uint16_t)gd[d], (uint16_t)ud[d]) |
               (swiglu_bits((uint16_t)(gd[d] >> 16), (uint16_t)(ud[d] >> 16)) << 16);
    return make_uint4(r[0], r[1], r[2], r[3]);
}

// 1x128 groups: one 16-lane team per group of one row, 8 elements a lane,
// the SwiGLU values computed in registers and quantized as
// quant_g128_kernel does.
__global__ __launch_bounds__(256) void silu_mul_quant_g128_kernel(
    uint8_t* __restrict__ q, float* __restrict__ scales, const uint16_t* __restrict__ gate,
    const uint16_t* __restrict__ up, int n, long ld, long n_groups)
{
    const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long gi = t >> 4;
    const int j = threadIdx.x & 15;
    const bool live = gi < n_groups;
    const int G = n / kChunk;
    const long row = live ? gi / G : 0, g = live ? gi % G : 0;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (live) {
        const size_t off = (size_t)row * ld + (size_t)g * kChunk + j * 8;
        v = swiglu8(ldg16u(gate + off), ldg16u(up + off));
    }
    uint32_t mb = absmax_bits8(v);
    for (int o = 1; o < 16; o <<= 1) mb = max(mb, shfl_xor_u(mb, o));
    if (__builtin_amdgcn_ballot_w64(mb > 0x7F80u) != 0) {
        mb = absmax_bits8_skip_nan(v);
        for (int o = 1; o < 16; o <<= 1) mb = max(mb, shfl_xor_u(mb, o));
    }
    float s, inv;
    group_scale(bf16_bits_f32(mb), s, inv);
    if (live) {
        *reinterpret_cast<uint2*>(q + (size_t)row * n + g * kChunk + j * 8) = quant8(v, inv);
        if (j == 0) scales[row * G + g] = s;
    }
}

// Per-token groups: one workgroup per row, the row's SwiGLU values staged
// in LDS, then quantized as quant_row_kernel does.
__global__ __launch_bounds__(256) void silu_mul_quant_row_kernel(uint8_t* q, float* scales,
                                                                 const uint16_t* gate,
                                                                 const uint16_t* up, int n,
                                                                 long ld)
{
    extern __shared__ __attribute__((aligned(16))) uint16_t yrow[];    // n bf16
    const size_t off = (size_t)blockIdx.x * ld;
    for (int k = threadIdx.x * 8; k < n; k += 256 * 8)
        *reinterpret_cast<uint4*>(yrow + k) = swiglu8(ldg16u(gate + off + k), ldg16u(up + off + k));
    __syncthreads();
    quant_row_from_lds(yrow, n, n, q + (size_t)blockIdx.x * n, scales + blockIdx.x);
}

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

}  // namespace heph

using namespace heph;

extern "C" {

int heph_rmsnorm_quant_fp8(uint8_t* q, float* scales, const uint16_t* x_bf16,
                           const uint16_t* gamma_bf16, int rows, int cols, float eps, int group_k,
                           void* stream)
{
    if (!q || !scales || !x_bf16 || !gamma_bf16) return HEPH_ERR_NULL;
    if (rows < 1 || cols < kChunk || cols % kChunk) return HEPH_ERR_SHAPE;
    if (group_k != kChunk && group_k != cols) return HEPH_ERR_GROUP;
    if (cols > kProdMaxCols) return HEPH_ERR_UNSUPPORTED;
    if (!a16(q)) return HEPH_ERR_ALIGN;
    if (int st = check_device()) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int per = (cols + 255) / 256;
    const size_t lds = (size_t)cols * 2;
    if (per <= 10)
        rmsnorm_quant_kernel<10><<<rows, 256, lds, s>>>(q, scales, x_bf16, gamma_bf16, cols, eps,
                                                      group_k);
    else if (per <= 16)
        rmsnorm_quant_kernel<16><<<rows, 256, lds, s>>>(q, scales, x_bf16, gamma_bf16, cols, eps,
                                                      group_k);
    else if (per <= 40)
        rmsnorm_quant_kernel<40><<<rows, 256, lds, s>>>(q, scales, x_bf16, gamma_bf16, cols, eps,
                                                      group_k);
    else
        rmsnorm_quant_kernel<0><<<rows, 256, lds, s>>>(q, scales, x_bf16, gamma_bf16, cols, eps,
                                                     group_k);
    return hipGetLastError() == hipSuccess ? HEPH_OK : HEPH_ERR_LAUNCH;
}

int heph_silu_mul_quant_fp8(uint8_t* q, float* scales, const uint16_t* gate_bf16,
                            const uint16_t* up_bf16, int rows, int n, int ld, int group_k,
                            void* stream)
{
    if (!q || !scales || !gate_bf16 || !up_bf16) return HEPH_ERR_NULL;
    if (rows < 1 || n < kChunk || n % kChunk || ld < n || ld % 8) return HEPH_ERR_SHAPE;
    if (group_k != kChunk && group_k != n) return HEPH_ERR_GROUP;
    if (group_k == n && n > kProdMaxCols) return HEPH_ERR_UNSUPPORTED;
    if (!a16(q) || !a16(gate_bf16) || !a16(up_bf16)) return HEPH_ERR_ALIGN;
    if (int st = check_device()) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (group_k == kChunk) {
        const long n_groups = (long)rows * (n / kChunk);
        const unsigned blocks = (unsigned)((n_groups * 16 + 255) / 256);
        silu_mul_quant_g128_kernel<<<blocks, 256, 0, s>>>(q, scales, gate_bf16, up_bf16, n,
                                                          (long)ld, n_groups);
    } else {
        silu_mul_quant_row_kernel<<<rows, 256, (size_t)n * 2, s>>>(q, scales, gate_bf16, up_bf16,
                                                                    n, (long)ld);
    }
    return hipGetLastError() == hipSuccess ? HEPH_OK : HEPH_ERR_LAUNCH;
}

}  // extern "C"
