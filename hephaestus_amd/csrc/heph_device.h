// heph_device.h - gfx950 device helpers shared by the FP8 linear kernels.
//
// Operand layout used by every MFMA kernel here (v_mfma_f32_16x16x128_f8f6f4,
// wave64): lane l holds row (l & 15) of the A tile and column (l & 15) of the
// B tile; its 32 operand bytes are the K positions
//   [s*16, s*16+16) and [64 + s*16, 64 + s*16 + 16)   with s = l >> 4
// of the 128-wide K chunk. A and B use the same lane -> K assignment, so the
// contraction is exact whatever order the hardware walks the 32 bytes in.
// Result layout (4 floats per lane): element i is row (l >> 4) * 4 + i,
// column l & 15 of the 16x16 tile.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "group_scale.h"

namespace heph {

typedef int      i32x4 __attribute__((ext_vector_type(4)));
typedef int      i32x8 __attribute__((ext_vector_type(8)));
typedef float    f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16   bf16x8 __attribute__((ext_vector_type(8)));

constexpr float kE4M3Max = 448.0f;
constexpr int kChunk = 128;  // K positions per MFMA / per scale group

// D = A(16x128, e4m3) * B(128x16, e4m3) + C, fp32 accumulation.
// The scale operands are zero, so the compiler emits the unscaled
// v_mfma_f32_16x16x128_f8f6f4 (format code 0 = E4M3 for both operands).
__device__ __forceinline__ f32x4 mfma_e4m3(const i32x8& a, const i32x8& b,
                                           const f32x4& c)
{
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0,
                                                            0, 0);
}

// D = A(16x32, bf16) * B(32x16, bf16) + C.
__device__ __forceinline__ f32x4 mfma_bf16(const bf16x8& a, const bf16x8& b,
                                           const f32x4& c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ i32x8 join(const i32x4& lo, const i32x4& hi)
{
    return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Two bf16 packed in a dword -> two floats (exact).
__device__ __forceinline__ float bf16lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// f32 -> bf16 bits, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// SwiGLU of one element from bf16 bits g and u (low 16 bits), as the decode
// step's silu_mul rounds it: bf16(bf16(g / (1 + exp(-g))) * u).
__device__ __forceinline__ uint32_t swiglu_bits(uint32_t g16, uint32_t u16)
{
    const float g = __uint_as_float(g16 << 16);
    const float s = __uint_as_float((uint32_t)f32_to_bf16(__fdiv_rn(g, 1.0f + expf(-g))) << 16);
    return f32_to_bf16(s * __uint_as_float(u16 << 16));
}

// Four floats -> four E4M3FN codes (byte i = code of value i) with the
// hardware converter (round to nearest even).
__device__ __forceinline__ uint32_t pack4_e4m3(float a, float b, float c, float d)
{
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    return (uint32_t)w;
}

// Largest |x| over bf16 values held two per dword, as bf16 magnitude bits
// (0 .. 0x7FFF). For values that are not NaN, |x| orders as the unsigned
// integer bits & 0x7FFF, so two values cost one AND and one packed 16-bit
// max. A result above 0x7F80 means a NaN is present; then the reference's
// amax, whose `v > local` test skips NaN (kernels.mojo:153-160), is the
// *_skip_nan form. (A float max chain is no substitute: v_max3_f32 returns
// NaN for a signalling-NaN operand and so drops the running maximum.)
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

template <int N>
__device__ __forceinline__ uint32_t absmax_bits(const uint32_t (&d)[N], uint32_t m = 0)
{
    u16x2 p = {0, 0};
#pragma unroll
    for (int i = 0; i < N; ++i)
        p = __builtin_elementwise_max(p, __builtin_bit_cast(u16x2, d[i] & 0x7FFF7FFFu));
    const uint32_t r = p.x > p.y ? p.x : p.y;
    return r > m ? r : m;
}

template <int N>
__device__ __forceinline__ uint32_t absmax_bits_skip_nan(const uint32_t (&d)[N], uint32_t m = 0)
{
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const uint32_t lo = d[i] & 0x7FFFu, hi = (d[i] >> 16) & 0x7FFFu;
        if (lo <= 0x7F80u && lo > m) m = lo;
        if (hi <= 0x7F80u && hi > m) m = hi;
    }
    return m;
}

__device__ __forceinline__ uint32_t absmax_bits8(const uint4& v, uint32_t m = 0)
{
    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
    return absmax_bits(d, m);
}

__device__ __forceinline__ uint32_t absmax_bits8_skip_nan(const uint4& v, uint32_t m = 0)
{
    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
    return absmax_bits_skip_nan(d, m);
}

// The magnitude bits as the float they encode.
__device__ __forceinline__ float bf16_bits_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ uint32_t shfl_xor_u(uint32_t v, int o)
{
    return (uint32_t)__shfl_xor((int)v, o);
}

// Eight bf16 times inv -> eight codes in two dwords.
__device__ __forceinline__ uint2 quant8(const uint4& v, float inv)
{
    uint2 r;
    r.x = pack4_e4m3(bf16lo(v.x) * inv, bf16hi(v.x) * inv, bf16lo(v.y) * inv,
                     bf16hi(v.y) * inv);
    r.y = pack4_e4m3(bf16lo(v.z) * inv, bf16hi(v.z) * inv, bf16lo(v.w) * inv,
                     bf16hi(v.w) * inv);
    return r;
}

// Group scale of the reference quantizer for a bf16 amax: s = RN(amax/448)
// (1.0 when below 1e-12) and inv = RN(1/s), division-free (group_scale.h):
// mantissa parts from an FMA-corrected product and an FMA Newton step on
// the hardware reciprocal, exponents by ldexp. amax must be the magnitude
// of a bf16 value (low 16 bits zero); zero and subnormal amax take the
// floor, an infinite amax gives s = inf, inv = 0 as the division would.
// Branch-free: a short dependent chain, as it sits between an activation
// load and the first MFMA that uses it.
__device__ __forceinline__ void group_scale(float amax, float& s, float& inv)
{
    const uint32_t u = __float_as_uint(amax);
    const int e = (int)(u >> 23);
    const float q = scale_mant((float)(int)(128u + ((u >> 16) & 0x7Fu)));
    const float y = inv_mant(q, __builtin_amdgcn_rcpf(q));
    s = __builtin_amdgcn_ldexpf(q, e - 140);
    inv = __builtin_amdgcn_ldexpf(y, 140 - e);
    if (e == 255) {
        s = __builtin_inff();
        inv = 0.0f;
    }
    if (e == 0 || s < 1e-12f) {
        s = 1.0f;
        inv = 1.0f;
    }
}

__device__ __forceinline__ i32x4 ldg16(const void* p)
{
    return *reinterpret_cast<const i32x4*>(p);
}

// The fold v[l] += v[l + h], h = 32, 16, ..., 1, over the 64 lanes of a
// wave, lane 0's result broadcast. Every level stays in the VALU: h = 32
// and 16 by v_permlane32_swap / v_permlane16_swap (lane l < h receives lane
// l + h), 8 and 4 by DPP row_ror (within a 16-lane row, lane l < h reads
// lane l + h), 2 and 1 by DPP quad_perm (lane l ^ h). Lane 0 forms exactly
// the sums the fold's lane 0 forms (float addition commutes), without the
// LDS round trip of each level that ds_bpermute (__shfl_down) takes.
__device__ __forceinline__ float wave_fold_sum64(float v)
{
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xf, 0xf, false));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
}

// Max over the 64 lanes of a wave (exact in any order), in every lane: the
// same six exchanges; each level leaves equal values in the lanes the next
// one pairs, so every lane ends with the maximum.
__device__ __forceinline__ float wave_fold_max64(float v)
{
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xf, 0xf, false)));
    return v;
}

// RMSNorm's sum of squares over one row: thread t < 256 of the workgroup
// brings v = its fma chain over elements t, t + 256, ...; the 256 sums are
// folded as s[t] += s[t + h] for h = 128, 64, ..., 1, the first two levels
// read by wave 0 from LDS as (s[t] + s[t+128]) + (s[t+64] + s[t+192]), the
// rest moved between its lanes: two barriers (every thread of the
// workgroup calls it). red holds 256 floats, out one.
__device__ __forceinline__ float fold256_wave0(float v, float* red, float* out)
{
    const int t = threadIdx.x;
    if (t < 256) red[t] = v;
    __syncthreads();
    if (t < 64) {
        const float a = (red[t] + red[t + 128]) + (red[t + 64] + red[t + 192]);
        const float r = wave_fold_sum64(a);
        if (t == 0) *out = r;
    }
    __syncthreads();
    return *out;
}

// The same fold with its result in every wave and one barrier: after the
// first level's barrier each wave repeats wave 0's part (same operands, same
// order) and takes lane 0's sum.
__device__ __forceinline__ float fold256_every_wave(float v, float* red)
{
    const int t = threadIdx.x, l = t & 63;
    if (t < 256) red[t] = v;
    __syncthreads();
    const float a = (red[l] + red[l + 128]) + (red[l + 64] + red[l + 192]);
    return wave_fold_sum64(a);
}

// sqrt(a) rounded to nearest, for the RMS factors. __fsqrt_rn compiles to
// v_sqrt_f32, which is within one ulp but not always the nearest float (a
// 512-row RMSNorm test met one row off by an ulp against the host's sqrtf).
// With y that estimate and d, u its neighbours below and above: sqrt(a) is
// nearer d than y iff a <= d*y, nearer u iff a > u*y. (The midpoint m of y
// and d has m^2 = d*y + (y-d)^2/4, and that excess is ~2^-48 of a, far
// below a's own spacing of ~2^-23, so no float a lies between d*y and m^2;
// equality a == d*y puts sqrt(a) below m. Likewise for u.) Each product is
// compared exactly through the sign of one FMA. a <= 0, inf and NaN keep
// the estimate.
__device__ __forceinline__ float sqrt_rn(float a)
{
    const float y = __fsqrt_rn(a);
    if (!(a > 0.0f) || !__builtin_isfinite(a)) return y;
    const uint32_t b = __float_as_uint(y);
    const float d = __uint_as_float(b - 1u), u = __uint_as_float(b + 1u);
    if (__builtin_fmaf(-d, y, a) <= 0.0f) return d;
    if (__builtin_fmaf(-u, y, a) > 0.0f) return u;
    return y;
}

__device__ __forceinline__ float rms_inv(float ss, int cols, float eps)
{
    return __fdiv_rn(1.0f, sqrt_rn(__fdiv_rn(ss, (float)cols) + eps));
}

__device__ __forceinline__ uint4 ldg16u(const void* p)
{
    return *reinterpret_cast<const uint4*>(p);
}

}  // namespace heph
