// group_scale.h - exact group scales from a bf16 amax without division.
//
// The quantizer needs s = RN(amax / 448) and inv = RN(1 / s) in f32
// (reference src/hephaestus/kernels.mojo:173-182). A group's amax is the
// magnitude of one bf16 element, so for a normal amax
//     amax = a * 2^(e - 134),   a = 128 + (7 fraction bits), e = f32 exponent
// and, because 448 = 7 * 2^6 and scaling by a power of two commutes with
// rounding in the normal range,
//     s   = RN(a / 7)     * 2^(e - 140)
//     inv = RN(1 / RN(a/7)) * 2^(140 - e)
// Both stay normal for every amax that survives the 1e-12 floor (s >=
// 1e-12, inv <= 1e12; the largest bf16 gives s ~ 7.6e35, inv ~ 1.3e-36).
//
// The two mantissa functions need no division:
//   * RN(a/7) for the integers a in [128, 255]: q0 = RN(a * RN(1/7)), the
//     remainder r = a - 7*q0 (exact in one FMA), q = RN(q0 + r * RN(1/7));
//   * RN(1/q) from any y0 within one ulp of 1/q (the hardware reciprocal):
//     one Newton step with FMAs, y = RN(y0 + y0 * (1 - q*y0)).
// Both are exact for every one of the 128 mantissas (and, for the second,
// each of the three f32 values within one ulp of 1/q); the host test
// compiles this header and checks them against IEEE division.
#pragma once

#if defined(__HIPCC__) || defined(__HIP__)
#define HEPH_HD __host__ __device__
#else
#define HEPH_HD
#endif

namespace heph {

// RN(a / 7) for an integer a in [128, 255].
HEPH_HD inline float scale_mant(float a)
{
    constexpr float k7 = 1.0f / 7.0f;
#if defined(__HIP_DEVICE_COMPILE__)
    const float q0 = __fmul_rn(a, k7);    // one rounded product, never contracted
#else
    volatile float q0v = a * k7;
    const float q0 = q0v;
#endif
    return __builtin_fmaf(__builtin_fmaf(-q0, 7.0f, a), k7, q0);
}

// RN(1 / q) from y0 within one ulp of 1 / q, q = scale_mant(a).
HEPH_HD inline float inv_mant(float q, float y0)
{
    return __builtin_fmaf(__builtin_fmaf(-q, y0, 1.0f), y0, y0);
}

}  // namespace heph
