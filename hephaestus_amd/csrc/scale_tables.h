// scale_tables.h - exact group scales from a bf16 amax without division.
//
// The quantizer needs s = RN(amax / 448) and inv = RN(1 / s) in f32
// (reference src/hephaestus/kernels.mojo:173-182). A group's amax is the
// magnitude of one bf16 element, so for a normal amax
//     amax = (128 + m) * 2^(e - 134),   m = 7 fraction bits, e = f32 exponent
// and, because scaling by a power of two commutes with rounding in the
// normal range,
//     s   = RN((128 + m) / 448) * 2^(e - 134)      = kScaleMant[m]  * 2^(e-134)
//     inv = RN(1 / RN((128 + m)/448)) * 2^(134 - e) = kInvMant[m]   * 2^(134-e)
// Both results stay normal for every amax that survives the 1e-12 floor
// (s >= 1e-12, inv <= 1e12; the largest bf16 gives s ~ 7.6e35, inv ~
// 1.3e-36). The two 128-entry tables are constant-folded by the compiler,
// whose floating-point folding is correctly rounded.
#pragma once

#include <stdint.h>

namespace heph {

struct ScaleTables {
    float scale[128];
    float inv[128];
};

constexpr ScaleTables make_scale_tables()
{
    ScaleTables t{};
    for (int m = 0; m < 128; ++m) {
        t.scale[m] = (float)(128 + m) / 448.0f;
        t.inv[m] = 1.0f / t.scale[m];
    }
    return t;
}

inline constexpr ScaleTables kScaleTables = make_scale_tables();

}  // namespace heph
