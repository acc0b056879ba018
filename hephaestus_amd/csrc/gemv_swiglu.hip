// gemv_swiglu.hip - the decode step's feed-forward input in one launch:
// RMSNorm (optional) + the gate/up linear + SwiGLU for one row, through the
// chunk-slot GEMV's SwiGLU epilogue (gemv_kernel.h).
//
// Replaces rms_norm + linear_fp8(gate_proj) + linear_fp8(up_proj) + silu_mul
// of the reference's decode step (src/hephaestus/forward.mojo:537-578;
// silu_mul, kernels.mojo:1243-1278). The weight holds the gate rows then the
// up rows; each workgroup finishes TW/2 gate and TW/2 up columns, so the
// SwiGLU of a column pair runs once, where both sums are, and neither the
// gate/up output nor a SwiGLU launch exists. The launch shape (chunk
// slots, waves, steps per batch) is the one the M = 1 GEMV takes for the
// same N x K (with the norm: the RMSNorm-fused GEMV's), so every sum runs in
// the same order: the output is bit for bit the two-launch form's.
#include "gemv_kernel.h"

namespace heph {

namespace {

template <int WAVES, int KS, int U>
hipError_t launch_glu(const GemvArgs& a, hipStream_t stream, const LaunchTiming& t)
{
    const dim3 grid(a.op.N / (16 / KS)), block(WAVES * 64);
    if (a.gamma) {
        if (a.op.w_block)
            return launch(fp8_gemv_kernel<WAVES, KS, 1, 1, U, true, kGemvBlock, true, true>, grid,
                          block, 0, stream, t, a);
        return launch(fp8_gemv_kernel<WAVES, KS, 1, 1, U, true, kGemvChannel, true, true>, grid,
                      block, 0, stream, t, a);
    }
    if (a.op.w_block)
        return launch(fp8_gemv_kernel<WAVES, KS, 1, 1, U, true, kGemvBlock, false, true>, grid,
                      block, 0, stream, t, a);
    return launch(fp8_gemv_kernel<WAVES, KS, 1, 1, U, true, kGemvChannel, false, true>, grid,
                  block, 0, stream, t, a);
}

template <int WAVES, int U>
hipError_t launch_glu_ks(const GemvArgs& a, int ks, hipStream_t stream, const LaunchTiming& t)
{
    switch (ks) {
    case 8: return launch_glu<WAVES, 8, U>(a, stream, t);
    case 4: return launch_glu<WAVES, 4, U>(a, stream, t);
    case 2: return launch_glu<WAVES, 2, U>(a, stream, t);
    default: return launch_glu<WAVES, 1, U>(a, stream, t);
    }
}

}  // namespace

hipError_t launch_fp8_gemv_swiglu(const Fp8Operands& op, hipStream_t stream,
                                  const LaunchTiming& t, const char** name,
                                  const uint16_t* gamma, float eps)
{
    const GemvArgs a{op, true, gamma, eps};
    int ks, waves, u;
    gemv_shape(1, op.N, op.K, Tuning{}, &ks, &waves, &u, gamma != nullptr);
    *name = gamma ? "fp8_gemv_rmsnorm_swiglu_m1" : "fp8_gemv_swiglu_m1";
    // M = 1 takes 4, 5, 8 or 10 waves (gemv_shape; 5 and 10 in one-step batches)
    switch (waves) {
    case 4:
        return u == 2 ? launch_glu_ks<4, 2>(a, ks, stream, t) : launch_glu_ks<4, 1>(a, ks, stream, t);
    case 5: return launch_glu_ks<5, 1>(a, ks, stream, t);
    case 10: return launch_glu_ks<10, 1>(a, ks, stream, t);
    default:
        return u == 2 ? launch_glu_ks<8, 2>(a, ks, stream, t) : launch_glu_ks<8, 1>(a, ks, stream, t);
    }
}

}  // namespace heph
