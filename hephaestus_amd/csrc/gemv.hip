// gemv.hip - launch shapes and launchers of the chunk-slot GEMV
// (gemv_kernel.h) for 1 <= M <= 32.
#include "gemv_kernel.h"

namespace heph {

namespace {

template <int WAVES, int KS, int MR, int MT, int U>
hipError_t launch_ks(const GemvArgs& a, bool fused, hipStream_t stream, const LaunchTiming& t)
{
    const dim3 grid(a.op.N / (16 / KS));
    const dim3 block(WAVES * 64);
    if (a.gamma) {
        if constexpr (MR == 1 && MT == 1 && WAVES >= 4) {
            if (a.op.w_block)
                return launch(fp8_gemv_kernel<WAVES, KS, MR, MT, U, true, kGemvBlock, true>, grid,
                              block, 0, stream, t, a);
            return launch(fp8_gemv_kernel<WAVES, KS, MR, MT, U, true, kGemvChannel, true>, grid,
                          block, 0, stream, t, a);
        }
        return hipErrorInvalidValue;
    }
    if (fused) {
        if (a.op.w_block)
            return launch(fp8_gemv_kernel<WAVES, KS, MR, MT, U, true, kGemvBlock>, grid, block,
                          0, stream, t, a);
        return launch(fp8_gemv_kernel<WAVES, KS, MR, MT, U, true, kGemvChannel>, grid, block,
                      0, stream, t, a);
    }
    if (a.op.w_block)
        return launch(fp8_gemv_kernel<WAVES, KS, MR, MT, U, false, kGemvBlock>, grid, block,
                      0, stream, t, a);
    if (a.op.s_step == 0)
        return launch(fp8_gemv_kernel<WAVES, KS, MR, MT, U, false, kGemvConst>, grid, block,
                      0, stream, t, a);
    return launch(fp8_gemv_kernel<WAVES, KS, MR, MT, U, false, kGemvChannel>, grid, block, 0,
                  stream, t, a);
}

template <int WAVES, int MR, int MT, int U>
hipError_t launch_mr(const GemvArgs& a, bool fused, int ks, hipStream_t stream,
                     const LaunchTiming& t)
{
    if constexpr (8 * MR <= 16)
        if (ks == 8) return launch_ks<WAVES, 8, MR, MT, U>(a, fused, stream, t);
    if constexpr (4 * MR <= 16)
        if (ks == 4) return launch_ks<WAVES, 4, MR, MT, U>(a, fused, stream, t);
    if constexpr (2 * MR <= 16)
        if (ks == 2) return launch_ks<WAVES, 2, MR, MT, U>(a, fused, stream, t);
    return launch_ks<WAVES, 1, MR, MT, U>(a, fused, stream, t);
}

template <int WAVES, int U>
hipError_t launch_wu(const GemvArgs& a, bool fused, int ks, int mr, hipStream_t stream,
                     const LaunchTiming& t)
{
    // 16-wave workgroups (128 VGPRs a lane) serve the one-slot, one-tile
    // shapes of 8 < M <= 16 only, where N/16 workgroups are few.
    if constexpr (WAVES < 16) {
        switch (mr) {
        case 1: return launch_mr<WAVES, 1, 1, U>(a, fused, ks, stream, t);
        case 2: return launch_mr<WAVES, 2, 1, U>(a, fused, ks, stream, t);
        case 4: return launch_mr<WAVES, 4, 1, U>(a, fused, ks, stream, t);
        case 8: return launch_mr<WAVES, 8, 1, U>(a, fused, ks, stream, t);
        default: break;
        }
        if (a.op.M > 16) return launch_ks<WAVES, 1, 16, 2, U>(a, fused, stream, t);
    }
    return launch_ks<WAVES, 1, 16, 1, U>(a, fused, stream, t);
}

// Two column groups per workgroup (fused, M = 1, four chunk slots: 8
// columns a workgroup).
template <int WAVES, int U>
hipError_t launch_groups2(const GemvArgs& a, hipStream_t stream, const LaunchTiming& t)
{
    const dim3 grid(a.op.N / 8);
    const dim3 block(WAVES * 64);
    if (a.op.w_block)
        return launch(fp8_gemv_kernel<WAVES, 4, 1, 1, U, true, kGemvBlock, false, false, 2>, grid,
                      block, 0, stream, t, a);
    return launch(fp8_gemv_kernel<WAVES, 4, 1, 1, U, true, kGemvChannel, false, false, 2>, grid,
                  block, 0, stream, t, a);
}

}  // namespace

// Fused quantization re-quantizes x in every workgroup (N*KS/16 of them).
// Up to M = 16 that costs less than a separate quantizer launch on every
// config shape; with two 16-row tiles it pays only while N*K is small
// (measured on MI355X: faster at qkv and o_proj, slower at gate_up and
// down, M = 32).
bool gemv_fuses(int M, int N, int K)
{
    return M <= 16 || (long)N * K <= (16L << 20);
}

int gemv_rows(int M)
{
    return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16;
}

// Launch shape. M = 1 without a fused norm: four chunk slots from K = 1024
// on (fewer only where N is large enough without them), and waves for one
// step each, else two, while the workgroups' waves fit the CUs at once (32
// per CU); past that 4 waves. MI355X, graph-replayed per call over rotated
// weights, against the norm forms' shape below: gate_up 11.0 against 11.8
// us (4 slots x 4 waves, 4864 workgroups), down 8.1 against 8.3 (4 x 10),
// qkv 5.5 against 5.6 (4 x 5), q_proj 4.6 against 4.7 (4 x 5), o_proj
// unchanged (4 x 8).
// Otherwise chunk slots: at M <= 2 the fewest (at most 16 / rows per
// slot) that give >= 600 workgroups (about 2.3 per CU; the norm forms
// >= 256); at 4 and 8 rows
// per slot one, as every workgroup quantizes all M x K activations again
// and wider workgroups do that less often (MI355X, graph-replayed, fused:
// M = 8 qkv 7.6 against 9.1 us with two slots, o_proj 6.3 against 7.6,
// down 13.3 against 16.5); 16 rows: one.
// Waves: at M = 1 (norm forms), 8 from 4 steps on (o_proj 4.85 against
// 5.06 us with 4 waves of 2-step batches, q_proj 4.70 against 4.97); at
// M >= 2, 4 when there are fewer than 8 steps, else 8; at 4 and 8 rows per
// slot 10 when K >= 8192, at 4 rows 4 from 1024 workgroups on (below); at 9..16
// rows 4 up to 24 steps (M = 16 qkv 9.9 against 10.9 us); 16 only when
// forced, for 8 < M <= 16. Steps per batch: at M = 1 (norm forms) two
// when each wave has exactly 2 steps; at 3..4 rows with K >= 8192 two;
// else one (wider activation tiles need the registers).
void gemv_shape(int M, int N, int K, const Tuning& tune, int* ks, int* waves, int* u,
                bool norm, int* groups)
{
    const int mr = gemv_rows(M);
    const int kmax = mr >= 2 ? 16 / mr : 8;
    const int tiles = N / 16, KC = K / kChunk;
    const bool plain1 = mr == 1 && !norm;
    int k = 1;
    // the norm forms: enough workgroups for one per CU (each repeats the
    // norm; MI355X decode step with qkv at 384 workgroups instead of 768:
    // -17 us per token); else >= 600
    const int min_wgs = mr == 1 && norm ? 256 : 600;
    if (mr <= 2)
        while (k < kmax && tiles * k < min_wgs) k *= 2;
    else if (mr == 4 && K >= 8192)
        k = 2;
    if (plain1 && k < 4 && KC >= 8) k = 4;
    // 4 and 8 rows per slot with K >= 8192: one slot (10 waves below)
    const bool long_k = (mr == 4 || mr == 8) && K >= 8192;
    if (long_k) k = 1;
    const int fk = tune.gemv_ks;
    if (fk) k = fk < kmax ? fk : kmax;
    const int S = (KC + k - 1) / k;
    int w = mr == 1 ? (S <= 3 ? 4 : 8) : (S < 8 ? 4 : 8);
    // 4 and 8 rows per slot: 10 waves over a long K; at 4 rows 4 waves
    // where there are >= 1024 workgroups (MI355X, bf16 rows, graph-replayed,
    // interleaved repeats: M = 4 down 10.8 against 11.5 us, gate_up 12.5
    // against 13.8; M = 8 down 13.2 against 13.3; M = 8 gate_up unchanged
    // by 4 waves)
    if (long_k) w = 10;
    else if (mr == 4 && (long)tiles * k >= 1024) w = 4;
    // Column groups (fused M = 1 with four slots): two where that still
    // leaves >= 640 workgroups. Every workgroup reads all K activations for
    // its columns, 2 bytes each: with four columns that is half as many
    // bytes again as its weights, and a one-pass read of the weights with
    // those activation loads beside them took (MI355X, graph-replayed)
    // 5.1 against 4.5 us (qkv) and 10.8 against 9.5 (gate_up); with eight
    // columns 4.4 and 9.9.
    int cg = 1;
    if (groups && plain1 && k == 4 && (long)tiles * k / 2 >= 640) cg = 2;
    if (groups && tune.gemv_groups) cg = plain1 && k == 4 ? tune.gemv_groups : 1;
    if (plain1) {
        // the fewest steps per wave (1, then 2) whose wave count, rounded up
        // to one of 4, 5, 8, 10, fits every workgroup on the CUs at once
        const long budget = 32L * kPlanCUs, wgs = (long)tiles * k / cg;
        w = 4;
        for (int p = 1; p <= 2; ++p) {
            int need = (S + p - 1) / p;
            need = need <= 4 ? 4 : need <= 5 ? 5 : need <= 8 ? 8 : need <= 10 ? 10 : 0;
            if (need && wgs * need <= budget) {
                w = need;
                break;
            }
        }
    }
    if (mr == 16 && M <= 16 && S <= 24) w = 4;
    const int fw = tune.gemv_waves;
    if (fw)
        w = (fw == 16 && (mr != 16 || M > 16)) || (fw == 5 && mr != 1) ||
                    (fw == 10 && mr != 1 && mr != 4 && mr != 8)
                ? 8
                : fw;
    int uu = 1;
    if (mr == 1 && !plain1 && (S + w - 1) / w == 2) uu = 2;
    if (long_k && mr == 4) uu = 2;
    const int fu = tune.gemv_u;
    if (fu) uu = fu;
    if (w == 16) uu = 1;    // two-step batches would not fit 128 VGPRs
    *ks = k;
    *waves = w;
    *u = uu;
    if (groups) *groups = cg;
}

hipError_t launch_fp8_gemv(const Fp8Operands& op, bool fused, hipStream_t stream,
                           const LaunchTiming& t, const char** name, const uint16_t* gamma,
                           float eps)
{
    GemvArgs a{op, fused, gamma, eps};
    int ks, waves, u, cg = 1;
    gemv_shape(op.M, op.N, op.K, op.tune, &ks, &waves, &u, gamma != nullptr,
               fused && !gamma ? &cg : nullptr);
    const int mr = gemv_rows(op.M);
    if (op.M == 1) *name = gamma ? "fp8_gemv_rmsnorm_m1" : fused ? "fp8_gemv_fused_m1" : "fp8_gemv_m1";
    else if (op.M <= 16) *name = fused ? "fp8_gemv_fused_m16" : "fp8_gemv_m16";
    else *name = fused ? "fp8_gemv_fused_m32" : "fp8_gemv_m32";
    if (cg == 2) {
        switch (waves) {
        case 5: return u == 2 ? launch_groups2<5, 2>(a, stream, t) : launch_groups2<5, 1>(a, stream, t);
        case 8: return u == 2 ? launch_groups2<8, 2>(a, stream, t) : launch_groups2<8, 1>(a, stream, t);
        case 10: return u == 2 ? launch_groups2<10, 2>(a, stream, t) : launch_groups2<10, 1>(a, stream, t);
        default: return u == 2 ? launch_groups2<4, 2>(a, stream, t) : launch_groups2<4, 1>(a, stream, t);
        }
    }
    if ((mr == 4 || mr == 8) && waves == 10) {
        if (mr == 4)
            return u == 2 ? launch_mr<10, 4, 1, 2>(a, fused, ks, stream, t)
                          : launch_mr<10, 4, 1, 1>(a, fused, ks, stream, t);
        return u == 2 ? launch_mr<10, 8, 1, 2>(a, fused, ks, stream, t)
                      : launch_mr<10, 8, 1, 1>(a, fused, ks, stream, t);
    }
    if (mr == 1 && (waves == 5 || waves == 10)) {
        if (waves == 5)
            return u == 2 ? launch_mr<5, 1, 1, 2>(a, fused, ks, stream, t)
                          : launch_mr<5, 1, 1, 1>(a, fused, ks, stream, t);
        return u == 2 ? launch_mr<10, 1, 1, 2>(a, fused, ks, stream, t)
                      : launch_mr<10, 1, 1, 1>(a, fused, ks, stream, t);
    }
    switch (waves) {
    case 16: return launch_wu<16, 1>(a, fused, ks, mr, stream, t);
    case 8:
        return u == 2 ? launch_wu<8, 2>(a, fused, ks, mr, stream, t)
                      : launch_wu<8, 1>(a, fused, ks, mr, stream, t);
    default:
        return u == 2 ? launch_wu<4, 2>(a, fused, ks, mr, stream, t)
                      : launch_wu<4, 1>(a, fused, ks, mr, stream, t);
    }
}

}  // namespace heph
