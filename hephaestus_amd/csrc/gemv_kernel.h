// gemv_kernel.h - the chunk-slot GEMV kernel: W8A8 FP8 linear for 1 <= M <= 32
// (decode GEMV and batched decode), included by gemv.hip and gemv_swiglu.hip.
//
// Replaces the reference's decode GEMV and small-M kernels
// (src/hephaestus/wmma_gfx12.mojo:650-744 and :906-1019, reached through
// gemv_fp8 / linear_fp8, src/hephaestus/kernels.mojo:372-470). Those give
// one 32-lane wave a 16-column tile over all of K.
//
// At M <= 32 the work is bound by streaming the E4M3 weights from HBM, and
// with M rows only M of the 16 rows of a 16x16 MFMA tile carry data. This
// kernel fills the other rows with further K-chunks instead ("chunk
// slots"): with KS slots of MR rows each (KS * MR <= 16; MR = M rounded up
// to a power of two), A row t*MR + m holds row m of the activations at the
// chunk of slot t, and MFMA column c holds output column n0 + c % TW
// (TW = 16 / KS) at K-chunk step*KS + c / TW. The wanted products of
// column c are then C[(c / TW)*MR + m][c]; every other C element is unused.
// One v_mfma_f32_16x16x128_f8f6f4 covers KS chunks of TW columns, so a
// workgroup owns only TW output columns and the grid has N*KS/16
// workgroups: enough to cover the 256 CUs even at N = 2560 for M <= 4,
// with no reduction across workgroups. M = 17..32 runs two 16-row tiles
// with one slot.
//   * workgroup = TW output columns; its WAVES waves split the KC/KS steps
//     into contiguous runs; loads go out in batches of U steps, two batches
//     in flight, each lane issuing two 16-byte weight loads per step;
//   * fused mode (1x128 groups) quantizes x inside the kernel:
//     64/(KS*MR) lanes share an A row's 128-element group, its max (on the
//     bf16 magnitude bits, two per packed 16-bit max, NaN skipped) is
//     reduced with DPP and lane swaps, the scale is the reference's
//     (amax/448, 1/s, both rounded to nearest even) computed without a
//     division (group_scale in heph_device.h), and the codes reach
//     the MFMA A layout through a per-wave LDS tile. Workgroup 0 also
//     writes q/s to the workspace so later SKIP_QUANT calls can reuse them;
//   * each lane rescales its candidate C elements by sa[row, chunk] *
//     sw[block, chunk] in registers, the row scales passed between lanes
//     by ds_bpermute from the lane that quantized (or loaded) that A row;
//     per-channel/per-token scales (the
//     reference's own granularity) accumulate unscaled and apply the
//     reference association at the end: acc*(sa*sw) at M = 1
//     (wmma_gfx12.mojo:711-712), (acc*sa)*sw otherwise (:973, :848);
//   * after one workgroup barrier wave 0 sums the waves' slot partials in
//     a fixed order (deterministic) and stores bf16 or f32, optionally
//     adding the residual first (wmma_gfx12.mojo:712-715).
#pragma once

#include <type_traits>

#include "heph_kernels.h"

namespace heph {

struct GemvArgs {
    Fp8Operands op;
    bool write_ws;
    // RMSNorm prologue (M = 1, fused): x is the un-normalized row, each
    // activation becomes bf16(gamma * bf16(x * r)) before its quantization
    const uint16_t* gamma;
    float eps;
};

enum GemvScale { kGemvBlock = 0, kGemvChannel = 1, kGemvConst = 2 };

namespace {

// E consecutive bf16 activations (E = 2, 4, 8, 16 or 32) as E/2 dwords.
template <int E>
struct XVec {
    uint32_t d[E / 2];
};

template <int E>
__device__ __forceinline__ XVec<E> load_xvec(const uint16_t* p)
{
    XVec<E> v;
    if constexpr (E == 2) {
        v.d[0] = *reinterpret_cast<const uint32_t*>(p);
    } else if constexpr (E == 4) {
        const uint2 t = *reinterpret_cast<const uint2*>(p);
        v.d[0] = t.x;
        v.d[1] = t.y;
    } else {
#pragma unroll
        for (int h = 0; h < E / 8; ++h) {
            const uint4 t = ldg16u(p + h * 8);
            v.d[4 * h] = t.x;
            v.d[4 * h + 1] = t.y;
            v.d[4 * h + 2] = t.z;
            v.d[4 * h + 3] = t.w;
        }
    }
    return v;
}

template <int E>
__device__ __forceinline__ void store_codes(uint8_t* p, const uint32_t* cd)
{
    if constexpr (E == 2) *reinterpret_cast<uint16_t*>(p) = (uint16_t)cd[0];
    else if constexpr (E == 4) *reinterpret_cast<uint32_t*>(p) = cd[0];
    else if constexpr (E == 8) *reinterpret_cast<uint2*>(p) = make_uint2(cd[0], cd[1]);
    else {
#pragma unroll
        for (int h = 0; h < E / 16; ++h)
            reinterpret_cast<uint4*>(p)[h] =
                make_uint4(cd[4 * h], cd[4 * h + 1], cd[4 * h + 2], cd[4 * h + 3]);
    }
}

// Max over each aligned run of LPR lanes, unsigned integers, left in every
// lane of the run: DPP within each 16-lane row, then gfx950's lane swaps
// (v_permlane16_swap pairs rows 0-1 and 2-3, v_permlane32_swap the two
// halves), which stay in the VALU instead of going through LDS.
template <int LPR>
__device__ __forceinline__ uint32_t lanes_max_u(uint32_t m)
{
    auto dpp = [](uint32_t x, auto ctrl) {
        return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, decltype(ctrl)::value, 0xf, 0xf, false);
    };
    m = max(m, dpp(m, std::integral_constant<int, 0xB1>{}));
    m = max(m, dpp(m, std::integral_constant<int, 0x4E>{}));
    if constexpr (LPR >= 8) m = max(m, dpp(m, std::integral_constant<int, 0x141>{}));
    if constexpr (LPR >= 16) m = max(m, dpp(m, std::integral_constant<int, 0x140>{}));
    if constexpr (LPR >= 32) {
        const auto r = __builtin_amdgcn_permlane16_swap(m, m, false, false);
        m = max((uint32_t)r[0], (uint32_t)r[1]);
    }
    if constexpr (LPR == 64) {
        const auto r = __builtin_amdgcn_permlane32_swap(m, m, false, false);
        m = max((uint32_t)r[0], (uint32_t)r[1]);
    }
    return m;
}

// Four floats -> four E4M3FN codes (byte i = code of value i), RNE. The
// first conversion writes the low half of a register whose other half the
// second one overwrites, so its previous contents do not matter.
__device__ __forceinline__ uint32_t pack4_any(float a, float b, float c, float d, uint32_t junk)
{
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int)junk, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    return (uint32_t)w;
}

__device__ __forceinline__ float pick(const f32x4& p, int e)
{
    return e == 0 ? p[0] : e == 1 ? p[1] : e == 2 ? p[2] : p[3];
}

}  // namespace

// GLU: SwiGLU epilogue (M = 1): the weight rows are a gate half [0, N/2)
// and an up half [N/2, N); of a workgroup's TW columns the first TW/2 are
// gate columns j = (TW/2) b .. and the rest the up columns N/2 + j, and it
// stores act[j] = bf16(bf16(g / (1 + exp(-g))) * up) of their bf16-rounded
// values: with the launch shape of the plain kernel, the GEMV output and
// silu_mul of the two-launch form bit for bit.
//
// CG: column groups per workgroup (1 or 2). With 2, every step of a wave
// contracts the same A tile (the quantized activations of its chunks) with
// the weights of two groups of TW columns, so a workgroup owns 2 TW columns
// and reads the activations once for both: the activation bytes a workgroup
// reads per weight byte halve, and so do the workgroups.
template <int WAVES, int KS, int MR, int MT, int U, bool FUSED, int SM, bool NORM = false,
          bool GLU = false, int CG = 1>
__global__ __launch_bounds__(WAVES * 64) void fp8_gemv_kernel(GemvArgs args)
{
    static_assert(!NORM || (FUSED && MR == 1 && MT == 1 && WAVES >= 4),
                  "RMSNorm prologue: fused M = 1 with at least 256 threads");
    static_assert(!GLU || (FUSED && MR == 1 && MT == 1 && KS <= 8),
                  "SwiGLU epilogue: fused M = 1, at least two columns per workgroup");
    static_assert(KS == 1 || KS == 2 || KS == 4 || KS == 8, "chunk slots");
    static_assert(MR == 1 || MR == 2 || MR == 4 || MR == 8 || MR == 16, "rows per slot");
    static_assert(KS * MR <= 16, "slots x rows must fit the 16 MFMA rows");
    static_assert(MT == 1 || (MT == 2 && MR == 16 && KS == 1), "two row tiles: one slot of 16");
    static_assert(!(FUSED && SM == kGemvConst), "fused quantization: 1x128 groups");
    static_assert(CG == 1 || (CG == 2 && MT == 1 && !GLU), "two column groups: one row tile");
    constexpr int R = KS * MR;           // A rows in use
    constexpr int TW = 16 / KS;          // output columns per workgroup
    constexpr int LPR = 64 / R;          // quantizing lanes per A row
    constexpr int E = 128 / LPR;         // activations per quantizing lane
    constexpr int NE = MR < 4 ? MR : 4;  // candidate C elements per lane and tile
    const Fp8Operands& op = args.op;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int t = r16 / TW;              // chunk slot of this lane's column
    // This lane's candidate C elements are rows rho + i (i < NE) of the
    // tile, element e0 + i of its MFMA result: the rows of slot t when
    // MR < 4 (they sit in lane group t*MR/4), else rows 4g .. 4g+3.
    const int rho = MR < 4 ? t * MR : 4 * g;
    const int e0 = MR < 4 ? rho & 3 : 0;
    const int M = op.M, K = op.K;
    const int KC = K >> 7;
    const int S = (KC + KS - 1) / KS;    // steps of KS chunks
    const int n0 = blockIdx.x * (TW * CG);
    const int per = (S + WAVES - 1) / WAVES;
    const int sb = min(S, wave * per);
    const int se = min(S, sb + per);
    // fused: this lane quantizes piece qpiece of A row qrow (slot tq, row mq)
    const int qrow = lane / LPR, qpiece = lane % LPR;
    const int tq = qrow / MR, mq = qrow % MR;
    // separate quantization: this lane loads A row r16 (slot ta, row ma)
    const int ta = r16 / MR, ma = r16 % MR;

    __shared__ float red[WAVES][CG * MT * NE][64];
    __shared__ __attribute__((aligned(16))) uint8_t qlds[FUSED ? WAVES : 1][FUSED ? U : 1]
                                                        [FUSED ? MT : 1][R * kChunk];
    // NORM: the row and gamma (bf16)
    __shared__ __attribute__((aligned(16))) uint16_t nrow[NORM ? kNormMaxK : 1];
    __shared__ __attribute__((aligned(16))) uint16_t ngam[NORM ? kNormMaxK : 1];

    // GLU: column c < TW/2 is gate row (TW/2) b + c, the others the up rows
    // N/2 + (TW/2) b + c - TW/2
    constexpr int HALF = TW / 2;
    const int cw = r16 % TW;
    const int n = !GLU ? n0 + cw
                : cw < HALF ? HALF * (int)blockIdx.x + cw
                            : op.N / 2 + HALF * (int)blockIdx.x + cw - HALF;
    // column group h reads the rows h*TW further on
    const uint8_t* wrow = op.w + (size_t)n * K + g * 16;
    // the 128-row block of the workgroup's columns (GLU: of the lane's
    // half, so a per-lane load); with two groups both lie in it (2 TW
    // divides 128)
    const float* swb = op.sw + (size_t)((GLU ? n : n0) >> 7) * op.sw_ld;
    float swc[CG];
#pragma unroll
    for (int h = 0; h < CG; ++h) swc[h] = SM == kGemvBlock ? 0.0f : op.sw[n + h * TW];

    struct Batch {
        i32x4 blo[U][CG], bhi[U][CG];
        i32x4 alo[FUSED ? 1 : U][MT], ahi[FUSED ? 1 : U][MT];
        XVec<E> xv[FUSED ? U : 1][MT];
        float sw[U];
        // MR = 1: the scale of this lane's candidate row; else the scale of
        // its own A row r16, passed to the candidate rows by ds_bpermute
        float sa[FUSED ? 1 : U][MT];
    };

    // Loads are unconditional and clamped, so a batch is one straight run
    // of memory instructions: a step past se re-reads step se-1 (never
    // consumed), a chunk past KC re-reads chunk KC-1 and a row past M
    // re-reads row M-1, both with zero activations. Activation loads go
    // first so their quantization can run while the weights are in flight.
    auto issue = [&](Batch& b, int s) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int st = min(s + u, se - 1);
            if constexpr (NORM) {
                // the row and gamma come from LDS at quantization time
            } else if constexpr (FUSED) {
                const int jx = st * KS + tq;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int row = mt * 16 + mq;
                    const XVec<E> v =
                        load_xvec<E>(op.x + (size_t)min(row, M - 1) * K +
                                     (size_t)min(jx, KC - 1) * kChunk + qpiece * E);
                    const bool live = jx < KC && row < M;
#pragma unroll
                    for (int d = 0; d < E / 2; ++d) b.xv[u][mt].d[d] = live ? v.d[d] : 0u;
                }
            } else {
                // Only the R lanes per column group that hold a real A row
                // (r16 < R) load it; the others keep zeros and issue no
                // load, so codes from the workspace cost R/16 of a full
                // 16-row A tile per step.
                const int ja = st * KS + ta;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int row = mt * 16 + ma;
                    const uint8_t* p = op.q + (size_t)min(row, M - 1) * K +
                                       (size_t)min(ja, KC - 1) * kChunk + g * 16;
                    i32x4 lo = i32x4{0, 0, 0, 0}, hi = i32x4{0, 0, 0, 0};
                    if (r16 < R) {
                        lo = ldg16(p);
                        hi = ldg16(p + 64);
                    }
                    const bool live = r16 < R && row < M && ja < KC;
                    b.alo[u][mt] = live ? lo : i32x4{0, 0, 0, 0};
                    b.ahi[u][mt] = live ? hi : i32x4{0, 0, 0, 0};
                    if constexpr (SM != kGemvConst) {
                        const int tok = MR == 1 ? 0 : min(row, M - 1);
                        const int j = min(st * KS + (MR == 1 ? t : ta), KC - 1);
                        b.sa[u][mt] = op.s[(size_t)tok * op.s_ld + (size_t)j * op.s_step];
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int st = min(s + u, se - 1);
            const int jb = min(st * KS + t, KC - 1);
            const uint8_t* p = wrow + (size_t)jb * kChunk;
#pragma unroll
            for (int h = 0; h < CG; ++h) {
                b.blo[u][h] = ldg16(p + (size_t)h * TW * K);
                b.bhi[u][h] = ldg16(p + (size_t)h * TW * K + 64);
            }
            if constexpr (SM == kGemvBlock) b.sw[u] = swb[jb];
        }
    };

    float acc[CG][MT][NE];
#pragma unroll
    for (int h = 0; h < CG; ++h)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < NE; ++i) acc[h][mt][i] = 0.0f;
    float rn = 1.0f;    // RMSNorm factor (NORM)

    auto contract = [&](int h, int mt, const i32x4& alo, const i32x4& ahi, const i32x4& blo,
                        const i32x4& bhi, const float* scl) {
        const f32x4 p = mfma_e4m3(join(alo, ahi), join(blo, bhi), f32x4{0, 0, 0, 0});
#pragma unroll
        for (int i = 0; i < NE; ++i) {
            const float v = MR >= 4 ? p[i] : pick(p, e0 + i);
            if constexpr (SM == kGemvConst) acc[h][mt][i] += v;
            else acc[h][mt][i] += v * scl[i];
        }
    };

    auto consume = [&](Batch& b, int s) {
        if constexpr (FUSED) {
            // 1. quantize the batch's chunks into this wave's LDS tiles
            float sc[U][MT];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (s + u >= se) break;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    XVec<E>& xv = b.xv[u][mt];
                    if constexpr (NORM) {
                        // the RMSNorm output, as the standalone kernel
                        // rounds it: bf16(gamma * bf16(x * r)), from the row
                        // and gamma the prologue left in LDS (zero past K)
                        const int jx = (s + u) * KS + tq;
                        const int k0 = jx * kChunk + qpiece * E;
                        const bool live = jx < KC;
#pragma unroll
                        for (int d = 0; d < E / 2; ++d) {
                            const int k = k0 + 2 * d;
                            const uint32_t xd =
                                live ? (uint32_t)nrow[k] | ((uint32_t)nrow[k + 1] << 16) : 0u;
                            const uint32_t gd =
                                live ? (uint32_t)ngam[k] | ((uint32_t)ngam[k + 1] << 16) : 0u;
                            const float yl = bf16lo((uint32_t)f32_to_bf16(bf16lo(xd) * rn));
                            const float yh = bf16lo((uint32_t)f32_to_bf16(bf16hi(xd) * rn));
                            const uint32_t lo = f32_to_bf16(bf16lo(gd) * yl);
                            const uint32_t hi = f32_to_bf16(bf16hi(gd) * yh);
                            xv.d[d] = lo | (hi << 16);
                        }
                    }
                    // a lane holding a NaN takes the NaN-skipping max of its
                    // own elements before the cross-lane max (rare; a
                    // divergent branch that no lane takes costs two scalar
                    // instructions)
                    uint32_t mb = absmax_bits(xv.d);
                    if (mb > 0x7F80u) mb = absmax_bits_skip_nan(xv.d);
                    mb = lanes_max_u<LPR>(mb);
                    float inv;
                    group_scale(bf16_bits_f32(mb), sc[u][mt], inv);
                    uint32_t cd[(E + 3) / 4];
                    if constexpr (E == 2) {
                        cd[0] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(
                            bf16lo(xv.d[0]) * inv, bf16hi(xv.d[0]) * inv, 0, false);
                    } else {
#pragma unroll
                        for (int d = 0; d < E / 4; ++d) {
                            const uint32_t a0 = xv.d[2 * d], a1 = xv.d[2 * d + 1];
                            cd[d] = pack4_any(bf16lo(a0) * inv, bf16hi(a0) * inv,
                                              bf16lo(a1) * inv, bf16hi(a1) * inv, a0);
                        }
                    }
                    store_codes<E>(qlds[wave][u][mt] + qrow * kChunk + qpiece * E, cd);
                    const int jx = (s + u) * KS + tq;
                    const int row = mt * 16 + mq;
                    if (args.write_ws && blockIdx.x == 0 && jx < KC && row < M) {
                        store_codes<E>(op.q + (size_t)row * K + (size_t)jx * kChunk + qpiece * E,
                                       cd);
                        if (qpiece == 0) op.s[(size_t)row * op.s_ld + jx] = sc[u][mt];
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();
            // 2. contract: A rows 0..R-1 from LDS, each candidate row's scale
            //    from the lanes that quantized it
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (s + u >= se) break;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const uint8_t* tile = qlds[wave][u][mt];
                    i32x4 lo = i32x4{0, 0, 0, 0}, hi = i32x4{0, 0, 0, 0};
                    if (r16 < R) {
                        lo = *reinterpret_cast<const i32x4*>(tile + r16 * kChunk + g * 16);
                        hi = *reinterpret_cast<const i32x4*>(tile + r16 * kChunk + 64 + g * 16);
                    }
                    float sa[NE];
#pragma unroll
                    for (int i = 0; i < NE; ++i)
                        sa[i] = R == 1 ? sc[u][mt]
                                       : __int_as_float(__builtin_amdgcn_ds_bpermute(
                                             (rho + i) * LPR * 4, __float_as_int(sc[u][mt])));
#pragma unroll
                    for (int h = 0; h < CG; ++h) {
                        const float sw = SM == kGemvBlock ? b.sw[u] : swc[h];
                        float scl[NE];
#pragma unroll
                        for (int i = 0; i < NE; ++i) scl[i] = sa[i] * sw;
                        contract(h, mt, lo, hi, b.blo[u][h], b.bhi[u][h], scl);
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (s + u >= se) break;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    float sa[NE];
#pragma unroll
                    for (int i = 0; i < NE; ++i) {
                        sa[i] = 0.0f;
                        if constexpr (SM != kGemvConst)
                            sa[i] = MR == 1 ? b.sa[u][mt]
                                            : __int_as_float(__builtin_amdgcn_ds_bpermute(
                                                  (rho + i) * 4, __float_as_int(b.sa[u][mt])));
                    }
#pragma unroll
                    for (int h = 0; h < CG; ++h) {
                        const float sw = SM == kGemvBlock ? b.sw[u] : swc[h];
                        float scl[NE];
#pragma unroll
                        for (int i = 0; i < NE; ++i) scl[i] = sa[i] * sw;
                        contract(h, mt, b.alo[u][mt], b.ahi[u][mt], b.blo[u][h], b.bhi[u][h],
                                 scl);
                    }
                }
            }
        }
    };

    // Two batches in flight, then each consumed batch is replaced by the
    // next U steps. With NORM both go out before the norm's prologue (its
    // loads and barriers would otherwise leave one batch's latency exposed:
    // MI355X, fused-norm o_proj 9.45 -> 8.25 us, gate_up 16.3 -> 14.5);
    // without, one after the other.
    Batch b0, b1;
    // RMSNorm (NORM): the row and gamma are loaded in 16-byte pieces spread
    // over all threads before the weight batches (a wave's loads return in
    // order, and the norm should not wait behind the weights), stored to LDS
    // once per workgroup, and then threads t < 256 sum the squares of
    // elements t, t + 256, ... by fma from LDS, the standalone kernel's
    // order; the quantizing lanes take their slices from LDS too.
    // K <= kNormMaxK.
    constexpr int kRowPieces = NORM ? (kNormMaxK / 8 + WAVES * 64 - 1) / (WAVES * 64) : 1;
    uint4 xq[kRowPieces], gq[kRowPieces];
    if constexpr (NORM) {
#pragma unroll
        for (int p = 0; p < kRowPieces; ++p) {
            const int pc = (int)threadIdx.x + p * WAVES * 64;
            if (pc < K / 8) {
                xq[p] = ldg16u(op.x + 8 * pc);
                gq[p] = ldg16u(args.gamma + 8 * pc);
            }
        }
    }
    if (sb < se) issue(b0, sb);
    if constexpr (NORM) {
        if (sb + U < se) issue(b1, sb + U);
#pragma unroll
        for (int p = 0; p < kRowPieces; ++p) {
            const int pc = (int)threadIdx.x + p * WAVES * 64;
            if (pc < K / 8) {
                *reinterpret_cast<uint4*>(nrow + 8 * pc) = xq[p];
                *reinterpret_cast<uint4*>(ngam + 8 * pc) = gq[p];
            }
        }
        __syncthreads();
        // the sum of squares and the fold of the 256 sums, as fold256_wave0
        __shared__ float nred[256];
        float ss = 0.0f;
        if (threadIdx.x < 256) {
            // unrolled so that a thread's LDS reads go out together (the
            // sums stay in order; MI355X decode step: -27 us per token)
#pragma unroll 8
            for (int i = threadIdx.x; i < K; i += 256) {
                const float v = bf16lo((uint32_t)nrow[i]);
                ss = __builtin_fmaf(v, v, ss);
            }
        }
        rn = rms_inv(fold256_every_wave(ss, nred), K, args.eps);
    } else {
        // no barrier before the loop: the waves start their batches as they
        // are dispatched (a workgroup barrier here, with the first batch in
        // flight, cost 1-2 % on every config shape on MI355X)
        if (sb + U < se) issue(b1, sb + U);
    }
    for (int s = sb; s < se; s += 2 * U) {
        consume(b0, s);
        if (s + 2 * U < se) issue(b0, s + 2 * U);
        if (s + U >= se) break;
        consume(b1, s + U);
        if (s + 3 * U < se) issue(b1, s + 3 * U);
    }

    // ---- wave 0 sums the partials in a fixed order after one barrier ----
#pragma unroll
    for (int h = 0; h < CG; ++h)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < NE; ++i) red[wave][(h * MT + mt) * NE + i][lane] = acc[h][mt][i];
    __syncthreads();
    if (wave != 0) return;

    if constexpr (GLU) {
        // lane c < TW sums column c over the waves and slots in the plain
        // epilogue's order; lanes c < TW/2 then take the up value of lane
        // c + TW/2
        const int c2 = lane % TW;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w)
#pragma unroll
            for (int ts = 0; ts < KS; ++ts) v += red[w][0][(ts >> 2) * 16 + ts * TW + c2];
        const uint32_t h = f32_to_bf16(v);
        const uint32_t up = (uint32_t)__shfl((int)h, lane % HALF + HALF, 64);
        if (lane < HALF)
            static_cast<uint16_t*>(op.c)[HALF * blockIdx.x + lane] = (uint16_t)swiglu_bits(h, up);
        return;
    }

    // output (token mt*16 + m, column n0 + h*TW + c2) = sum over waves w and
    // slots ts of C row ts*MR + m, column ts*TW + c2 of group h
    constexpr int OUTS = CG * MT * MR * TW;
    for (int o = lane; o < OUTS; o += 64) {
        const int c2 = o % TW, m = (o / TW) % MR, mt = (o / (TW * MR)) % MT;
        const int h = o / (TW * MR * MT);
        const int tok = mt * 16 + m;
        if (tok >= M) continue;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w)
#pragma unroll
            for (int ts = 0; ts < KS; ++ts) {
                const int rr = ts * MR + m;
                v += red[w][(h * MT + mt) * NE + (MR >= 4 ? (rr & 3) : m)]
                         [(rr >> 2) * 16 + ts * TW + c2];
            }
        const int col = n0 + h * TW + c2;
        if constexpr (SM == kGemvConst) {
            const float sa = op.s[(size_t)tok * op.s_ld], sw = op.sw[col];
            v = M == 1 ? v * (sa * sw) : (v * sa) * sw;
        }
        const size_t oi = (size_t)tok * op.N + col;
        if (op.c_f32) {
            float* c = static_cast<float*>(op.c);
            c[oi] = op.residual ? v + c[oi] : v;
        } else {
            uint16_t* c = static_cast<uint16_t*>(op.c);
            if (op.residual) v += __uint_as_float((uint32_t)c[oi] << 16);
            c[oi] = f32_to_bf16(v);
        }
    }
}

}  // namespace heph
