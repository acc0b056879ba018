// skinny.hip - W8A8 FP8 linear for M <= 32 (decode GEMV and batched decode).
//
// Replaces the reference's decode GEMV and small-M kernels
// (src/hephaestus/wmma_gfx12.mojo:650-744 and :906-1019). Those give one
// 32-lane wave a 16x16 (or 16x64) tile over all of K with 16-wide K steps.
// At M <= 32 the work is bound by streaming the E4M3 weights from HBM, so
// this kernel is built around the weight stream instead:
//   * workgroup = 16*NT output columns; its WAVES waves split K into
//     contiguous runs of 128-wide chunks, so even N = 2560 puts thousands
//     of waves in flight;
//   * each lane issues two 16-byte loads per 16-column tile per chunk
//     (16 rows x 64 contiguous bytes per instruction); loads are issued in
//     batches of U chunks, two batches in flight (software pipelined);
//   * one v_mfma_f32_16x16x128_f8f6f4 per chunk and tile contracts all M
//     rows at once (rows >= M are zero);
//   * the chunk partial is rescaled in registers by sa[m, chunk] * sw[block]
//     (the 1x128 activation groups and 128x128 weight blocks line up with
//     the chunk), then the waves' partials are summed through LDS;
//   * with the reference's own granularity (per-channel weight scale,
//     per-token activation scale; both constant over K) the MFMA sums are
//     accumulated unscaled and the epilogue applies the reference's
//     association: acc*(sa*sw) at M = 1 (wmma_gfx12.mojo:711-712),
//     (acc*sa)*sw otherwise (:973, :848);
//   * fused mode (group 128, M <= 4) quantizes x inside the kernel: lane l
//     quantizes 8 elements of row l/16 (one 16-byte load), the row's
//     128-element group max (on bf16 magnitude bits, NaN skipped) is
//     reduced across its 16 lanes with DPP, and
//     the codes reach the MFMA operand layout through a per-wave LDS slot.
//     Workgroup 0 also writes q/s so later SKIP_QUANT calls can reuse them.
#include <atomic>

#include "heph_kernels.h"

namespace heph {

struct SkinnyArgs {
    Fp8Operands op;
    bool write_ws;
};

// Scale modes: kBlock (128x128 weight blocks), kChannel (per-channel weight
// scale, per-chunk activation scale), kConst (per-channel weight and
// per-token activation scale: nothing varies along K).
enum ScaleMode { kBlock = 0, kChannel = 1, kConst = 2 };

namespace {

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x)
{
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, CTRL, 0xf, 0xf, false);
}

// max over the 16 lanes of each DPP row (lanes 16r .. 16r+15):
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror.
__device__ __forceinline__ uint32_t row16_max_u(uint32_t v)
{
    v = max(v, dpp_u<0xB1>(v));
    v = max(v, dpp_u<0x4E>(v));
    v = max(v, dpp_u<0x141>(v));
    v = max(v, dpp_u<0x140>(v));
    return v;
}

}  // namespace

// XM > 0: fused quantization of XM rows (1, 2 or 4; M <= XM). Lane l
// quantizes E = 2*XM elements of row l / (64/XM): for M = 1 the whole wave
// shares one 128-element group (2 elements a lane).
template <int XM>
struct XLayout {
    static constexpr int LPR = XM ? 64 / XM : 64;   // lanes per row
    static constexpr int E = 128 / LPR;              // elements per lane
};

template <int E>
__device__ __forceinline__ uint4 load_x(const uint16_t* p)
{
    if constexpr (E == 2) return make_uint4(*reinterpret_cast<const uint32_t*>(p), 0, 0, 0);
    else if constexpr (E == 4) {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        return make_uint4(v.x, v.y, 0, 0);
    } else return ldg16u(p);
}

template <int WAVES, int MT, int NT, int U, int XM, int SM>
__global__ __launch_bounds__(WAVES * 64) void fp8_skinny_kernel(SkinnyArgs args)
{
    // SMALL: M <= 4 with one 16-row tile: the live output rows are 0..3 of
    // lane group 0, so activation scales are wave-uniform.
    constexpr bool SMALL = MT == 1 && NT == 1;
    constexpr bool FUSED = XM > 0;
    static_assert(!FUSED || SMALL, "fused quantization serves M <= 4");
    constexpr int LPR = XLayout<XM>::LPR, E = XLayout<XM>::E;
    constexpr int TILES = MT * NT;
    const Fp8Operands& op = args.op;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15;
    const int slice = lane >> 4;
    const int M = op.M, N = op.N, K = op.K;
    const int KC = K >> 7;
    const int n0 = blockIdx.x * (16 * NT);
    const int per = (KC + WAVES - 1) / WAVES;
    const int kb = min(KC, wave * per);
    const int ke = min(KC, kb + per);

    __shared__ float red[WAVES][TILES * 4][64];
    __shared__ int arrive;
    __shared__ __attribute__((aligned(16))) uint8_t qlds[FUSED ? WAVES : 1][FUSED ? U : 1][512];
    if (threadIdx.x == 0) arrive = 0;
    __syncthreads();

    const uint8_t* wp[NT];
    float swc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int n = min(n0 + nt * 16, N - 16) + r16;
        wp[nt] = op.w + (size_t)n * K + slice * 16;
        swc[nt] = SM == kChannel ? op.sw[n] : 0.0f;
    }
    const float* swb = op.sw + (size_t)(n0 >> 7) * op.sw_ld;
    const int qrow = lane / LPR, qpiece = lane % LPR;

    f32x4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0, 0, 0, 0};

    struct Batch {
        i32x4 blo[U][NT], bhi[U][NT];
        i32x4 alo[FUSED ? 1 : U][MT], ahi[FUSED ? 1 : U][MT];
        uint4 xv[FUSED ? U : 1];
        float sw[U];
        float sa[U][MT][4];
    };

    // Loads are unconditional, so a batch is one straight run of memory
    // instructions and every wait covers exactly what the next chunk needs:
    // a tail chunk past ke re-reads chunk ke-1 (an L2 hit, never consumed),
    // rows >= M read row 0 and are zeroed, columns past N read the last
    // tile and are never stored. Activation loads go first so their
    // quantization can run while the weights are still in flight.
    auto issue = [&](Batch& b, int kc) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = min(kc + u, ke - 1);
            if constexpr (FUSED) {
                const uint4 v = load_x<E>(op.x + (size_t)(qrow < M ? qrow : 0) * K +
                                          j * kChunk + qpiece * E);
                b.xv[u] = qrow < M ? v : make_uint4(0, 0, 0, 0);
            } else {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int row = mt * 16 + r16;
                    const uint8_t* p =
                        op.q + (size_t)(row < M ? row : 0) * K + j * kChunk + slice * 16;
                    const i32x4 lo = ldg16(p), hi = ldg16(p + 64);
                    b.alo[u][mt] = row < M ? lo : i32x4{0, 0, 0, 0};
                    b.ahi[u][mt] = row < M ? hi : i32x4{0, 0, 0, 0};
                    if constexpr (SM != kConst) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            // SMALL: rows 0..3 for every lane (uniform loads).
                            const int orow = SMALL ? i : mt * 16 + slice * 4 + i;
                            const float v =
                                op.s[(size_t)(orow < M ? orow : 0) * op.s_ld + j * op.s_step];
                            b.sa[u][mt][i] = orow < M ? v : 0.0f;
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = min(kc + u, ke - 1);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const uint8_t* p = wp[nt] + (size_t)j * kChunk;
                b.blo[u][nt] = ldg16(p);
                b.bhi[u][nt] = ldg16(p + 64);
            }
            if constexpr (SM == kBlock) b.sw[u] = swb[j];
        }
    };

    auto consume = [&](Batch& b, int kc) {
        if constexpr (FUSED) {
            // 1. quantize every chunk of the batch into its LDS slot
            float scl[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int j = kc + u;
                if (j >= ke) break;
                // group amax on the bf16 magnitude bits (NaN skipped)
                auto group_max = [&](uint32_t v) {
                    v = row16_max_u(v);
                    if constexpr (LPR == 32) v = max(v, shfl_xor_u(v, 16));
                    if constexpr (LPR == 64) {
                        const uint32_t m0 = __builtin_amdgcn_readlane((int)v, 0);
                        const uint32_t m1 = __builtin_amdgcn_readlane((int)v, 16);
                        const uint32_t m2 = __builtin_amdgcn_readlane((int)v, 32);
                        const uint32_t m3 = __builtin_amdgcn_readlane((int)v, 48);
                        v = max(max(m0, m1), max(m2, m3));
                    }
                    return v;
                };
                uint32_t mb = group_max(absmax_bits8(b.xv[u]));
                if (__builtin_amdgcn_ballot_w64(mb > 0x7F80u) != 0)
                    mb = group_max(absmax_bits8_skip_nan(b.xv[u]));
                float sc, inv;
                group_scale(bf16_bits_f32(mb), sc, inv);
                scl[u] = sc;
                const uint2 c = quant8(b.xv[u], inv);
                uint8_t* slot = qlds[wave][u] + qrow * 128 + qpiece * E;
                uint8_t* qg = op.q + (size_t)qrow * K + j * kChunk + qpiece * E;
                const bool ws = args.write_ws && blockIdx.x == 0 && qrow < M;
                if constexpr (E == 2) {
                    *reinterpret_cast<uint16_t*>(slot) = (uint16_t)c.x;
                    if (ws) *reinterpret_cast<uint16_t*>(qg) = (uint16_t)c.x;
                } else if constexpr (E == 4) {
                    *reinterpret_cast<uint32_t*>(slot) = c.x;
                    if (ws) *reinterpret_cast<uint32_t*>(qg) = c.x;
                } else {
                    *reinterpret_cast<uint2*>(slot) = c;
                    if (ws) *reinterpret_cast<uint2*>(qg) = c;
                }
                if (ws && qpiece == 0) op.s[(size_t)qrow * KC + j] = sc;
            }
            __builtin_amdgcn_wave_barrier();
            // 2. contract: A fragments from LDS, one MFMA per chunk
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int j = kc + u;
                if (j >= ke) break;
                const uint8_t* slot = qlds[wave][u];
                i32x4 lo = i32x4{0, 0, 0, 0}, hi = i32x4{0, 0, 0, 0};
                if (r16 < M) {
                    lo = *reinterpret_cast<const i32x4*>(slot + r16 * 128 + slice * 16);
                    hi = *reinterpret_cast<const i32x4*>(slot + r16 * 128 + 64 + slice * 16);
                }
                float sa[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    sa[i] = i < XM ? __int_as_float(__builtin_amdgcn_readlane(
                                         __float_as_int(scl[u]), LPR * i))
                                   : 0.0f;
                const float swj = SM == kBlock ? b.sw[u] : swc[0];
                const f32x4 p =
                    mfma_e4m3(join(lo, hi), join(b.blo[u][0], b.bhi[u][0]), f32x4{0, 0, 0, 0});
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[0][0][i] += p[i] * (sa[i] * swj);
            }
            __builtin_amdgcn_wave_barrier();
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int j = kc + u;
                if (j >= ke) break;
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const i32x8 bb = join(b.blo[u][nt], b.bhi[u][nt]);
                    const float swj = SM == kBlock ? b.sw[u] : swc[nt];
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const i32x8 a = join(b.alo[u][mt], b.ahi[u][mt]);
                        if constexpr (SM == kConst) {
                            acc[mt][nt] = mfma_e4m3(a, bb, acc[mt][nt]);
                        } else {
                            const f32x4 p = mfma_e4m3(a, bb, f32x4{0, 0, 0, 0});
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                acc[mt][nt][i] += p[i] * (b.sa[u][mt][i] * swj);
                        }
                    }
                }
            }
        }
    };

    // Two batches in flight: issue the next U chunks before consuming the
    // current ones.
    Batch b0, b1;
    if (kb < ke) issue(b0, kb);
    for (int kc = kb; kc < ke; kc += 2 * U) {
        if (kc + U < ke) issue(b1, kc + U);
        consume(b0, kc);
        if (kc + U >= ke) break;
        if (kc + 2 * U < ke) issue(b0, kc + 2 * U);
        consume(b1, kc + U);
    }

    // ---- sum the waves' partials: the last wave to arrive does it, in a
    // fixed order (deterministic), and the other waves exit at once ----
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave][(mt * NT + nt) * 4 + i][lane] = acc[mt][nt][i];
    int old = 0;
    if (lane == 0)
        old = __hip_atomic_fetch_add(&arrive, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old != WAVES - 1) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");

    for (int idx = 0; idx < TILES * 4; ++idx) {
        const int i = idx & 3;
        const int nt = (idx >> 2) % NT;
        const int mt = (idx >> 2) / NT;
        const int row = mt * 16 + (lane >> 4) * 4 + i;
        const int col = n0 + nt * 16 + (lane & 15);
        if (row >= M || col >= N) continue;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) v += red[w][idx][lane];
        if constexpr (SM == kConst) {
            const float sa = op.s[row], sw = op.sw[col];
            v = M == 1 ? v * (sa * sw) : (v * sa) * sw;
        }
        const size_t o = (size_t)row * N + col;
        if (op.c_f32) {
            float* c = static_cast<float*>(op.c);
            c[o] = op.residual ? v + c[o] : v;
        } else {
            uint16_t* c = static_cast<uint16_t*>(op.c);
            if (op.residual) v += __uint_as_float((uint32_t)c[o] << 16);
            c[o] = f32_to_bf16(v);
        }
    }
}

namespace {

std::atomic<int> g_tune_waves{0};
std::atomic<int> g_tune_u{0};

template <int WAVES, int MT, int NT, int U, int XM>
hipError_t launch_cfg(const SkinnyArgs& a, hipStream_t stream, const LaunchTiming& t)
{
    const dim3 grid((a.op.N + 16 * NT - 1) / (16 * NT));
    const dim3 block(WAVES * 64);
    if (a.op.w_block)
        return launch(fp8_skinny_kernel<WAVES, MT, NT, U, XM, kBlock>, grid, block, 0,
                      stream, t, a);
    if constexpr (XM == 0) {
        if (a.op.s_step == 0)
            return launch(fp8_skinny_kernel<WAVES, MT, NT, U, 0, kConst>, grid, block,
                          0, stream, t, a);
    }
    return launch(fp8_skinny_kernel<WAVES, MT, NT, U, XM, kChannel>, grid, block, 0,
                  stream, t, a);
}

template <int MT, int NT, int U, int XM>
hipError_t launch_u(const SkinnyArgs& a, hipStream_t stream, const LaunchTiming& t, int waves)
{
    // 16-wave workgroups must fit 128 VGPRs: only the 2-chunk batch with a
    // single tile does.
    switch (waves) {
    case 16:
        if constexpr (MT * NT == 1 && U == 2) return launch_cfg<16, MT, NT, U, XM>(a, stream, t);
        else return launch_cfg<8, MT, NT, U, XM>(a, stream, t);
    case 8: return launch_cfg<8, MT, NT, U, XM>(a, stream, t);
    case 2: return launch_cfg<2, MT, NT, U, XM>(a, stream, t);
    default: return launch_cfg<4, MT, NT, U, XM>(a, stream, t);
    }
}

// Waves per workgroup: enough waves in total to keep the weight stream
// deep (small N gets more waves per column tile, splitting K finer).
int pick_waves(int tiles, int KC, int U)
{
    const int forced = g_tune_waves.load(std::memory_order_relaxed);
    if (forced) return forced;
    int w = 4;
    while (w < 16 && tiles * w < 4096 && KC >= 2 * w * U) w *= 2;
    return w;
}

template <int MT, int NT, int XM>
hipError_t launch_tiles(const SkinnyArgs& a, hipStream_t stream, const LaunchTiming& t)
{
    const int tiles = (a.op.N + 16 * NT - 1) / (16 * NT);
    const int KC = a.op.K / kChunk;
    if constexpr (MT * NT == 1) {
        if (g_tune_u.load(std::memory_order_relaxed) == 4)
            return launch_u<MT, NT, 4, XM>(a, stream, t, pick_waves(tiles, KC, 4));
    }
    return launch_u<MT, NT, 2, XM>(a, stream, t, pick_waves(tiles, KC, 2));
}

}  // namespace

hipError_t launch_fp8_skinny(const Fp8Operands& op, bool fused, hipStream_t stream,
                             const LaunchTiming& t, const char** name)
{
    SkinnyArgs a{op, fused};
    if (fused) {
        *name = "fp8_skinny_fused_m4";
        if (op.M == 1) return launch_tiles<1, 1, 1>(a, stream, t);
        if (op.M == 2) return launch_tiles<1, 1, 2>(a, stream, t);
        return launch_tiles<1, 1, 4>(a, stream, t);
    }
    if (op.M <= 4) {
        *name = "fp8_skinny_m4";
        return launch_tiles<1, 1, 0>(a, stream, t);
    }
    if (op.M <= 16) {
        *name = "fp8_skinny_m16";
        return launch_tiles<1, 2, 0>(a, stream, t);
    }
    *name = "fp8_skinny_m32";
    return launch_tiles<2, 2, 0>(a, stream, t);
}

void skinny_tune(int waves, int u)
{
    g_tune_waves.store(waves, std::memory_order_relaxed);
    g_tune_u.store(u, std::memory_order_relaxed);
}

}  // namespace heph
