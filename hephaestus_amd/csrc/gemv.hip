// gemv.hip - W8A8 FP8 linear at M = 1 (the decode GEMV).
//
// Replaces the reference's decode GEMV (src/hephaestus/wmma_gfx12.mojo:650-744,
// reached through gemv_fp8 / linear_fp8, src/hephaestus/kernels.mojo:372-470),
// which gives one 32-lane wave a 16-column tile over all of K.
//
// At M = 1 only one row of the 16x16 MFMA tile carries data. This kernel
// fills the other rows with further K-chunks instead ("chunk slots"): with
// KS slots, MFMA column c holds output column n0 + c % TW (TW = 16 / KS) at
// K-chunk step*KS + c / TW, and A row t holds the activation chunk of slot
// t. The wanted product of column c is then C[c / TW][c]; every other C
// element is unused. One v_mfma_f32_16x16x128_f8f6f4 covers KS chunks of
// TW columns, so a workgroup owns only TW output columns and the grid has
// N*KS/16 workgroups: enough to cover all 256 CUs even at N = 2560, with
// no reduction across workgroups.
//   * workgroup = TW output columns; its WAVES waves split the KC/KS steps
//     into contiguous runs; loads go out in batches of U steps, two batches
//     in flight, each lane issuing two 16-byte weight loads per step;
//   * fused mode (1x128 groups) quantizes x inside the kernel: 64/KS lanes
//     share a slot's 128-element group, its max is reduced with DPP, the
//     scale is the reference's own division (amax/448, 1/s, both rounded to
//     nearest even), and the codes reach the MFMA A layout through a
//     per-wave LDS tile. Workgroup 0 also writes q/s to the workspace so
//     later SKIP_QUANT calls can reuse them;
//   * each lane rescales its own C element by sa[chunk] * sw[block, chunk]
//     in registers; per-channel/per-token scales (the reference's own
//     granularity) accumulate unscaled and apply acc*(sa*sw) at the end
//     (wmma_gfx12.mojo:711-712);
//   * the last wave of a workgroup to finish sums the waves' slot partials
//     in a fixed order (deterministic) and stores bf16 or f32, optionally
//     adding the residual first (wmma_gfx12.mojo:712-715).
#include <atomic>

#include "heph_kernels.h"

namespace heph {

struct GemvArgs {
    Fp8Operands op;
    bool write_ws;
};

enum GemvScale { kGemvBlock = 0, kGemvChannel = 1, kGemvConst = 2 };

namespace {

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float readlane_f(float v, int l)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Max over each aligned run of LPR lanes (LPR = 8, 16, 32 or 64).
template <int LPR>
__device__ __forceinline__ float lanes_max(float m)
{
    m = fmaxf(m, dpp_f<0xB1>(m));    // quad_perm [1,0,3,2]
    m = fmaxf(m, dpp_f<0x4E>(m));    // quad_perm [2,3,0,1]
    m = fmaxf(m, dpp_f<0x141>(m));   // row_half_mirror: runs of 8
    if constexpr (LPR >= 16) m = fmaxf(m, dpp_f<0x140>(m));   // row_mirror: 16
    if constexpr (LPR >= 32) m = fmaxf(m, __shfl_xor(m, 16));
    if constexpr (LPR == 64) m = fmaxf(readlane_f(m, 0), readlane_f(m, 32));
    return m;
}

// The reference group scale (kernels.mojo:173-181): s = amax / 448, 1.0
// below 1e-12, inv = 1 / s; both divisions IEEE round-to-nearest-even.
__device__ __forceinline__ void group_scale_div(float amax, float& s, float& inv)
{
    s = __fdiv_rn(amax, kE4M3Max);
    if (s < 1e-12f) s = 1.0f;
    inv = __frcp_rn(s);
}

// E consecutive bf16 activations (E = 2, 4, 8 or 16) as E/2 dwords.
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
    else *reinterpret_cast<uint4*>(p) = make_uint4(cd[0], cd[1], cd[2], cd[3]);
}

}  // namespace

template <int WAVES, int KS, int U, bool FUSED, int SM>
__global__ __launch_bounds__(WAVES * 64) void fp8_gemv_kernel(GemvArgs args)
{
    static_assert(KS == 1 || KS == 2 || KS == 4 || KS == 8, "chunk slots");
    static_assert(!(FUSED && SM == kGemvConst), "per-token quantization is not fused");
    constexpr int TW = 16 / KS;          // output columns per workgroup
    constexpr int LPR = 64 / KS;         // quantizing lanes per slot
    constexpr int E = 128 / LPR;         // activations per quantizing lane
    const Fp8Operands& op = args.op;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int t = r16 / TW;              // chunk slot of this lane's column
    const int ei = t & 3;                // its C element: row t, in lane group t/4
    const int K = op.K;
    const int KC = K >> 7;
    const int S = (KC + KS - 1) / KS;    // steps of KS chunks
    const int n0 = blockIdx.x * TW;
    const int per = (S + WAVES - 1) / WAVES;
    const int sb = min(S, wave * per);
    const int se = min(S, sb + per);
    const int qrow = lane / LPR, qpiece = lane % LPR;

    __shared__ float red[WAVES][64];
    __shared__ int arrive;
    __shared__ __attribute__((aligned(16))) uint8_t qlds[FUSED ? WAVES : 1][FUSED ? U : 1]
                                                        [KS * kChunk];
    if (threadIdx.x == 0) arrive = 0;
    __syncthreads();

    const int n = n0 + r16 % TW;
    const uint8_t* wrow = op.w + (size_t)n * K + g * 16;
    const float* swb = op.sw + (size_t)(n0 >> 7) * op.sw_ld;
    const float swc = SM == kGemvBlock ? 0.0f : op.sw[n];

    struct Batch {
        i32x4 blo[U], bhi[U];
        i32x4 alo[FUSED ? 1 : U], ahi[FUSED ? 1 : U];
        XVec<E> xv[FUSED ? U : 1];
        float sw[U];
        float sa[FUSED ? 1 : U];
    };

    // Loads are unconditional and clamped, so a batch is one straight run
    // of memory instructions: a step past se re-reads step se-1 (never
    // consumed) and a chunk past KC re-reads chunk KC-1 with a zero
    // activation row. Activation loads go first so their quantization can
    // run while the weights are still in flight.
    auto issue = [&](Batch& b, int s) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int st = min(s + u, se - 1);
            if constexpr (FUSED) {
                const int jx = st * KS + qrow;
                const XVec<E> v =
                    load_xvec<E>(op.x + (size_t)min(jx, KC - 1) * kChunk + qpiece * E);
#pragma unroll
                for (int d = 0; d < E / 2; ++d) b.xv[u].d[d] = jx < KC ? v.d[d] : 0u;
            } else {
                const int ja = st * KS + r16;
                const uint8_t* p = op.q + (size_t)min(ja, KC - 1) * kChunk + g * 16;
                const i32x4 lo = ldg16(p), hi = ldg16(p + 64);
                const bool live = r16 < KS && ja < KC;
                b.alo[u] = live ? lo : i32x4{0, 0, 0, 0};
                b.ahi[u] = live ? hi : i32x4{0, 0, 0, 0};
                if constexpr (SM != kGemvConst)
                    b.sa[u] = op.s[(size_t)min(st * KS + t, KC - 1) * op.s_step];
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int st = min(s + u, se - 1);
            const int jb = min(st * KS + t, KC - 1);
            const uint8_t* p = wrow + (size_t)jb * kChunk;
            b.blo[u] = ldg16(p);
            b.bhi[u] = ldg16(p + 64);
            if constexpr (SM == kGemvBlock) b.sw[u] = swb[jb];
        }
    };

    float acc = 0.0f;
    auto contract = [&](const i32x4& alo, const i32x4& ahi, const i32x4& blo,
                        const i32x4& bhi, float scale) {
        const f32x4 p = mfma_e4m3(join(alo, ahi), join(blo, bhi), f32x4{0, 0, 0, 0});
        const float v = ei == 0 ? p[0] : ei == 1 ? p[1] : ei == 2 ? p[2] : p[3];
        if constexpr (SM == kGemvConst) acc += v;
        else acc += v * scale;
    };

    auto consume = [&](Batch& b, int s) {
        if constexpr (FUSED) {
            // 1. quantize the batch's chunks into this wave's LDS tiles
            float sc[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (s + u >= se) break;
                float m = 0.0f;
#pragma unroll
                for (int d = 0; d < E / 2; ++d)
                    m = fmaxf(m, fmaxf(fabsf(bf16lo(b.xv[u].d[d])), fabsf(bf16hi(b.xv[u].d[d]))));
                m = lanes_max<LPR>(m);
                float inv;
                group_scale_div(m, sc[u], inv);
                uint32_t cd[(E + 3) / 4];
                if constexpr (E == 2) {
                    cd[0] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(
                        bf16lo(b.xv[u].d[0]) * inv, bf16hi(b.xv[u].d[0]) * inv, 0, false);
                } else {
#pragma unroll
                    for (int d = 0; d < E / 4; ++d) {
                        const uint32_t a0 = b.xv[u].d[2 * d], a1 = b.xv[u].d[2 * d + 1];
                        cd[d] = pack4_e4m3(bf16lo(a0) * inv, bf16hi(a0) * inv,
                                           bf16lo(a1) * inv, bf16hi(a1) * inv);
                    }
                }
                store_codes<E>(qlds[wave][u] + qrow * kChunk + qpiece * E, cd);
                const int jx = (s + u) * KS + qrow;
                if (args.write_ws && blockIdx.x == 0 && jx < KC) {
                    store_codes<E>(op.q + (size_t)jx * kChunk + qpiece * E, cd);
                    if (qpiece == 0) op.s[jx] = sc[u];
                }
            }
            __builtin_amdgcn_wave_barrier();
            // 2. contract: A rows 0..KS-1 from LDS, the slot's scale from the
            //    lanes that quantized it
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (s + u >= se) break;
                const uint8_t* tile = qlds[wave][u];
                i32x4 lo = i32x4{0, 0, 0, 0}, hi = i32x4{0, 0, 0, 0};
                if (r16 < KS) {
                    lo = *reinterpret_cast<const i32x4*>(tile + r16 * kChunk + g * 16);
                    hi = *reinterpret_cast<const i32x4*>(tile + r16 * kChunk + 64 + g * 16);
                }
                const float sa = KS == 1 ? sc[u]
                                         : __int_as_float(__builtin_amdgcn_ds_bpermute(
                                               t * LPR * 4, __float_as_int(sc[u])));
                const float sw = SM == kGemvBlock ? b.sw[u] : swc;
                contract(lo, hi, b.blo[u], b.bhi[u], sa * sw);
            }
            __builtin_amdgcn_wave_barrier();
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (s + u >= se) break;
                const float sw = SM == kGemvBlock ? b.sw[u] : swc;
                contract(b.alo[u], b.ahi[u], b.blo[u], b.bhi[u],
                         SM == kGemvConst ? 0.0f : b.sa[u] * sw);
            }
        }
    };

    // Two batches in flight: issue the next U steps before consuming the
    // current ones.
    Batch b0, b1;
    if (sb < se) issue(b0, sb);
    for (int s = sb; s < se; s += 2 * U) {
        if (s + U < se) issue(b1, s + U);
        consume(b0, s);
        if (s + U >= se) break;
        if (s + 2 * U < se) issue(b0, s + 2 * U);
        consume(b1, s + U);
    }

    // ---- the last wave to arrive sums the partials in a fixed order ----
    red[wave][lane] = acc;
    int old = 0;
    if (lane == 0)
        old = __hip_atomic_fetch_add(&arrive, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old != WAVES - 1) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");

    if (lane < TW) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w)
#pragma unroll
            for (int ts = 0; ts < KS; ++ts) v += red[w][(ts >> 2) * 16 + ts * TW + lane];
        const int col = n0 + lane;
        if constexpr (SM == kGemvConst) v = v * (op.s[0] * op.sw[col]);
        if (op.c_f32) {
            float* c = static_cast<float*>(op.c);
            c[col] = op.residual ? v + c[col] : v;
        } else {
            uint16_t* c = static_cast<uint16_t*>(op.c);
            if (op.residual) v += __uint_as_float((uint32_t)c[col] << 16);
            c[col] = f32_to_bf16(v);
        }
    }
}

namespace {

std::atomic<int> g_tune_ks{0};
std::atomic<int> g_tune_waves{0};
std::atomic<int> g_tune_u{0};

template <int WAVES, int KS, int U>
hipError_t launch_ks(const GemvArgs& a, bool fused, hipStream_t stream, const LaunchTiming& t)
{
    const dim3 grid(a.op.N / (16 / KS));
    const dim3 block(WAVES * 64);
    if (fused) {
        if (a.op.w_block)
            return launch(fp8_gemv_kernel<WAVES, KS, U, true, kGemvBlock>, grid, block, 0,
                          stream, t, a);
        return launch(fp8_gemv_kernel<WAVES, KS, U, true, kGemvChannel>, grid, block, 0,
                      stream, t, a);
    }
    if (a.op.w_block)
        return launch(fp8_gemv_kernel<WAVES, KS, U, false, kGemvBlock>, grid, block, 0,
                      stream, t, a);
    if (a.op.s_step == 0)
        return launch(fp8_gemv_kernel<WAVES, KS, U, false, kGemvConst>, grid, block, 0,
                      stream, t, a);
    return launch(fp8_gemv_kernel<WAVES, KS, U, false, kGemvChannel>, grid, block, 0,
                  stream, t, a);
}

template <int WAVES, int U>
hipError_t launch_wu(const GemvArgs& a, bool fused, int ks, hipStream_t stream,
                     const LaunchTiming& t)
{
    switch (ks) {
    case 8: return launch_ks<WAVES, 8, U>(a, fused, stream, t);
    case 4: return launch_ks<WAVES, 4, U>(a, fused, stream, t);
    case 2: return launch_ks<WAVES, 2, U>(a, fused, stream, t);
    default: return launch_ks<WAVES, 1, U>(a, fused, stream, t);
    }
}

}  // namespace

// Launch shape: the fewest chunk slots that give >= 600 workgroups (about
// 2.3 per CU); 4 waves when there are at most 8 steps, else 8; 2-step
// batches when each wave has at most 2 steps, else 1-step batches.
void gemv_shape(int N, int K, int* ks, int* waves, int* u)
{
    const int tiles = N / 16, KC = K / kChunk;
    int k = 1;
    while (k < 8 && tiles * k < 600) k *= 2;
    const int S = (KC + k - 1) / k;
    int w = S <= 8 ? 4 : 8;
    int uu = (S + w - 1) / w <= 2 ? 2 : 1;
    const int fk = g_tune_ks.load(std::memory_order_relaxed);
    const int fw = g_tune_waves.load(std::memory_order_relaxed);
    const int fu = g_tune_u.load(std::memory_order_relaxed);
    *ks = fk ? fk : k;
    *waves = fw ? fw : w;
    *u = fu ? fu : uu;
}

hipError_t launch_fp8_gemv(const Fp8Operands& op, bool fused, hipStream_t stream,
                           const LaunchTiming& t, const char** name)
{
    GemvArgs a{op, fused};
    int ks, waves, u;
    gemv_shape(op.N, op.K, &ks, &waves, &u);
    *name = fused ? "fp8_gemv_fused_m1" : "fp8_gemv_m1";
    if (waves == 8)
        return u == 2 ? launch_wu<8, 2>(a, fused, ks, stream, t)
                      : launch_wu<8, 1>(a, fused, ks, stream, t);
    return u == 2 ? launch_wu<4, 2>(a, fused, ks, stream, t)
                  : launch_wu<4, 1>(a, fused, ks, stream, t);
}

void gemv_tune(int ks, int waves, int u)
{
    g_tune_ks.store(ks, std::memory_order_relaxed);
    g_tune_waves.store(waves, std::memory_order_relaxed);
    g_tune_u.store(u, std::memory_order_relaxed);
}

}  // namespace heph
