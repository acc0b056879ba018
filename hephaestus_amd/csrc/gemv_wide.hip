// gemv_wide.hip - W8A8 FP8 linear for batched decode (M <= 32) with wide
// column tiles over all of K: no sums across workgroups.
//
// Replaces the reference's small-M kernel (src/hephaestus/wmma_gfx12.mojo:
// 900-1019, reached through linear_fp8, kernels.mojo:410-470) for batches
// of up to 32 rows. At M = 1 the chunk-slot GEMV fills the 16 MFMA rows
// with K chunks; from about M = 9 on, M activation rows fill them by
// themselves, and what costs is the activation side: every workgroup needs
// all M x K activations of its K range. Here a workgroup covers 16*T output
// columns over all of K, so one activation operand serves T weight tiles
// in registers, and no workgroup waits for another's partial sums (a sum
// across workgroups goes through the coherent level, ~1 us a round trip).
//   * operands: the weights are the MFMA's first operand (16 output
//     columns as its rows), the activations its second (16 activation rows
//     as its columns), so lane l's four results are output columns
//     16t + 4*(l >> 4) + i of activation row l & 15;
//   * it reads activation codes and scales from the workspace (written by
//     the quantizer launch or by a producer): quantizing inside would
//     repeat all M x K activations in every workgroup, which on MI355X
//     cost more than the separate launch from M = 9 on (qkv at M = 32:
//     14.4 against 2.3 + 8.2 us);
//   * workgroup = 16*T columns; its WAVES waves split the K chunks into
//     contiguous runs; loads go out in batches of U chunks, two batches in
//     flight, activations first (L2-resident), then the weight fragments
//     (two 16-byte loads per lane, tile and chunk, in the operand layout);
//   * activations reach the operand layout through a per-wave LDS tile:
//     in the operand layout one 16-byte load per lane touches 16 rows x
//     64 bytes, and from the L2 that ran at about half the rate of loads
//     of whole 128-byte lines (MI355X, down_proj at M = 32: 13.5 against
//     8.0 us for the activation loads alone), so the rows are loaded in
//     whole lines and rearranged in LDS (16-byte pieces XOR-swizzled by
//     row). Weights stream from HBM, where the two patterns run alike;
//   * per chunk, row tile and column tile one v_mfma_f32_16x16x128_f8f6f4,
//     acc += p * (sa * sw) (block scales; per-channel: sw of each column),
//     the association of the library's other kernels; per-token activation
//     scales with per-channel weights accumulate unscaled and apply
//     (acc * sa) * sw at the end (wmma_gfx12.mojo:973);
//   * the waves' sums meet in LDS (each wave's staging tile, reused) after
//     one barrier and are added in wave order (deterministic); each thread
//     then finishes four consecutive columns of one row: residual (f32 add
//     of the bf16 value), bf16 or f32 store.
#include "heph_kernels.h"

namespace heph {

namespace {

enum WideScale { kWideBlock = 0, kWideChannel = 1, kWideConst = 2 };

// Byte offset of 16-byte piece p of row r in a 16-row x 128-byte LDS tile.
__device__ __forceinline__ int stage_off(int r, int p) { return r * kChunk + ((p ^ (r & 7)) << 4); }

}  // namespace

template <int WAVES, int T, int RT, int U, int SM>
__global__ __launch_bounds__(WAVES * 64) void fp8_gemv_wide_kernel(Fp8Operands op)
{
    static_assert(T == 1 || T == 2 || T == 4, "column tiles per workgroup");
    static_assert(RT == 1 || RT == 2, "row tiles");
    constexpr int NT = 16 * T;
    constexpr int NACC = T * RT * 4;
    constexpr int kTile = 16 * kChunk;                     // one row tile's codes
    constexpr int kRegion = RT * kTile > NACC * 256 ? RT * kTile : NACC * 256;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int M = op.M, K = op.K;
    const int KC = K >> 7;
    const int n0 = blockIdx.x * NT;
    const int per = (KC + WAVES - 1) / WAVES;
    const int jb = min(KC, wave * per);
    const int je = min(KC, jb + per);

    // per wave: the staging tiles during the loop, its partial sums after
    __shared__ __attribute__((aligned(16))) uint8_t region[WAVES][kRegion];
    uint8_t* tile = region[wave];

    const uint8_t* wrow = op.w + (size_t)(n0 + r16) * K + g * 16;
    const float* swb = op.sw + (size_t)(n0 >> 7) * op.sw_ld;
    float swc[T][4];
    if constexpr (SM == kWideChannel) {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) swc[t][i] = op.sw[n0 + 16 * t + 4 * g + i];
    }
    bool live[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) live[rt] = rt * 16 + r16 < M;
    // whole-line activation loads: lane -> rows (lane >> 3) and + 8,
    // 16-byte piece lane & 7
    const int lrow = lane >> 3, lpc = lane & 7;

    struct Batch {
        i32x4 wlo[U][T], whi[U][T];
        uint4 a[U][RT][2];
        float sa[U][RT];
        float sw[U];    // block scale: 16*T divides 128, one block per tile
    };

    // Loads are unconditional: a chunk past je re-reads chunk je-1 (never
    // consumed), a row past M re-reads row M-1 (masked when consumed).
    auto issue = [&](Batch& b, int j) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int jj = min(j + u, je - 1);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const size_t row = (size_t)min(rt * 16 + lrow + 8 * h, M - 1);
                    b.a[u][rt][h] = ldg16u(op.q + row * K + (size_t)jj * kChunk + lpc * 16);
                }
                if constexpr (SM != kWideConst) {
                    const int m = min(rt * 16 + r16, M - 1);
                    b.sa[u][rt] = op.s[(size_t)m * op.s_ld + (size_t)jj * op.s_step];
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int jj = min(j + u, je - 1);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const uint8_t* p = wrow + (size_t)(16 * t) * K + (size_t)jj * kChunk;
                b.wlo[u][t] = ldg16(p);
                b.whi[u][t] = ldg16(p + 64);
            }
            if constexpr (SM == kWideBlock) b.sw[u] = swb[jj];
        }
    };

    float acc[T][RT][4];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t][rt][i] = 0.0f;

    auto consume = [&](Batch& b, int j) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (j + u >= je) break;
            // 1. this wave's staging tiles
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    *reinterpret_cast<uint4*>(tile + rt * kTile + stage_off(lrow + 8 * h, lpc)) =
                        b.a[u][rt][h];
            __builtin_amdgcn_wave_barrier();
            // 2. operands from the tiles, MFMAs
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const uint8_t* tl = tile + rt * kTile;
                i32x4 alo = *reinterpret_cast<const i32x4*>(tl + stage_off(r16, g));
                i32x4 ahi = *reinterpret_cast<const i32x4*>(tl + stage_off(r16, g + 4));
                if (!live[rt]) {
                    alo = i32x4{0, 0, 0, 0};
                    ahi = i32x4{0, 0, 0, 0};
                }
                float sa = 0.0f;
                if constexpr (SM != kWideConst) sa = b.sa[u][rt];
                const i32x8 a = join(alo, ahi);
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    const f32x4 p = mfma_e4m3(join(b.wlo[u][t], b.whi[u][t]), a,
                                              f32x4{0, 0, 0, 0});
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if constexpr (SM == kWideConst) acc[t][rt][i] += p[i];
                        else if constexpr (SM == kWideBlock)
                            acc[t][rt][i] += p[i] * (sa * b.sw[u]);
                        else acc[t][rt][i] += p[i] * (sa * swc[t][i]);
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();
        }
    };

    Batch b0, b1;
    if (jb < je) issue(b0, jb);
    if (jb + U < je) issue(b1, jb + U);
    for (int j = jb; j < je; j += 2 * U) {
        consume(b0, j);
        if (j + 2 * U < je) issue(b0, j + 2 * U);
        if (j + U >= je) break;
        consume(b1, j + U);
        if (j + 3 * U < je) issue(b1, j + 3 * U);
    }

    float* red = reinterpret_cast<float*>(tile);
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[((t * RT + rt) * 4 + i) * 64 + lane] = acc[t][rt][i];
    __syncthreads();

    // thread o: columns n0 + 4*cg .. +3 of row m, from lane gg*16 + m%16 of
    // each wave's tile t = cg / 4, elements 0..3
    constexpr int GROUPS = NT / 4;
    for (int o = threadIdx.x; o < M * GROUPS; o += WAVES * 64) {
        const int m = o / GROUPS, cg = o % GROUPS;
        const int t = cg >> 2, gg = cg & 3, rt = m >> 4;
        const int ln = gg * 16 + (m & 15);
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w)
                s += reinterpret_cast<const float*>(region[w])[((t * RT + rt) * 4 + i) * 64 + ln];
            v[i] = s;
        }
        const int col = n0 + 4 * cg;
        if constexpr (SM == kWideConst) {
            const float sa = op.s[(size_t)m * op.s_ld];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float sw = op.sw[col + i];
                v[i] = M == 1 ? v[i] * (sa * sw) : (v[i] * sa) * sw;
            }
        }
        const size_t oi = (size_t)m * op.N + col;
        if (op.c_f32) {
            f32x4* c = reinterpret_cast<f32x4*>(static_cast<float*>(op.c) + oi);
            f32x4 r = f32x4{v[0], v[1], v[2], v[3]};
            if (op.residual) r += *c;
            *c = r;
        } else {
            uint2* c = reinterpret_cast<uint2*>(static_cast<uint16_t*>(op.c) + oi);
            if (op.residual) {
                const uint2 rv = *c;
                v[0] += bf16lo(rv.x);
                v[1] += bf16hi(rv.x);
                v[2] += bf16lo(rv.y);
                v[3] += bf16hi(rv.y);
            }
            *c = make_uint2((uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16),
                            (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16));
        }
    }
}

namespace {

template <int WAVES, int T, int RT, int U>
hipError_t launch_wide_t(const Fp8Operands& op, hipStream_t stream, const LaunchTiming& lt)
{
    const dim3 grid(op.N / (16 * T));
    const dim3 block(WAVES * 64);
    if (op.w_block)
        return launch(fp8_gemv_wide_kernel<WAVES, T, RT, U, kWideBlock>, grid, block, 0, stream,
                      lt, op);
    if (op.s_step == 0)
        return launch(fp8_gemv_wide_kernel<WAVES, T, RT, U, kWideConst>, grid, block, 0, stream,
                      lt, op);
    return launch(fp8_gemv_wide_kernel<WAVES, T, RT, U, kWideChannel>, grid, block, 0, stream,
                  lt, op);
}

template <int WAVES, int T, int U>
hipError_t launch_wide_rt(const Fp8Operands& op, hipStream_t stream, const LaunchTiming& lt)
{
    if (op.M > 16) return launch_wide_t<WAVES, T, 2, U>(op, stream, lt);
    return launch_wide_t<WAVES, T, 1, U>(op, stream, lt);
}

template <int WAVES, int U>
hipError_t launch_wide_w(const Fp8Operands& op, int tiles, hipStream_t stream,
                         const LaunchTiming& lt)
{
    if (tiles == 4) return launch_wide_rt<WAVES, 4, U>(op, stream, lt);
    if (tiles == 2) return launch_wide_rt<WAVES, 2, U>(op, stream, lt);
    return launch_wide_rt<WAVES, 1, U>(op, stream, lt);
}

}  // namespace

// Default route (MI355X, graph-replayed per call over HBM-streamed
// weights, codes from the workspace): from M = 8 on codes and M = 9 on bf16
// rows (the separate quantizer launch costs ~2.3 us; up to M = 8 the
// chunk-slot GEMV's fused quantization is cheaper), except past M = 24 on
// large weights, where the K-split kernels read fewer activation bytes per
// workgroup (M = 32: gate_up 17.0 against 17.8 us, down_proj 15.0 against
// 15.7 on codes; qkv 8.2 against 12.2 and o_proj 7.5 against 9.1 go here).
bool gemv_wide_routes(int M, int N, int K, bool codes)
{
    if (M < (codes ? 8 : 9) || M > 32) return false;
    return !(M > 24 && ((long)N * K >= (32L << 20) || K >= 8192));
}

// Launch shape: two column tiles where that still gives >= 192 workgroups,
// else one (qkv, gate_up: 2; N = 2560: 1); 8 waves from K = 4096 on, else
// 4; one-chunk batches, two at K >= 8192 with two row tiles. Overrides
// from op.tune (wide_tiles > 0, wide_waves, gemv_u); the tile count is
// halved until it divides N / 16. Sixteen waves take one column tile and
// one row tile (LDS), four column tiles with two row tiles one-chunk
// batches (registers).
void gemv_wide_shape(int M, int N, int K, const Tuning& tune, int* tiles, int* waves, int* u)
{
    const int nt = N / 16;
    int t = nt % 2 == 0 && nt / 2 >= 192 ? 2 : 1;
    if (tune.wide_tiles > 0) t = tune.wide_tiles;
    while (t > 1 && nt % t != 0) t >>= 1;
    int w = K >= 4096 ? 8 : 4;
    if (tune.wide_waves) w = tune.wide_waves;
    int uu = K >= 8192 && M > 16 ? 2 : 1;
    if (tune.gemv_u) uu = tune.gemv_u;
    if (w == 16) {
        t = 1;
        uu = 1;
        if (M > 16) w = 8;
    }
    if (t == 4 && M > 16) uu = 1;
    *tiles = t;
    *waves = w;
    *u = uu;
}

hipError_t launch_fp8_gemv_wide(const Fp8Operands& op, hipStream_t stream,
                                const LaunchTiming& lt, const char** name)
{
    int tiles, waves, u;
    gemv_wide_shape(op.M, op.N, op.K, op.tune, &tiles, &waves, &u);
    *name = "fp8_gemv_wide";
    if (waves == 16) return launch_wide_t<16, 1, 1, 1>(op, stream, lt);
    if (waves == 8)
        return u == 2 ? launch_wide_w<8, 2>(op, tiles, stream, lt)
                      : launch_wide_w<8, 1>(op, tiles, stream, lt);
    return u == 2 ? launch_wide_w<4, 2>(op, tiles, stream, lt)
                  : launch_wide_w<4, 1>(op, tiles, stream, lt);
}

}  // namespace heph
