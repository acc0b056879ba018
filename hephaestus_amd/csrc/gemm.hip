// gemm.hip - W8A8 FP8 GEMM for prefill (any M; chosen for M > 32).
//
// Replaces the reference's prefill kernel wmma_gemm_kernel_v3a_fp8
// (src/hephaestus/wmma_gfx12.mojo:756-888: 64x64 tile, BK=16, single LDS
// buffer, two barriers per 16-wide K step, rank-1 scale epilogue). Here:
//   * 128x128 output tile per 256-thread workgroup, 2x2 waves of 64x64,
//     each wave 4x4 v_mfma_f32_16x16x128_f8f6f4 per 128-wide K chunk;
//   * K advances one 128-wide chunk per step, which is exactly one
//     activation group and one weight block, so each MFMA result is a
//     chunk partial that is rescaled in registers by sa[m,j] * sw[n/128,j]
//     and accumulated in fp32 (one FMA per accumulator per chunk);
//   * with the reference's granularity (per-channel weight, per-token
//     activation scale) nothing varies along K: the MFMAs accumulate
//     directly and the epilogue applies (acc*sa)*sw as the reference's
//     prefill kernel does (wmma_gfx12.mojo:848; acc*(sa*sw) at M = 1 to
//     match its decode kernel, :711-712);
//   * A/B tiles are double buffered in LDS (one barrier per chunk), with
//     the next chunk's global loads in flight during the MFMAs; LDS rows
//     are padded to 144 bytes to spread the 16-byte fragment reads;
//   * the block -> tile order gives each XCD a contiguous run of tiles in
//     a grouped (8 tile-rows) order, so A and B tiles are reused from that
//     XCD's L2.
#include "heph_kernels.h"

namespace heph {

namespace {
constexpr int BM = 128;
constexpr int BN = 128;
constexpr int LDSTR = kChunk + 16;  // bytes per LDS row
constexpr int GROUP_M = 8;
constexpr int NXCD = 8;

__device__ __forceinline__ i32x4 lds16(const uint8_t* p)
{
    return *reinterpret_cast<const i32x4*>(p);
}

// Block id -> (tile_m, tile_n): contiguous ranges per XCD (blocks are
// handed to the 8 XCDs round robin), then grouped row-major order.
__device__ __forceinline__ void tile_of_block(int bid, int tiles_m, int tiles_n,
                                              int* tm, int* tn)
{
    const int nb = tiles_m * tiles_n;
    const int per = nb / NXCD, rem = nb % NXCD;
    const int x = bid % NXCD, k = bid / NXCD;
    const int lin = x * per + min(x, rem) + k;
    const int width = GROUP_M * tiles_n;
    const int g = lin / width;
    const int first_m = g * GROUP_M;
    const int gsize = min(tiles_m - first_m, GROUP_M);
    const int r = lin % width;
    *tm = first_m + r % gsize;
    *tn = r / gsize;
}
}  // namespace

// SM: 0 = 128x128 weight blocks, 1 = per-channel weights with per-chunk
// activation scales, 2 = per-channel weights and per-token activations.
template <int SM>
__global__ __launch_bounds__(256, 2) void fp8_gemm_kernel(Fp8Operands op)
{
    __shared__ __attribute__((aligned(16))) uint8_t As[2][BM * LDSTR];
    __shared__ __attribute__((aligned(16))) uint8_t Bs[2][BN * LDSTR];
    __shared__ float Ss[2][BM];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int r16 = lane & 15, slice = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;
    const int M = op.M, N = op.N, K = op.K, KC = K >> 7;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int tm, tn;
    tile_of_block(blockIdx.x, tiles_m, tiles_n, &tm, &tn);
    const int m0 = tm * BM, n0 = tn * BN;

    // Global -> LDS staging: 1024 16-byte pieces per operand tile, four per
    // thread; eight consecutive threads cover one 128-byte row.
    const int lrow = tid >> 3, lcol = (tid & 7) * 16;
    const uint8_t* ag[4];
    const uint8_t* bg[4];
    bool aok[4], bok[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = m0 + lrow + 32 * r, n = n0 + lrow + 32 * r;
        aok[r] = m < M;
        bok[r] = n < N;
        ag[r] = op.q + (size_t)(aok[r] ? m : 0) * K + lcol;
        bg[r] = op.w + (size_t)(bok[r] ? n : 0) * K + lcol;
    }
    const bool sok = tid < BM && m0 + tid < M;
    const float* sg = op.s + (size_t)(sok ? m0 + tid : 0) * op.s_ld;

    i32x4 ra[4], rb[4];
    float rs = 0.0f;
    auto gload = [&](int j) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            ra[r] = aok[r] ? ldg16(ag[r] + (size_t)j * kChunk) : i32x4{0, 0, 0, 0};
            rb[r] = bok[r] ? ldg16(bg[r] + (size_t)j * kChunk) : i32x4{0, 0, 0, 0};
        }
        rs = sok ? sg[j * op.s_step] : 0.0f;
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            *reinterpret_cast<i32x4*>(&As[buf][(lrow + 32 * r) * LDSTR + lcol]) = ra[r];
            *reinterpret_cast<i32x4*>(&Bs[buf][(lrow + 32 * r) * LDSTR + lcol]) = rb[r];
        }
        if (tid < BM) Ss[buf][tid] = rs;
    };

    float swc[4];
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
        const int n = n0 + wn * 64 + ni * 16 + r16;
        swc[ni] = SM == 1 ? op.sw[n < N ? n : 0] : 0.0f;
    }
    const float* swb = op.sw + (size_t)(n0 >> 7) * op.sw_ld;

    f32x4 acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = f32x4{0, 0, 0, 0};

    gload(0);
    lstore(0);
    __syncthreads();

    for (int j = 0; j < KC; ++j) {
        const int cur = j & 1;
        if (j + 1 < KC) gload(j + 1);

        i32x8 a[4], b[4];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
            const uint8_t* p = &As[cur][(wm * 64 + mi * 16 + r16) * LDSTR + slice * 16];
            a[mi] = join(lds16(p), lds16(p + 64));
        }
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            const uint8_t* p = &Bs[cur][(wn * 64 + ni * 16 + r16) * LDSTR + slice * 16];
            b[ni] = join(lds16(p), lds16(p + 64));
        }
        if constexpr (SM == 2) {
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma_e4m3(a[mi], b[ni], acc[mi][ni]);
        } else {
            const float swj = SM == 0 ? swb[j] : 1.0f;
            float sc[4][4];
#pragma unroll
            for (int mi = 0; mi < 4; ++mi) {
                const f32x4 s4 =
                    *reinterpret_cast<const f32x4*>(&Ss[cur][wm * 64 + mi * 16 + slice * 4]);
#pragma unroll
                for (int i = 0; i < 4; ++i) sc[mi][i] = s4[i] * swj;
            }
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) {
                    const f32x4 p = mfma_e4m3(a[mi], b[ni], f32x4{0, 0, 0, 0});
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[mi][ni][i] += p[i] * (SM == 0 ? sc[mi][i] : sc[mi][i] * swc[ni]);
                }
        }

        if (j + 1 < KC) lstore(cur ^ 1);
        __syncthreads();
    }

    // Epilogue: lane holds rows (slice*4 + i) of each 16x16 tile, column r16.
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            const int col = n0 + wn * 64 + ni * 16 + r16;
            if (col >= N) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = m0 + wm * 64 + mi * 16 + slice * 4 + i;
                if (row >= M) continue;
                const size_t o = (size_t)row * N + col;
                float v = acc[mi][ni][i];
                if constexpr (SM == 2) {
                    const float sa = op.s[row], sw = op.sw[col];
                    v = M == 1 ? v * (sa * sw) : (v * sa) * sw;
                }
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
}

hipError_t launch_fp8_gemm(const Fp8Operands& op, hipStream_t stream,
                           const LaunchTiming& t, const char** name)
{
    const int tiles = ((op.M + BM - 1) / BM) * ((op.N + BN - 1) / BN);
    *name = "fp8_gemm_128x128";
    if (op.w_block)
        return launch(fp8_gemm_kernel<0>, dim3(tiles), dim3(256), 0, stream, t, op);
    if (op.s_step == 0)
        return launch(fp8_gemm_kernel<2>, dim3(tiles), dim3(256), 0, stream, t, op);
    return launch(fp8_gemm_kernel<1>, dim3(tiles), dim3(256), 0, stream, t, op);
}

}  // namespace heph
