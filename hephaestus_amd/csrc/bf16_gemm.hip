// bf16_gemm.hip - unquantized bf16 linear for M > 32.
//
// Replaces the reference's bf16 GEMM for more than one row
// (src/hephaestus/wmma_gfx12.mojo:428-473, wmma_gemm_bf16, reached through
// `linear`, src/hephaestus/kernels.mojo:108-118), e.g. the lm_head over
// every position of a prompt. Rows up to 32 take the weight-streaming
// kernel in bf16_skinny.hip.
//   * 128 x 128 output tile per 256-thread workgroup, 2 x 2 waves of
//     64 x 64, each wave 4 x 4 v_mfma_f32_16x16x32_bf16 per 32-wide K step,
//     two steps per 64-element (128-byte) chunk; the MFMAs accumulate in
//     fp32 across all of K;
//   * the weights are the MFMA's first operand, so lane l's four results
//     are output columns 4*(l >> 4) + i of activation row l & 15: four
//     consecutive outputs per lane, stored together;
//   * chunks are double buffered in LDS with the next chunk's global loads
//     in flight during the MFMAs, one barrier per chunk; LDS rows padded to
//     144 bytes, so the 16 rows of a fragment read fall in distinct banks;
//   * workgroups walk the tiles in groups of 8 tile rows (each weight tile
//     is reused by 8 consecutive workgroups while it is in the L2);
//   * epilogue: the residual (the output buffer's bf16 or f32 values) is
//     added in f32 before the one rounding; rows past M and columns past N
//     are computed on clamped rows and not stored.
#include "heph_kernels.h"

namespace heph {

namespace {
constexpr int kGbM = 128, kGbN = 128;
constexpr int kGbChunk = 64;              // bf16 elements per chunk (128 bytes)
constexpr int kGbLd = 144;                // LDS bytes per row
constexpr int kGbGroup = 8;               // tile rows per group

__device__ __forceinline__ bf16x8 lds_frag(const uint8_t* p)
{
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const i32x4*>(p));
}
}  // namespace

__global__ __launch_bounds__(256, 2) void bf16_gemm_kernel(Bf16GemmArgs a)
{
    __shared__ __attribute__((aligned(16))) uint8_t As[2][kGbM * kGbLd];
    __shared__ __attribute__((aligned(16))) uint8_t Bs[2][kGbN * kGbLd];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int r16 = lane & 15, slice = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;
    const int M = a.M, N = a.N, K = a.K, KC = K / kGbChunk;
    const int tiles_m = (M + kGbM - 1) / kGbM, tiles_n = (N + kGbN - 1) / kGbN;
    // grouped order: kGbGroup tile rows sweep each tile column together
    const int bid = blockIdx.x;
    const int width = kGbGroup * tiles_n;
    const int first_m = (bid / width) * kGbGroup;
    const int gsize = min(tiles_m - first_m, kGbGroup);
    const int r = bid % width;
    const int m0 = (first_m + r % gsize) * kGbM, n0 = (r / gsize) * kGbN;

    // global -> LDS staging: 1024 16-byte pieces per operand tile, four per
    // thread; eight consecutive threads cover one 128-byte row chunk. Rows
    // past M (N) are clamped to the last row.
    const int lrow = tid >> 3, lcol = (tid & 7) * 8;    // elements
    const uint16_t* ag[4];
    const uint16_t* bg[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        ag[q] = a.x + (size_t)min(m0 + lrow + 32 * q, M - 1) * K + lcol;
        bg[q] = a.w + (size_t)min(n0 + lrow + 32 * q, N - 1) * K + lcol;
    }
    i32x4 ra[4], rb[4];
    auto gload = [&](int j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            ra[q] = ldg16(ag[q] + (size_t)j * kGbChunk);
            rb[q] = ldg16(bg[q] + (size_t)j * kGbChunk);
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            *reinterpret_cast<i32x4*>(&As[buf][(lrow + 32 * q) * kGbLd + lcol * 2]) = ra[q];
            *reinterpret_cast<i32x4*>(&Bs[buf][(lrow + 32 * q) * kGbLd + lcol * 2]) = rb[q];
        }
    };

    f32x4 acc[4][4];    // [activation row tile][weight column tile]
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
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            // lane (r16, slice): elements ks*32 + slice*8 .. +7 of its row
            const int off = ks * 64 + slice * 16;
            bf16x8 xa[4], wb[4];
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
                xa[mi] = lds_frag(&As[cur][(wm * 64 + mi * 16 + r16) * kGbLd + off]);
#pragma unroll
            for (int ni = 0; ni < 4; ++ni)
                wb[ni] = lds_frag(&Bs[cur][(wn * 64 + ni * 16 + r16) * kGbLd + off]);
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma_bf16(wb[ni], xa[mi], acc[mi][ni]);
        }
        if (j + 1 < KC) lstore(cur ^ 1);
        __syncthreads();
    }

    // lane (r16, slice): row m0 + wm*64 + mi*16 + r16, columns
    // n0 + wn*64 + ni*16 + 4*slice .. +3
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
        const int row = m0 + wm * 64 + mi * 16 + r16;
        if (row >= M) continue;
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            const int col = n0 + wn * 64 + ni * 16 + 4 * slice;
            if (col >= N) continue;
            f32x4 v = acc[mi][ni];
            const size_t o = (size_t)row * N + col;
            if (a.c_f32) {
                f32x4* c = reinterpret_cast<f32x4*>(static_cast<float*>(a.c) + o);
                if (a.residual) v += *c;
                *c = v;
            } else {
                uint2* c = reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.c) + o);
                if (a.residual) {
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
}

hipError_t launch_bf16_gemm(void* c, bool c_f32, bool residual, const uint16_t* x,
                            const uint16_t* w, int M, int N, int K, hipStream_t stream,
                            const LaunchTiming& t, const char** name)
{
    const Bf16GemmArgs a{c, x, w, M, N, K, c_f32, residual};
    const long tiles = (long)((M + kGbM - 1) / kGbM) * ((N + kGbN - 1) / kGbN);
    if (tiles > 0x7fffffffL) return hipErrorInvalidValue;
    *name = "bf16_gemm_128x128";
    return launch(bf16_gemm_kernel, dim3((unsigned)tiles), dim3(256), 0, stream, t, a);
}

}  // namespace heph
