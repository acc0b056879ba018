// bf16_skinny.hip - unquantized bf16 linear for M <= 32 (the lm_head).
//
// Replaces the reference's `linear` decode path for the lm_head
// (src/hephaestus/kernels.mojo:89-121, which calls the third-party MAX
// gemv_gpu for M = 1 and keeps F32 logits). The 151936 x 2560 bf16 weight
// (778 MB) is streamed once: a workgroup owns 16 output columns, its waves
// split K into 128-wide chunks, every lane issues four 16-byte loads per
// chunk, and four v_mfma_f32_16x16x32_bf16 contract the chunk for all M
// rows (rows >= M are zero). Partials are summed through LDS.
#include "heph_kernels.h"

namespace heph {

struct Bf16Args {
    void* c;
    const uint16_t* x;
    const uint16_t* w;
    int M, N, K;
    bool c_f32;
    bool residual;
};

template <int WAVES, int MT, int U>
__global__ __launch_bounds__(WAVES * 64) void bf16_skinny_kernel(Bf16Args a)
{
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r16 = lane & 15, slice = lane >> 4;
    const int M = a.M, N = a.N, K = a.K;
    const int KC = K >> 7;
    const int n0 = blockIdx.x * 16;
    const int per = (KC + WAVES - 1) / WAVES;
    const int kb = min(KC, wave * per);
    const int ke = min(KC, kb + per);
    // Lane (r16, slice) holds elements kk*32 + slice*8 + [0, 8) of a chunk.
    const uint16_t* wp = a.w + (size_t)(n0 + r16) * K + slice * 8;

    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0, 0, 0, 0};

    for (int kc = kb; kc < ke; kc += U) {
        i32x4 b[U][4];
        i32x4 x[U][MT][4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool live = kc + u < ke;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                b[u][kk] = live ? ldg16(wp + (size_t)(kc + u) * kChunk + kk * 32)
                                : i32x4{0, 0, 0, 0};
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int row = mt * 16 + r16;
                const uint16_t* xp = a.x + (size_t)row * K + (kc + u) * kChunk + slice * 8;
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
                    x[u][mt][kk] = (live && row < M) ? ldg16(xp + kk * 32) : i32x4{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (kc + u >= ke) break;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
                    acc[mt] = mfma_bf16(__builtin_bit_cast(bf16x8, x[u][mt][kk]),
                                        __builtin_bit_cast(bf16x8, b[u][kk]), acc[mt]);
        }
    }

    __shared__ float red[WAVES][MT * 4][64];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][mt * 4 + i][lane] = acc[mt][i];
    __syncthreads();
    for (int e = threadIdx.x; e < MT * 256; e += WAVES * 64) {
        const int l = e & 63, idx = e >> 6;
        const int i = idx & 3, mt = idx >> 2;
        const int row = mt * 16 + (l >> 4) * 4 + i;
        const int col = n0 + (l & 15);
        if (row >= M || col >= N) continue;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) v += red[w][idx][l];
        const size_t o = (size_t)row * N + col;
        if (a.c_f32) {
            float* c = static_cast<float*>(a.c);
            c[o] = a.residual ? v + c[o] : v;
        } else {
            uint16_t* c = static_cast<uint16_t*>(a.c);
            if (a.residual) v += __uint_as_float((uint32_t)c[o] << 16);
            c[o] = f32_to_bf16(v);
        }
    }
}

hipError_t launch_bf16_skinny(void* c, bool c_f32, bool residual, const uint16_t* x,
                              const uint16_t* w, int M, int N, int K,
                              hipStream_t stream, const LaunchTiming& t,
                              const char** name)
{
    const Bf16Args a{c, x, w, M, N, K, c_f32, residual};
    const dim3 grid(N / 16);
    if (M <= 16) {
        *name = "bf16_skinny_m16";
        return launch(bf16_skinny_kernel<4, 1, 2>, grid, dim3(256), 0, stream, t, a);
    }
    *name = "bf16_skinny_m32";
    return launch(bf16_skinny_kernel<4, 2, 2>, grid, dim3(256), 0, stream, t, a);
}

}  // namespace heph
