// gemm.hip - W8A8 FP8 GEMM for prefill (any M; chosen for M > 32).
//
// Replaces the reference's prefill kernel wmma_gemm_kernel_v3a_fp8
// (src/hephaestus/wmma_gfx12.mojo:756-888: 64x64 tile, BK=16, single LDS
// buffer, two barriers per 16-wide K step, rank-1 scale epilogue). Two
// kernels: the large-M BMx256 DMA kernel further down (every M while the
// operands' byte offsets fit 32 bits), and first the 128x128 kernel for
// larger operands:
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
#include <algorithm>
#include <type_traits>

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
    // K % 128 != 0 (per-token / per-channel scales only): the last chunk's
    // 16-byte pieces past K are zeros
    const int M = op.M, N = op.N, K = op.K, KC = (K + kChunk - 1) >> 7;
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
        const bool kin = j * kChunk + lcol + 16 <= K;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            ra[r] = aok[r] && kin ? ldg16(ag[r] + (size_t)j * kChunk) : i32x4{0, 0, 0, 0};
            rb[r] = bok[r] && kin ? ldg16(bg[r] + (size_t)j * kChunk) : i32x4{0, 0, 0, 0};
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

    // The block scale of chunk j + 1 is loaded with chunk j + 1's tiles.
    float sw_cur = SM == 0 ? swb[0] : 1.0f, sw_nxt = 1.0f;
    for (int j = 0; j < KC; ++j) {
        const int cur = j & 1;
        if (j + 1 < KC) {
            gload(j + 1);
            if constexpr (SM == 0) sw_nxt = swb[j + 1];
        }

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
            const float swj = sw_cur;
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

        sw_cur = sw_nxt;
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

// ---------------------------------------------------------------------------
// Large-M kernel: BMxBN tile per 512-thread workgroup (8 waves of
// (BM/2)x(BN/4), (BM/32)x(BN/64) MFMA 16x16x128 each). The weight fragment is the
// MFMA's first operand, so lane l holds row l&15 of each 16x16 output block
// at columns 4*(l>>4) .. +3: one activation-scale product per row tile and
// chunk, and four consecutive outputs to pack. Operand tiles reach LDS by
// direct DMA (buffer_load_dwordx4 ... lds, 1 KB = 8 rows per instruction,
// no VGPR staging); a 16-byte piece p of row r lands in slot p ^ (r & 7),
// which spreads the fragment reads over the banks. Stages of A BM*128 B,
// B BN*128 B and row scales BM*4 B (two, or three where LDS allows: see
// BigTile); one barrier per 128-wide chunk:
//   wait own DMA of chunk j -> barrier (chunk j visible everywhere, and
//   every wave is done with the stage read in chunk j-1) -> DMA chunk j+1
//   (j+2 with three stages) into that stage -> contract chunk j.
// The chunk loop is unrolled by the stage count so that each stage's LDS
// addresses are fixed registers plus instruction offsets (the B stage of
// the tiles with three B against two A stages is a run-time base), and
// the DMA advances through K
// with a scalar offset only: apart from the rescale (one FMA per
// accumulator and chunk, one multiply per row tile, or per row tile and
// 16-column block where a wave's columns span two weight blocks) the loop holds almost
// no VALU work, because a wave's VALU instructions do not overlap its own
// MFMAs. The block scales come through the scalar cache.
// The compiler does not model the DMA's LDS writes, so the waits are
// explicit s_waitcnt vmcnt(n) plus compiler memory barriers.
// Epilogue, bf16 output: the tile is rounded (v_cvt_pk_bf16_f32), written to
// LDS once as bf16 (8 bytes per lane and block) and stored as coalesced
// 16-byte row pieces. f32 output or a residual: staged in f32, BM/2 rows at
// a time, the residual added before the one rounding.
namespace {

// Tile BM x BN, BM in {64, 128, 192, 256}, BN in {192, 256, 320}: the 8
// waves form a 2 x 4 grid of (BM/2) x (BN/4) wave tiles. A smaller tile
// trades MFMA work per chunk for a tile count that fills the CUs (e.g. 256
// tiles of 128 x 320 instead of 160 of 256 x 256 at M = 4096, N = 2560).
template <int BM, int BN>
struct BigTile {
    static_assert(BM == 64 || BM == 128 || BM == 192 || BM == 256, "tile height");
    static_assert(BN == 192 || BN == 256 || BN == 320, "tile width");
    // 8 waves in a 2 x 4 grid of WM x WN wave tiles, MT x NT MFMA blocks
    static constexpr int WM = BM / 2, MT = WM / 16, WN = BN / 4, NT = WN / 16;
    // B rows (DMA instructions of 8 rows) per wave
    static constexpr int NBP = BN / 64;
    // the WN columns of every wave lie in one 128-column weight block
    static constexpr bool ONE_BLOCK = 128 % WN == 0 && BN % WN == 0;
    static constexpr int STAGE_A = BM * kChunk, STAGE_B = BN * kChunk, STAGE_S = BM * 4;
    static constexpr int STAGE = STAGE_A + STAGE_B + STAGE_S;
    // LDS stages. A short chunk is below the loaded HBM latency, so where
    // LDS allows, the DMA runs two chunks ahead: three whole stages (64 and
    // 128 rows by 256 columns, 64 x 192); else two A/scale stages and three B stages
    // (the weights, streamed from HBM in a real prefill, get the extra
    // chunk: 192 x 256, 256 x 192, 128 x 320); else two (256 x 256).
    static constexpr int kLds = 160 * 1024;
    static constexpr bool FULL3 = 3 * STAGE <= kLds;
    static constexpr bool SPLIT_B = !FULL3 && 2 * (STAGE_A + STAGE_S) + 3 * STAGE_B <= kLds;
    static constexpr int NS = FULL3 ? 3 : 2;                  // A and row-scale stages
    static constexpr int NB = FULL3 || SPLIT_B ? 3 : 2;       // B stages
    static constexpr int BYTES =
        SPLIT_B ? 2 * STAGE_A + 2 * STAGE_S + 3 * STAGE_B : NS * STAGE;
    // Byte offsets of A, B and row-scale stage k.
    static constexpr int a_at(int k) { return SPLIT_B ? k * STAGE_A : k * STAGE; }
    static constexpr int s_at(int k)
    {
        return SPLIT_B ? 2 * STAGE_A + k * STAGE_S : k * STAGE + STAGE_A + STAGE_B;
    }
    static constexpr int b_at(int k)
    {
        return SPLIT_B ? 2 * STAGE_A + 2 * STAGE_S + k * STAGE_B : k * STAGE + STAGE_A;
    }
};

template <int V>
using ic = std::integral_constant<int, V>;

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw buffer resource over [p, p + 2^31): offsets are byte offsets from p.
// Word 3 = 0x00020000 (32-bit data format, as gfx9 raw buffers need).
__device__ __forceinline__ rsrc_t make_rsrc(const void* p)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, 0x7fffffff, 0x00020000);
}
// 16 (4) bytes per lane from base + voff + soff straight into LDS at
// lds + 16 * lane (4 * lane); lds must be uniform.
__device__ __forceinline__ void dma16(rsrc_t r, uint32_t voff, uint32_t soff, void* lds)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16,
                                             voff, soff, 0, 0);
}
__device__ __forceinline__ void dma4(rsrc_t r, uint32_t voff, uint32_t soff, void* lds)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 4,
                                             voff, soff, 0, 0);
}
// The chunk-start wait of the large-M kernel: the wave's LDS reads and
// scalar loads done (lgkmcnt(0)) and all its vector memory instructions
// but the newest n (vmcnt(n), n = 9, 8, 4 or 0: with three stages the DMA
// of the next chunk may stay in flight).
__device__ __forceinline__ void wait_stage(int n)
{
    switch (n) {
    case 10: __builtin_amdgcn_s_waitcnt(0x007A); break;
    case 9: __builtin_amdgcn_s_waitcnt(0x0079); break;
    case 8: __builtin_amdgcn_s_waitcnt(0x0078); break;
    case 7: __builtin_amdgcn_s_waitcnt(0x0077); break;
    case 6: __builtin_amdgcn_s_waitcnt(0x0076); break;
    case 5: __builtin_amdgcn_s_waitcnt(0x0075); break;
    case 4: __builtin_amdgcn_s_waitcnt(0x0074); break;
    case 3: __builtin_amdgcn_s_waitcnt(0x0073); break;
    default: __builtin_amdgcn_s_waitcnt(0x0070); break;
    }
    asm volatile("" ::: "memory");
}
// Workgroup barrier after wait_stage: every wave's DMA into the stage about
// to be read has landed, and its reads of the stage about to be refilled
// are done. No memory fence (the fence of __syncthreads waits for every
// outstanding DMA, the next chunk's included); the clobber keeps the
// compiler from moving LDS accesses across it.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_barrier" ::: "memory"); }
// Keeps v where the program computes it: the scheduler may not sink the
// rescale FMAs below the next row tile's MFMAs (their partials would then
// all be live at once).
__device__ __forceinline__ void pin(f32x4& v) { asm volatile("" : "+v"(v)); }

typedef const __attribute__((address_space(4))) float* const_f32_ptr;
}  // namespace

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two floats -> two bf16 (round to nearest even) in one v_cvt_pk_bf16_f32;
// equal bit for bit to f32_to_bf16 on non-NaN values (checked on the GPU
// against the f32 output of the same kernel rounded on the host).
__device__ __forceinline__ uint32_t pack_bf16_hw(float a, float b)
{
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
// Epilogue of the large-M kernels: lane l holds C[row r16][cols 4*slice ..
// +3] of each 16x16 block of its (BM/2) x 64 wave tile, already scaled.
// K splits store the fp32 partial tile; bf16 output goes through LDS once
// as bf16 for coalesced 16-byte stores; f32 output or a residual in two
// f32 passes (the residual added before the one rounding). Every thread of
// the workgroup calls it; LDS_BYTES of smem are free to reuse.
template <int SM, int BM, int BN, int LDS_BYTES>
__device__ __forceinline__ void big_epilogue(const Fp8Operands& op,
                                             f32x4 (&acc)[BM / 32][BN / 64], uint8_t* smem,
                                             int m0, int n0, int split, int S)
{
    constexpr int L_BM = BM, L_WM = BM / 2, L_MT = BM / 32;
    constexpr int L_BN = BN, L_WN = BN / 4, L_NT = BN / 64;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, slice = lane >> 4;
    const int wm = wave >> 2, wn = wave & 3;
    const int M = op.M, N = op.N;
    // Lane l holds C[row r16][cols 4*slice .. +3] of each 16x16 block.
    const int r_lane = wm * L_WM + r16;                  // tile row of (mi = 0)
    const int c_lane = wn * L_WN + slice * 4;            // tile col of (ni = 0)
    if constexpr (SM != 2) {
        if (S > 1) {
            // split over K: the fp32 partial tile goes to the scratch
            // [split][M][N]; splitk_reduce_kernel finishes the output.
            float* pp = op.part + (size_t)split * M * N;
#pragma unroll
            for (int mi = 0; mi < L_MT; ++mi) {
                const int row = m0 + r_lane + mi * 16;
                if (row >= M) continue;
#pragma unroll
                for (int ni = 0; ni < L_NT; ++ni) {
                    const int col = n0 + c_lane + ni * 16;
                    if (col < N) *reinterpret_cast<f32x4*>(pp + (size_t)row * N + col) = acc[mi][ni];
                }
            }
            return;
        }
    }
    if (!op.residual && !op.c_f32) {
        // bf16 output: the whole tile goes through LDS once as bf16, rows
        // padded by 8 bytes (2 BN + 8: 130 dwords at 256 columns, consecutive
        // rows 2 banks apart), each lane writing 8 bytes per block; then
        // 16-byte coalesced stores.
        constexpr int RB = 2 * L_BN + 8;
        static_assert(L_BM * RB <= LDS_BYTES, "bf16 tile must fit the stage buffers");
        __syncthreads();
#pragma unroll
        for (int mi = 0; mi < L_MT; ++mi) {
            float sa = 1.0f;
            if constexpr (SM == 2) sa = op.s[min(m0 + r_lane + mi * 16, M - 1)];
#pragma unroll
            for (int ni = 0; ni < L_NT; ++ni) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = acc[mi][ni][e];
                    if constexpr (SM == 2)
                    {
                        // reference association: acc*(sa*sw) at M = 1
                        // (wmma_gfx12.mojo:711-712), (acc*sa)*sw otherwise (:848)
                        const float sw = op.sw[min(n0 + c_lane + ni * 16 + e, N - 1)];
                        v[e] = M == 1 ? v[e] * (sa * sw) : (v[e] * sa) * sw;
                    }
                }
                const uint2 pk = make_uint2(pack_bf16_hw(v[0], v[1]), pack_bf16_hw(v[2], v[3]));
                *reinterpret_cast<uint2*>(smem + (r_lane + mi * 16) * RB +
                                          (c_lane + ni * 16) * 2) = pk;
            }
        }
        __syncthreads();
        for (int e = tid; e < L_BM * (L_BN / 8); e += 512) {
            const int r = e / (L_BN / 8);
            const int c8 = (e % (L_BN / 8)) * 8;
            const int grow = m0 + r, gcol = n0 + c8;
            if (grow >= M || gcol >= N) continue;
            *reinterpret_cast<uint4*>(static_cast<uint16_t*>(op.c) + (size_t)grow * N + gcol) =
                *reinterpret_cast<const uint4*>(smem + r * RB + c8 * 2);
        }
        return;
    }
    // f32 output or residual: two passes of L_WM rows through LDS in f32
    // (the residual is added before the one rounding).
    constexpr int CST = L_BN + 4;
    static_assert(L_WM * CST * 4 <= LDS_BYTES, "epilogue tile must fit the stage buffers");
    float* Cs = reinterpret_cast<float*>(smem);
    float* cw = Cs + r16 * CST + c_lane;
    for (int pass = 0; pass < 2; ++pass) {
        __syncthreads();
        if (wm == pass) {
#pragma unroll
            for (int mi = 0; mi < L_MT; ++mi)
#pragma unroll
                for (int ni = 0; ni < L_NT; ++ni)
                    *reinterpret_cast<f32x4*>(cw + mi * 16 * CST + ni * 16) = acc[mi][ni];
        }
        __syncthreads();
        // L_WM rows x L_BN cols: each thread writes 8 consecutive outputs
        for (int e = tid; e < L_WM * (L_BN / 8); e += 512) {
            const int r = e / (L_BN / 8);
            const int c8 = (e % (L_BN / 8)) * 8;
            const int grow = m0 + pass * L_WM + r;
            const int gcol = n0 + c8;
            if (grow >= M || gcol >= N) continue;
            const f32x4 lo = *reinterpret_cast<const f32x4*>(&Cs[r * CST + c8]);
            const f32x4 hi = *reinterpret_cast<const f32x4*>(&Cs[r * CST + c8 + 4]);
            float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            if constexpr (SM == 2) {
                // reference association: acc*(sa*sw) at M = 1, else (acc*sa)*sw
                const float sa = op.s[grow];
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    v[t] = M == 1 ? v[t] * (sa * op.sw[gcol + t]) : (v[t] * sa) * op.sw[gcol + t];
            }
            const size_t o = (size_t)grow * N + gcol;
            if (op.c_f32) {
                float* c = static_cast<float*>(op.c) + o;
                if (op.residual) {
                    const float4 r0 = *reinterpret_cast<const float4*>(c);
                    const float4 r1 = *reinterpret_cast<const float4*>(c + 4);
                    v[0] += r0.x; v[1] += r0.y; v[2] += r0.z; v[3] += r0.w;
                    v[4] += r1.x; v[5] += r1.y; v[6] += r1.z; v[7] += r1.w;
                }
                *reinterpret_cast<float4*>(c) = make_float4(v[0], v[1], v[2], v[3]);
                *reinterpret_cast<float4*>(c + 4) = make_float4(v[4], v[5], v[6], v[7]);
            } else {
                uint16_t* c = static_cast<uint16_t*>(op.c) + o;
                const uint4 rr = *reinterpret_cast<const uint4*>(c);
                v[0] += bf16lo(rr.x); v[1] += bf16hi(rr.x);
                v[2] += bf16lo(rr.y); v[3] += bf16hi(rr.y);
                v[4] += bf16lo(rr.z); v[5] += bf16hi(rr.z);
                v[6] += bf16lo(rr.w); v[7] += bf16hi(rr.w);
                uint4 out;
                out.x = f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
                out.y = f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
                out.z = f32_to_bf16(v[4]) | ((uint32_t)f32_to_bf16(v[5]) << 16);
                out.w = f32_to_bf16(v[6]) | ((uint32_t)f32_to_bf16(v[7]) << 16);
                *reinterpret_cast<uint4*>(c) = out;
            }
        }
    }
}

template <int SM, int BM, int BN>
__global__ __launch_bounds__(512, 1) void fp8_gemm256_kernel(Fp8Operands op)
{
    using T = BigTile<BM, BN>;
    constexpr int L_BM = BM, L_WM = T::WM, L_MT = T::MT;
    constexpr int L_BN = BN, L_WN = T::WN, L_NT = T::NT, NBP = T::NBP;
    // With three stages, chunk j + 2's DMA goes out in chunk j: a chunk
    // (~0.8 us at 64 rows, ~1.3 us at 192) is below the loaded HBM latency,
    // and weights that are not in the Infinity Cache (each layer of a real
    // prefill) otherwise left every chunk waiting on its DMA (MI355X: M =
    // 512 qkv 16.4 us from the cache, 29.5 us from HBM with two stages).
    constexpr int NS = T::NS, NB = T::NB;
    constexpr bool SPLIT_B = T::SPLIT_B;
    // The kernel's only LDS variable: with a second one the LDS accesses get
    // alias scopes, the compiler then orders every fragment read after all
    // outstanding DMA (vmcnt(0)), and the pipeline serializes (MI355X: +40 %
    // per chunk). Extra LDS state goes into this array.
    __shared__ __attribute__((aligned(16))) uint8_t smem[T::BYTES];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, slice = lane >> 4;
    const int wm = wave >> 2, wn = wave & 3;
    const int M = op.M, N = op.N, K = op.K, KC = K >> 7;
    const int tiles_m = (M + L_BM - 1) / L_BM, tiles_n = (N + L_BN - 1) / L_BN;
    // Split over K: workgroup b takes tile b % tiles and the chunks
    // [split * KC / S, (split + 1) * KC / S) of split b / tiles.
    const int S = op.splits, tiles = tiles_m * tiles_n;
    const int split = blockIdx.x / tiles;
    const int jb = split * KC / S, je = (split + 1) * KC / S;
    int tm, tn;
    tile_of_block(blockIdx.x - split * tiles, tiles_m, tiles_n, &tm, &tn);
    const int m0 = tm * L_BM, n0 = tn * L_BN;

    // DMA sources: wave w moves operand rows [32w, 32w+32) of A (4
    // instructions) and [8 NBP w, 8 NBP (w+1)) of B (NBP = BN / 64
    // instructions); lane i covers row 8q + (i >> 3) of block q and global
    // piece (i & 7) ^ (row & 7). Rows past M (N) are clamped to the last
    // row: they feed output rows (columns) that are never stored. Each lane
    // keeps one 32-bit byte offset per block and operand; chunk j adds the
    // scalar offset 128 * j.
    const rsrc_t rq = make_rsrc(op.q), rw = make_rsrc(op.w), rs = make_rsrc(op.s);
    const int lr = lane >> 3;
    const int piece = ((lane & 7) ^ lr) * 16;     // rows 8q + lr share r & 7 = lr
    uint32_t aoff[4], boff[NBP];
#pragma unroll
    for (int q = 0; q < 4; ++q)
        aoff[q] = (uint32_t)min(m0 + wave * 32 + q * 8 + lr, M - 1) * (uint32_t)K + piece;
#pragma unroll
    for (int q = 0; q < NBP; ++q)
        boff[q] = (uint32_t)min(n0 + wave * 8 * NBP + q * 8 + lr, N - 1) * (uint32_t)K + piece;
    const uint32_t soff = (uint32_t)min(m0 + wave * 64 + lane, M - 1) * (uint32_t)op.s_ld * 4u;
    const uint32_t s_step = (uint32_t)op.s_step * 4u;

    // DMA instruction `part` (0 .. 4 + NBP) of this wave: parts 0-3 move A
    // rows of chunk ja into A stage abuf, then NBP parts B rows of chunk jw
    // into B stage bbuf and the last the row scales of chunk ja; with
    // separate B stages the row scales come fourth (part 4) and the B rows
    // last, so that the next chunk's wait can leave exactly the NBP B
    // instructions in flight.
    constexpr int kParts = 5 + NBP;
    constexpr int kFirstB = SPLIT_B ? 5 : 4, kScalePart = SPLIT_B ? 4 : 4 + NBP;
    // DMA parts per row tile (MI355X: 2 over the first five of 8 row tiles,
    // 3 over the first three of 6 or 4, fewest cycles per chunk; 5 and 4
    // over the 2 row tiles of BM = 64, so that every part goes out)
    constexpr int kPer = L_MT >= 8 ? 2 : L_MT >= 4 ? 3 : (kParts + L_MT - 1) / L_MT;
    static_assert(kPer * L_MT >= kParts, "every DMA part is issued");
    auto issue_part = [&](int ja, int jw, auto abufc, int bbuf, int part) {
        constexpr int abuf = decltype(abufc)::value;
        if (part < 4) {
            if (wave * 32 < L_BM)
                dma16(rq, aoff[part], (uint32_t)ja * kChunk,
                      smem + T::a_at(abuf) + (wave * 32 + part * 8) * kChunk);
        } else if (part == kScalePart) {
            if (SM != 2 && wave * 64 < L_BM)
                dma4(rs, soff, (uint32_t)ja * s_step, smem + T::s_at(abuf) + wave * 256);
        } else {
            const int q = part - kFirstB;
            dma16(rw, boff[q], (uint32_t)jw * kChunk,
                  smem + T::b_at(bbuf) + (wave * 8 * NBP + q * 8) * kChunk);
        }
    };

    // With the weight fragment as the MFMA's first operand, lane l holds
    // row r16 of each 16x16 block and its columns 4*slice .. 4*slice+3.
    float swc[L_NT][4];
#pragma unroll
    for (int ni = 0; ni < L_NT; ++ni)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int n = min(n0 + wn * L_WN + ni * 16 + slice * 4 + e, N - 1);
            swc[ni][e] = SM == 1 ? op.sw[n] : 0.0f;
        }
    // A wave whose columns all lie past N still reads a valid scale row
    // (its results are never stored). The rows are uniform per wave: the
    // block scales are scalar loads. Where a wave's columns span two
    // 128-column blocks (WN = 48 or 80), each 16-column block ni has its own.
    constexpr int NSW = T::ONE_BLOCK ? 1 : L_NT;
    const_f32_ptr swb[NSW];
#pragma unroll
    for (int k = 0; k < NSW; ++k)
        swb[k] = (const_f32_ptr)(op.sw + (size_t)min((n0 + wn * L_WN + k * 16) >> 7, (N - 1) >> 7) *
                                             op.sw_ld);

    // Per-lane LDS byte offsets inside a stage: fragment rows of A and B at
    // the two 16-byte slots this lane reads, and the row scale.
    const int sl0 = (slice ^ (r16 & 7)) * 16, sl1 = sl0 ^ 64;
    const int a_row = (wm * L_WM + r16) * kChunk;
    const int b_row = (wn * L_WN + r16) * kChunk;
    const int s_row = (wm * L_WM + r16) * 4;

    f32x4 acc[L_MT][L_NT];
#pragma unroll
    for (int mi = 0; mi < L_MT; ++mi)
#pragma unroll
        for (int ni = 0; ni < L_NT; ++ni) acc[mi][ni] = f32x4{0, 0, 0, 0};

    float sw_cur[NSW], sw_nxt[NSW];
#pragma unroll
    for (int k = 0; k < NSW; ++k) {
        sw_cur[k] = SM == 0 ? swb[k][jb] : 1.0f;
        sw_nxt[k] = 1.0f;
    }

    // Software pipeline over the row tiles of a wave: the MFMAs of tile mi
    // run while the rescale FMAs of tile mi - 1 execute and the A fragment
    // and row scale of tile mi + 1 are read. The last tile's FMAs are done
    // at the start of the next chunk, so its partials and scale product
    // live across the barrier.
    static_assert(L_MT % 2 == 0, "row tiles per wave must be even");
    f32x4 p[2][L_NT];
    float sc[2][NSW] = {};
    auto rescale = [&](int mi, int slot) {
#pragma unroll
        for (int ni = 0; ni < L_NT; ++ni) {
            const float s = sc[slot][NSW == 1 ? 0 : ni];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                acc[mi][ni][e] += p[slot][ni][e] * (SM == 0 ? s : s * swc[ni][e]);
            pin(acc[mi][ni]);
        }
    };

    // DMA instructions a wave issues per chunk (A rows, B rows, row scales).
    const int n_parts = (wave * 32 < L_BM ? 4 : 0) + NBP + (SM != 2 && wave * 64 < L_BM ? 1 : 0);

    // One 128-wide chunk j held in A stage buf (a compile-time constant)
    // and B stage bst. The wave's nine DMA instructions (A rows and scales
    // of chunk j + NS - 1, B rows of chunk j + NB - 1) go out kPer per row
    // tile from the first tile on: issued together right after the barrier,
    // the DMAs of all eight waves stall every wave's instruction issue;
    // spread to the last tile, the late ones are still in flight at the
    // next chunk's wait (MI355X: ~350 of ~3100 cycles a chunk).
    auto chunk = [&](auto bufc, int j, int bst) {
        constexpr int buf = decltype(bufc)::value;
        // with three stages the newest instructions, the next chunk's DMA
        // (all nine parts, or its four B parts with three B stages), may
        // stay in flight; with two, everything lands
        wait_stage(NB == 3 && j + 1 < je ? (SPLIT_B ? NBP : n_parts) : 0);
        stage_barrier();
        const bool more = j + 1 < je;
        const int ja = j + NS - 1, jw = j + NB - 1;
        const int bnext = SPLIT_B ? (bst == 0 ? 2 : bst - 1) : (buf + NB - 1) % NB;
        const uint8_t* sta = smem + T::a_at(buf);
        const uint8_t* sts = smem + T::s_at(buf);
        const uint8_t* stb = smem + T::b_at(bst);
        auto frag = [&](const uint8_t* st, int row_off) {
            return join(*reinterpret_cast<const i32x4*>(st + row_off + sl0),
                        *reinterpret_cast<const i32x4*>(st + row_off + sl1));
        };
        i32x8 b[L_NT];
#pragma unroll
        for (int ni = 0; ni < L_NT; ++ni) b[ni] = frag(stb, b_row + ni * 16 * kChunk);
        float swj[NSW];
#pragma unroll
        for (int k = 0; k < NSW; ++k) swj[k] = sw_cur[k];
        i32x8 a_[2];
        float sa_[2];
        a_[0] = frag(sta, a_row);
        sa_[0] = *reinterpret_cast<const float*>(sts + s_row);
        if constexpr (SM == 0) {
            if (more) {
#pragma unroll
                for (int k = 0; k < NSW; ++k) sw_nxt[k] = swb[k][j + 1];
            }
        }
#pragma unroll
        for (int k = 0; k < NSW; ++k) sw_cur[k] = sw_nxt[k];
#pragma unroll
        for (int mi = 0; mi < L_MT; ++mi) {
            const int cur = mi & 1, prv = cur ^ 1;
            if (mi + 1 < L_MT) {
                a_[prv] = frag(sta, a_row + (mi + 1) * 16 * kChunk);
                sa_[prv] = *reinterpret_cast<const float*>(sts + s_row + (mi + 1) * 64);
            }
            // Waves 4-7 (the second wave of each SIMD) win instruction issue
            // over the first half of the row tiles. Left to the oldest-first
            // arbiter, waves 0-3 finish every chunk ~600 cycles early and the
            // late waves then run alone up to the barrier, with no MFMA of
            // the other wave to hide their VALU work (MI355X: 1.5-3.5 % per
            // shape at M = 4096).
            if (wave >= 4) {
                if (mi == 0) __builtin_amdgcn_s_setprio(1);
                if (mi == L_MT / 2) __builtin_amdgcn_s_setprio(0);
            }
#pragma unroll
            for (int part = 0; part < kParts; ++part) {
                if (part / kPer != mi) continue;
                // the B parts stay behind the A and scale parts in issue
                // order (the next chunk's wait relies on it)
                if (SPLIT_B && part == kFirstB) __builtin_amdgcn_sched_barrier(0);
                if ((part >= kFirstB && part != kScalePart ? jw : ja) < je)
                    issue_part(ja, jw, ic<(buf + NS - 1) % NS>{}, bnext, part);
            }
            if constexpr (SM == 2) {
#pragma unroll
                for (int ni = 0; ni < L_NT; ++ni)
                    acc[mi][ni] = mfma_e4m3(b[ni], a_[cur], acc[mi][ni]);
            } else {
#pragma unroll
                for (int k = 0; k < NSW; ++k) sc[cur][k] = sa_[cur] * swj[k];
#pragma unroll
                for (int ni = 0; ni < L_NT; ++ni)
                    p[cur][ni] = mfma_e4m3(b[ni], a_[cur], f32x4{0, 0, 0, 0});
                if (mi > 0) rescale(mi - 1, prv);
                else if (j > jb) rescale(L_MT - 1, prv);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

#pragma unroll
    for (int part = 0; part < kParts; ++part) issue_part(jb, jb, ic<0>{}, 0, part);
    int j = jb;
    if constexpr (SPLIT_B) {
        // chunk jb + 1's B rows, last in issue order
        if (jb + 1 < je) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int q = 0; q < NBP; ++q) issue_part(jb, jb + 1, ic<0>{}, 1, kFirstB + q);
        }
    }
    if constexpr (NB == 2) {
        for (; j + 1 < je; j += 2) {
            chunk(ic<0>{}, j, 0);
            chunk(ic<1>{}, j + 1, 1);
        }
        if (j < je) chunk(ic<0>{}, j, 0);
    } else if constexpr (NS == 3) {
        if (jb + 1 < je) {
#pragma unroll
            for (int part = 0; part < kParts; ++part) issue_part(jb + 1, jb + 1, ic<1>{}, 1, part);
        }
        for (; j + 2 < je; j += 3) {
            chunk(ic<0>{}, j, 0);
            chunk(ic<1>{}, j + 1, 1);
            chunk(ic<2>{}, j + 2, 2);
        }
        if (j < je) chunk(ic<0>{}, j, 0);
        if (j + 1 < je) chunk(ic<1>{}, j + 1, 1);
    } else {
        // two A stages, three B stages (the B stage index runs at run time)
        int bst = 0;
        for (; j + 1 < je; j += 2) {
            chunk(ic<0>{}, j, bst);
            bst = bst == 2 ? 0 : bst + 1;
            chunk(ic<1>{}, j + 1, bst);
            bst = bst == 2 ? 0 : bst + 1;
        }
        if (j < je) chunk(ic<0>{}, j, bst);
    }
    if constexpr (SM != 2) rescale(L_MT - 1, (L_MT - 1) & 1);

    big_epilogue<SM, BM, BN, T::BYTES>(op, acc, smem, m0, n0, split, S);
}

// Sums the K-split partials of the large-M GEMM in split order, adds the
// residual and stores bf16 or f32 (four outputs per thread; N % 16 == 0).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(Fp8Operands op)
{
    const size_t mn = (size_t)op.M * op.N, n4 = mn / 4;
    const f32x4* part = reinterpret_cast<const f32x4*>(op.part);
    for (size_t i = blockIdx.x * (size_t)256 + threadIdx.x; i < n4;
         i += (size_t)gridDim.x * 256) {
        f32x4 v = part[i];
        for (int s = 1; s < op.splits; ++s) v += part[(size_t)s * n4 + i];
        if (op.c_f32) {
            f32x4* c = static_cast<f32x4*>(op.c) + i;
            if (op.residual) v += *c;
            *c = v;
        } else {
            uint2* c = static_cast<uint2*>(op.c) + i;
            if (op.residual) {
                const uint2 r = *c;
                v[0] += bf16lo(r.x);
                v[1] += bf16hi(r.x);
                v[2] += bf16lo(r.y);
                v[3] += bf16hi(r.y);
            }
            *c = make_uint2(pack_bf16_hw(v[0], v[1]), pack_bf16_hw(v[2], v[3]));
        }
    }
}

hipError_t launch_splitk_reduce(const Fp8Operands& op, hipStream_t stream, const LaunchTiming& t)
{
    const size_t n4 = (size_t)op.M * op.N / 4;
    const int blocks = (int)std::min<size_t>((n4 + 255) / 256, 4096);
    return launch(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, stream, t, op);
}

namespace {

template <int BM, int BN>
hipError_t launch_big(const Fp8Operands& op, hipStream_t stream, const LaunchTiming& t)
{
    const int tiles = ((op.M + BM - 1) / BM) * ((op.N + BN - 1) / BN);
    const dim3 grid(tiles * op.splits);
    if (op.splits > 1) {
        // the GEMM carries the start stamp, the reduction the stop stamp
        hipError_t e;
        if (op.w_block)
            e = launch(fp8_gemm256_kernel<0, BM, BN>, grid, dim3(512), 0, stream,
                       LaunchTiming{t.start, nullptr}, op);
        else
            e = launch(fp8_gemm256_kernel<1, BM, BN>, grid, dim3(512), 0, stream,
                       LaunchTiming{t.start, nullptr}, op);
        if (e != hipSuccess) return e;
        return launch_splitk_reduce(op, stream, LaunchTiming{nullptr, t.stop});
    }
    if (op.w_block)
        return launch(fp8_gemm256_kernel<0, BM, BN>, grid, dim3(512), 0, stream, t, op);
    if (op.s_step == 0)
        return launch(fp8_gemm256_kernel<2, BM, BN>, grid, dim3(512), 0, stream, t, op);
    return launch(fp8_gemm256_kernel<1, BM, BN>, grid, dim3(512), 0, stream, t, op);
}

}  // namespace

// Measured cost per tile (MI355X shader cycles at ~1.9 GHz, random E4M3
// data, weights from HBM): `chunk` per 128-wide chunk and `fixed` per
// workgroup (prologue, epilogue), fitted to the GEMM-only times of the
// config-1 shapes at M = 4096 (o_proj and down: one round of tiles each,
// K = 4096 against 9728); 64 x 256 fitted to M = 512. A bigger tile does
// more MFMA work per chunk, a smaller one fills the CUs in finer steps: at
// M = 4096 the fit ranks the tiles as measured on every config-1 shape
// (qkv 256 x 192 72.6 us against 75.7 at 256 x 256; o_proj 128 x 320 46.5
// against 47.9 at 192 x 256; gate_up 256 x 256 193.0 against 212.2; down
// 128 x 320 100.4 against 104.4), and at M = 512 as well (64 x 192 for qkv,
// 256 tiles, one round: 18.7 against 21.6 us at 64 x 256; 64 x 256 with 3 K
// splits for o_proj; 128 x 320 for gate_up; 128 x 256 with 6 splits for
// down). 64 x 192 is fitted to M = 512 qkv alone.
struct TileCost {
    int bm, bn;
    long chunk, fixed;
};
constexpr TileCost kTileCost[] = {{256, 256, 2535, 16730}, {256, 192, 2569, 11650},
                                  {192, 256, 2440, 12930}, {128, 320, 2327, 13880},
                                  {128, 256, 1734, 9887},  {64, 256, 1550, 7000},
                                  {64, 192, 1300, 6000}};

// Estimated time (us) of the large-M GEMM with tile tc and s K splits:
// rounds of (tile, split) workgroups over the CUs (one 512-thread
// workgroup per CU) times a workgroup's cost (its chunks and the fixed
// part) at ~1.9 GHz; a split adds the reduction: ~8 us of launch and
// per-workgroup set-up, and the partials (M*N*4 bytes a split) read back
// at ~5 TB/s.
static double gemm_estimate(int M, int N, int K, const TileCost& tc, int s, long cus)
{
    const long tiles = (long)((M + tc.bm - 1) / tc.bm) * ((N + tc.bn - 1) / tc.bn);
    const int KC = K / kChunk;
    const long rounds = (tiles * s + cus - 1) / cus;
    double t = (double)rounds * ((double)((KC + s - 1) / s) * tc.chunk + tc.fixed) / 1900.0;
    if (s > 1) t += 8.0 + (double)s * M * N * 4.0 / 5.0e6;
    return t;
}

// Tile and K splits of the large-M GEMM: the pair with the least estimated
// time, splitting only when allowed, into at most 8 splits of at least 4
// chunks; ties go to the earlier tile of kTileCost, then to fewer splits.
// A forced tile height (gemm_bm) or width (gemm_bn) keeps only the tiles
// that have it.
GemmPlan gemm_plan(int M, int N, int K, bool can_split, int forced_bm, int forced_bn)
{
    // MI355X's 256 CUs, not the visible count: the plan (and the K-split
    // summation order with it) does not change under a CU mask or partition
    const long cus = kPlanCUs;
    const int KC = K / kChunk;
    GemmPlan best{0, 0, 1};
    double best_t = -1.0;
    for (const auto& tc : kTileCost) {
        // 64 x 192 only where its fit holds (M >= 256): below, the K-split
        // plans of the small-M routes stay with the tiles they were measured on
        if (tc.bm == 64 && tc.bn == 192 && M < 256 && forced_bn != 192) continue;
        if (forced_bm >= 64 && tc.bm != forced_bm) continue;
        if (forced_bn && tc.bn != forced_bn) continue;
        for (int s = 1; s <= (can_split ? 8 : 1); ++s) {
            if (s > 1 && KC / s < 4) break;
            const double t = gemm_estimate(M, N, K, tc, s, cus);
            if (best_t < 0.0 || t < best_t) {
                best_t = t;
                best = GemmPlan{tc.bm, tc.bn, s};
            }
        }
    }
    if (best.bm == 0) best = GemmPlan{forced_bm >= 64 ? forced_bm : 256, 256, 1};
    return best;
}

bool gemm_splits_ready(const Fp8Operands& op)
{
    if (!op.part || op.s_step == 0) return false;
    const int s = gemm_plan(op.M, op.N, op.K, true, op.tune.gemm_bm, op.tune.gemm_bn).splits;
    return s > 1 && op.part_bytes >= (size_t)s * op.M * op.N * 4;
}

size_t gemm_split_bytes(int M, int N, int K)
{
    const int s = gemm_plan(M, N, K, true).splits;
    return s > 1 ? (size_t)s * M * N * 4 : 0;
}

hipError_t launch_fp8_gemm(const Fp8Operands& op, hipStream_t stream,
                           const LaunchTiming& t, const char** name)
{
    // The DMA kernel (tiles of 192-320 columns) for every M (N % 16 == 0
    // keeps every 8-wide output group inside the row), splitting K when its
    // tiles leave CUs idle; its 32-bit operand offsets need M*K and N*K below
    // 2^31, else the 128x128 kernel. (Without splits the two run alike below
    // M = 128; the DMA kernel is 1.3-2x faster from there on, MI355X.)
    const bool small_offsets = (long)op.M * op.K < (1L << 31) && (long)op.N * op.K < (1L << 31);
    const bool force_128 = op.tune.gemm_bm == 1;
    if (small_offsets && !force_128) {
        // K splits when the caller's scratch holds their partials (block or
        // per-channel weights with per-chunk activation scales).
        Fp8Operands o = op;
        const GemmPlan plan = gemm_plan(o.M, o.N, o.K, gemm_splits_ready(o), o.tune.gemm_bm,
                                        o.tune.gemm_bn);
        o.splits = plan.splits;
        const bool sk = o.splits > 1;
        if (plan.bn == 192 && plan.bm == 64) {
            *name = sk ? "fp8_gemm_64x192_splitk" : "fp8_gemm_64x192";
            return launch_big<64, 192>(o, stream, t);
        }
        if (plan.bn == 192) {
            *name = sk ? "fp8_gemm_256x192_splitk" : "fp8_gemm_256x192";
            return launch_big<256, 192>(o, stream, t);
        }
        if (plan.bn == 320) {
            *name = sk ? "fp8_gemm_128x320_splitk" : "fp8_gemm_128x320";
            return launch_big<128, 320>(o, stream, t);
        }
        switch (plan.bm) {
        case 64:
            *name = sk ? "fp8_gemm_64x256_splitk" : "fp8_gemm_64x256";
            return launch_big<64, 256>(o, stream, t);
        case 128:
            *name = sk ? "fp8_gemm_128x256_splitk" : "fp8_gemm_128x256";
            return launch_big<128, 256>(o, stream, t);
        case 192:
            *name = sk ? "fp8_gemm_192x256_splitk" : "fp8_gemm_192x256";
            return launch_big<192, 256>(o, stream, t);
        default:
            *name = sk ? "fp8_gemm_256x256_splitk" : "fp8_gemm_256x256";
            return launch_big<256, 256>(o, stream, t);
        }
    }
    const int tiles = ((op.M + BM - 1) / BM) * ((op.N + BN - 1) / BN);
    *name = "fp8_gemm_128x128";
    if (op.w_block)
        return launch(fp8_gemm_kernel<0>, dim3(tiles), dim3(256), 0, stream, t, op);
    if (op.s_step == 0)
        return launch(fp8_gemm_kernel<2>, dim3(tiles), dim3(256), 0, stream, t, op);
    return launch(fp8_gemm_kernel<1>, dim3(tiles), dim3(256), 0, stream, t, op);
}

}  // namespace heph
