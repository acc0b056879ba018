// gemv_split.hip - W8A8 FP8 linear for batched decode (M <= 32) as one
// launch of 64-column workgroups over K splits.
//
// Replaces the reference's small-M kernel (src/hephaestus/wmma_gfx12.mojo:
// 900-1019, reached through linear_fp8, kernels.mojo:410-470) at the batch
// sizes where the chunk-slot GEMV's 16-column workgroups re-read the whole
// activation matrix for every 16 output columns: at M = 32 that is four
// times the weight bytes each workgroup streams. Here a workgroup covers 64
// columns and at most 8 K chunks, so the activation bytes it reads are a
// fraction of its weight bytes, and the K splits supply the workgroups that
// a 64-column grid alone would not (N = 2560: 40 tiles).
//   * workgroup b takes column tile b % tiles_n and chunks [s*KC/S,
//     (s+1)*KC/S) of split s = b / tiles_n; wave w its 16 columns
//     n0 + 16w .. +15;
//   * load order: first the workgroup's activation slice (fused: the bf16
//     rows; otherwise codes and scales from the workspace; either way
//     L2-resident), then the wave's weight fragments for every chunk of the
//     split (two 16-byte loads per lane and chunk, all in flight at once).
//     Memory counters retire in issue order, so staging the activations
//     waits for the activation loads only, and each chunk's MFMAs wait for
//     that chunk's weights while later chunks are still arriving;
//   * staging: fused, eight lanes per 1x128 group load 16 bf16 each, take
//     the group amax (bf16 magnitude bits, NaN skipped, DPP across the 8
//     lanes) and the division-free group scale, and write one 16-byte code
//     piece each; column tile 0 also writes the codes and scales to the
//     workspace. Rows of 128 bytes in LDS, piece index XORed with the
//     row's low bits;
//   * per chunk and 16-row tile one v_mfma_f32_16x16x128_f8f6f4 with the
//     weights as the first operand: lane (r, g) (r = lane & 15,
//     g = lane >> 4) holds C[column 4g+e][activation row r], so it needs
//     one activation scale per tile and chunk; acc += p * (sa * sw), the
//     association of the other kernels of this library;
//   * one split: bf16/f32 output (plus the residual) directly, four
//     columns per lane. More than 3 splits: every split stores fp32
//     partials [split][M][N] and the large-M GEMM's reduction kernel sums
//     them in split order. 2 or 3 splits, in the same launch: splits
//     0..S-2 store fp32 partials [split][M][N] in the caller's scratch and
//     then their tile's completion flag, set to the call's 64-bit epoch
//     (both written through to the coherent level, the flag after the
//     partials have completed). Split S-1 holds the tile's highest workgroup index,
//     so it is dispatched after every workgroup it waits for: it polls the
//     S-1 flags, sums the partials in split order with its own sum last
//     (the order of the large-M GEMM's reduction kernel), adds the
//     residual, stores, and clears the flags. Flags left by earlier calls
//     hold other epochs; a replayed HIP graph repeats one epoch, and the
//     clearing puts the flags back into the waiting state between replays.
//     The wait is bounded. When it gives up, the last split swaps a
//     give-up mark into each flag it did not see (a flag that arrived in
//     between is taken back to the waiting state instead), writes NaN to
//     the tile, and counts the tile in the status word at the end of the
//     caller's workspace; a split that later finds the give-up mark in its
//     flag's place puts the flag back to the waiting state. So when the
//     launch ends every flag is waiting again: no later call, and no graph
//     replay of an earlier epoch, can take a stale flag for its own.

#include <atomic>
#include <chrono>
#include <random>

#include "heph_kernels.h"

namespace heph {

namespace {

constexpr int kSplitCols = 64;     // output columns per workgroup (4 waves x 16)
constexpr int kSplitMaxKB = 8;     // chunks per split at most
// Polls of a completion flag before the last split gives up: each poll is
// a load from the coherent level (~1 us) and a ~128-cycle sleep, so about
// a quarter to half a second in all.
constexpr int kSpinLimit = 1 << 18;
// Split counts up to this sum their partials inside the launch (the last
// split of a tile waits for the others); larger counts store every split's
// partials and leave the sum to the reduction kernel. On MI355X at M = 32
// the in-launch sum saved ~2 us at 3 splits (qkv) and lost 1-2 us at 4 and
// 10 (o_proj, down), where one workgroup per tile reads all the partials.
constexpr int kInLaunchMaxSplits = 3;
// A flag whose waiting split gave up (never an epoch: next_epoch skips it).
constexpr uint64_t kSplitGaveUp = 0xB5AD4ECEDA1CE2A9ull;
}  // namespace

// Max over each aligned run of 8 lanes (unsigned), left in all 8.
__device__ __forceinline__ uint32_t max8_lanes(uint32_t m)
{
    m = max(m, (uint32_t)__builtin_amdgcn_mov_dpp((int)m, 0xB1, 0xf, 0xf, false));   // l ^ 1
    m = max(m, (uint32_t)__builtin_amdgcn_mov_dpp((int)m, 0x4E, 0xf, 0xf, false));   // l ^ 2
    m = max(m, (uint32_t)__builtin_amdgcn_mov_dpp((int)m, 0x141, 0xf, 0xf, false));  // 7 - l
    return m;
}

// Byte offset of 16-byte piece p (0..7) of activation row r (0..31) of
// chunk c in the LDS code tile: rows of 128 bytes, the piece index XORed
// with r & 7 so that the 16 rows a fragment read touches fall in
// different banks.
__device__ __forceinline__ int code_off(int c, int r, int p)
{
    return ((c * 32 + r) * 8 + (p ^ (r & 7))) * 16;
}

// Cross-workgroup traffic of the split reduction. On gfx950 each XCD has
// its own L2, not coherent with the others, and a device-scope fence
// writes back or invalidates the whole L2; instead the partials and flags
// move with relaxed device-scope atomic stores and loads (sc1: written
// through to, and read from, the coherent level), ordered by waiting for
// this wave's vector memory operations to complete.
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void store_through(float* p, const f32x4& v)
{
    uint64_t* q = reinterpret_cast<uint64_t*>(p);
    __hip_atomic_store(q, __builtin_bit_cast(uint64_t, f32x2{v[0], v[1]}), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 1, __builtin_bit_cast(uint64_t, f32x2{v[2], v[3]}), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ f32x4 load_through(const float* p)
{
    const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
    const f32x2 lo = __builtin_bit_cast(
        f32x2, __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const f32x2 hi = __builtin_bit_cast(
        f32x2, __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    return f32x4{lo[0], lo[1], hi[0], hi[1]};
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt not waited for): every vector
// memory operation this wave issued has completed.
__device__ __forceinline__ void wait_vmem()
{
    __builtin_amdgcn_s_waitcnt(0x0F70);
}

// Completion flags of a split plan (S > 1): one 64-bit word per split
// 0..S-2 and column tile, after the S-1 partial slices [split][M][N].
__device__ __forceinline__ uint64_t* split_flags(const Fp8Operands& op, int S)
{
    return reinterpret_cast<uint64_t*>(op.part + (size_t)(S - 1) * op.M * op.N);
}
// Count of tiles whose wait gave up: the last 8-byte-aligned word of the
// scratch (HEPH_SPLIT_STATUS_OFFSET of the caller's q_ws_bytes).
__device__ __forceinline__ uint64_t* split_status(const Fp8Operands& op)
{
    return reinterpret_cast<uint64_t*>(reinterpret_cast<uint8_t*>(op.part) +
                                       ((op.part_bytes - 8) & ~(size_t)7));
}

// MT: 16-row tiles (1: M <= 16, 2: M <= 32). SM: 0 = 128x128 weight
// blocks, 1 = per-channel weights (both with per-chunk activation scales).
// FUSED: quantize the bf16 activations of the workgroup's chunks into LDS
// (workgroups of column tile 0 also write the codes and scales to the
// workspace); otherwise copy the codes and scales from the workspace.
template <int MT, int SM, bool FUSED>
__global__ __launch_bounds__(256) void fp8_gemv_split_kernel(Fp8Operands op)
{
    __shared__ __attribute__((aligned(16))) uint8_t codes[kSplitMaxKB * 32 * kChunk];
    __shared__ float sa_lds[kSplitMaxKB][32];
    __shared__ bool tile_ok;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int M = op.M, N = op.N, K = op.K, KC = K >> 7;
    const int tiles_n = (N + kSplitCols - 1) / kSplitCols;
    const int S = op.splits;
    const int tn = blockIdx.x % tiles_n, split = blockIdx.x / tiles_n;
    const int jb = split * KC / S, je = (split + 1) * KC / S, KB = je - jb;   // 1 <= KB <= 8
    const int n0 = tn * kSplitCols + wave * 16;                   // this wave's 16 columns

    // 1. the activation tile: rows 0..MT*16-1 (zero past M) x KB chunks,
    //    one 128-group per 8 lanes, 16 elements (one code piece) a lane;
    //    every pass's loads go out before the first is used
    const int li = tid & 7;
    constexpr int kGroupsPerPass = 32;
    constexpr int kPasses = MT * 16 * kSplitMaxKB / kGroupsPerPass;
    const int groups = MT * 16 * KB;
    uint4 xa[kPasses], xb[kPasses];
    float sc_in[kPasses];
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
        const int gi = ps * kGroupsPerPass + (tid >> 3);
        const int r = gi % (MT * 16), c = gi / (MT * 16);
        const bool live = gi < groups && r < M;
        xa[ps] = make_uint4(0, 0, 0, 0);
        xb[ps] = make_uint4(0, 0, 0, 0);
        sc_in[ps] = 1.0f;
        if (live) {
            const int jx = jb + c;
            if constexpr (FUSED) {
                const uint16_t* xp = op.x + (size_t)r * K + (size_t)jx * kChunk + li * 16;
                xa[ps] = ldg16u(xp);
                xb[ps] = ldg16u(xp + 8);
            } else {
                xa[ps] = ldg16u(op.q + (size_t)r * K + (size_t)jx * kChunk + li * 16);
                sc_in[ps] = op.s[(size_t)r * op.s_ld + jx];
            }
        }
    }
    // 2. this wave's weight fragments for all KB chunks (rows past N re-read
    //    row N-1 and are never stored; chunks past KB re-read the last one)
    const uint8_t* wrow = op.w + (size_t)min(n0 + r16, N - 1) * K + (size_t)jb * kChunk + g * 16;
    i32x4 wlo[kSplitMaxKB], whi[kSplitMaxKB];
#pragma unroll
    for (int c = 0; c < kSplitMaxKB; ++c) {
        const size_t ko = (size_t)min(c, KB - 1) * kChunk;
        wlo[c] = ldg16(wrow + ko);
        whi[c] = ldg16(wrow + ko + 64);
    }

    // 3. the activation codes and scales into LDS (quantized here if fused)
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
        const int gi = ps * kGroupsPerPass + (tid >> 3);
        if (ps * kGroupsPerPass >= groups) break;      // uniform: no group of this pass is live
        const int r = gi % (MT * 16), c = gi / (MT * 16);
        i32x4 piece;
        float sc = sc_in[ps];
        if constexpr (FUSED) {
            const uint32_t d[8] = {xa[ps].x, xa[ps].y, xa[ps].z, xa[ps].w,
                                   xb[ps].x, xb[ps].y, xb[ps].z, xb[ps].w};
            uint32_t mb = absmax_bits(d);
            if (mb > 0x7F80u) mb = absmax_bits_skip_nan(d);
            mb = max8_lanes(mb);
            float inv;
            group_scale(bf16_bits_f32(mb), sc, inv);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                piece[q] = (int)pack4_e4m3(bf16lo(d[2 * q]) * inv, bf16hi(d[2 * q]) * inv,
                                           bf16lo(d[2 * q + 1]) * inv, bf16hi(d[2 * q + 1]) * inv);
            if (tn == 0 && gi < groups && r < M) {
                const int jx = jb + c;
                *reinterpret_cast<i32x4*>(op.q + (size_t)r * K + (size_t)jx * kChunk + li * 16) = piece;
                if (li == 0) op.s[(size_t)r * op.s_ld + jx] = sc;
            }
        } else {
            piece = i32x4{(int)xa[ps].x, (int)xa[ps].y, (int)xa[ps].z, (int)xa[ps].w};
        }
        if (gi < groups) {
            *reinterpret_cast<i32x4*>(codes + code_off(c, r, li)) = piece;
            if (li == 0) sa_lds[c][r] = sc;
        }
    }
    __syncthreads();

    // 4. per chunk and 16-row tile one MFMA, weights as the first operand:
    //    lane (r16, g) holds C[column 4g+e][activation row r16]
    typedef const __attribute__((address_space(4))) float* cf32p;
    const cf32p swb = (cf32p)(op.sw + (size_t)(min(n0, N - 1) >> 7) * op.sw_ld + jb);
    float swc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) swc[e] = SM == 1 ? op.sw[min(n0 + 4 * g + e, N - 1)] : 0.0f;
    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < kSplitMaxKB; ++c) {
        if (c >= KB) break;
        const i32x8 wf = join(wlo[c], whi[c]);
        const float swj = SM == 0 ? swb[c] : 1.0f;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int r = mt * 16 + r16;
            const i32x8 af = join(*reinterpret_cast<const i32x4*>(codes + code_off(c, r, g)),
                                  *reinterpret_cast<const i32x4*>(codes + code_off(c, r, g + 4)));
            const float sa = sa_lds[c][r];
            const f32x4 p = mfma_e4m3(wf, af, f32x4{0, 0, 0, 0});
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[mt][e] += p[e] * (sa * (SM == 0 ? swj : swc[e]));
        }
    }

    // 5. without an epoch (more than kInLaunchMaxSplits splits): every
    //    split's partials, for the reduction kernel. With one: splits
    //    0..S-2 store theirs, then the tile's flag once every wave's
    //    partial stores have completed
    const int col = n0 + 4 * g;
    if (S > 1 && op.epoch == 0) {
        if (n0 < N) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int m = mt * 16 + r16;
                if (m < M)
                    *reinterpret_cast<f32x4*>(op.part + (size_t)split * M * N + (size_t)m * N +
                                              col) = acc[mt];
            }
        }
        return;
    }
    if (S > 1 && split < S - 1) {
        if (n0 < N) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int m = mt * 16 + r16;
                if (m < M) store_through(op.part + (size_t)split * M * N + (size_t)m * N + col, acc[mt]);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        wait_vmem();
        __syncthreads();
        if (tid == 0) {
            uint64_t* f = split_flags(op, S) + (size_t)split * tiles_n + tn;
            // the tile's last split gave up on this flag: back to waiting
            if (__hip_atomic_exchange(f, op.epoch, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT) ==
                kSplitGaveUp)
                __hip_atomic_store(f, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }

    // 6. the last split (or the only one): wait for the other splits of the
    //    tile (lane sp of wave 0 polls split sp's flag; S - 1 <= 2), then
    //    sum in split order
    static_assert(kInLaunchMaxSplits - 1 <= 64, "one flag per lane of wave 0");
    bool ok = true;
    bool got = false;   // lane sp of wave 0: split sp's flag came
    if (S > 1) {
        uint64_t* flags = split_flags(op, S) + tn;
        if (wave == 0) {
            bool seen = true;
            if (lane < S - 1) {
                uint64_t* f = flags + (size_t)lane * tiles_n;
                const int limit = op.tune.split_spin_limit ? op.tune.split_spin_limit : kSpinLimit;
                for (int spins = 0; limit > 0 && spins < limit; ++spins) {
                    if (__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                        op.epoch) {
                        got = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
                if (!got) {
                    // give up: leave the mark for the late split, or take
                    // back a flag that arrived meanwhile; the tile is NaN
                    if (__hip_atomic_exchange(f, kSplitGaveUp, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT) == op.epoch)
                        __hip_atomic_store(f, (uint64_t)0, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                    seen = false;
                }
            }
            const bool any_missing = __builtin_amdgcn_ballot_w64(!seen) != 0;
            if (any_missing && lane == 0)
                __hip_atomic_fetch_add(split_status(op), (uint64_t)1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            if (lane == 0) tile_ok = !any_missing;
        }
        __syncthreads();
        ok = tile_ok;
    }
    if (n0 >= N) return;
    // the partials of up to kSumBatch splits per round trip, both row
    // tiles' loads in flight together; summed as p0 + p1 + ... + own
    constexpr int kSumBatch = 8;
    f32x4 sum[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) sum[mt] = acc[mt];
    if (S > 1) {
        const size_t mn = (size_t)M * N;
        for (int sp0 = 0; sp0 < S - 1; sp0 += kSumBatch) {
            f32x4 pv[MT][kSumBatch];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int m = min(mt * 16 + r16, M - 1);
                const float* pp = op.part + (size_t)m * N + col;
#pragma unroll
                for (int b = 0; b < kSumBatch; ++b)
                    if (sp0 + b < S - 1) pv[mt][b] = load_through(pp + (size_t)(sp0 + b) * mn);
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int b = 0; b < kSumBatch; ++b) {
                    if (sp0 + b >= S - 1) break;
                    sum[mt] = sp0 + b == 0 ? pv[mt][b] : sum[mt] + pv[mt][b];
                }
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) sum[mt] += acc[mt];
    }
    {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int m = mt * 16 + r16;
            if (m >= M) continue;
            const size_t o = (size_t)m * N + col;
            float v[4] = {sum[mt][0], sum[mt][1], sum[mt][2], sum[mt][3]};
            if (!ok) {
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = __builtin_nanf("");
            }
            if (op.c_f32) {
                float* cp = static_cast<float*>(op.c) + o;
                if (op.residual) {
                    const f32x4 rv = *reinterpret_cast<const f32x4*>(cp);
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] += rv[e];
                }
                *reinterpret_cast<f32x4*>(cp) = f32x4{v[0], v[1], v[2], v[3]};
            } else {
                uint16_t* cp = static_cast<uint16_t*>(op.c) + o;
                if (op.residual) {
                    const uint2 rv = *reinterpret_cast<const uint2*>(cp);
                    v[0] += bf16lo(rv.x);
                    v[1] += bf16hi(rv.x);
                    v[2] += bf16lo(rv.y);
                    v[3] += bf16hi(rv.y);
                }
                *reinterpret_cast<uint2*>(cp) =
                    make_uint2(f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16),
                               f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16));
            }
        }
    }
    // the flags seen back to the waiting state, whether or not the tile
    // completed (one given up on is reset by its late split, or was above)
    if (S > 1 && wave == 0 && got)
        __hip_atomic_store(split_flags(op, S) + tn + (size_t)lane * tiles_n, (uint64_t)0,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// K splits for M x N x K: the fewest that keep every split at 8 chunks or
// less (the LDS code tile and the weight registers). More splits only add
// fp32 partials ((S-1)*M*N*4 bytes, written and read back) and
// per-workgroup staging: on MI355X every config shape at M = 8..32 ran
// fastest at the minimum. An override n > 0 is raised to that minimum and capped at one
// chunk a split.
int gemv_split_count(int M, int N, int K, int forced)
{
    (void)M;
    (void)N;
    const int KC = K / kChunk;
    const int s_min = (KC + kSplitMaxKB - 1) / kSplitMaxKB;
    const int s = forced > s_min ? forced : s_min;
    return s < KC ? s : KC;
}

// Scratch of an S-split launch: summed in the launch, S-1 partial slices,
// (S-1) x tiles flags and the status word; otherwise S partial slices.
static size_t split_scratch(int S, int M, int N)
{
    const size_t tiles = (size_t)(N + kSplitCols - 1) / kSplitCols;
    if (S <= 1) return 0;
    if (S > kInLaunchMaxSplits) return (size_t)S * M * N * 4;
    return (size_t)(S - 1) * M * N * 4 + (size_t)(S - 1) * tiles * 8 + 8;
}

size_t gemv_split_bytes(int M, int N, int K)
{
    return split_scratch(gemv_split_count(M, N, K), M, N);
}

// A fresh 64-bit epoch per split launch: consecutive from a random start,
// never 0 (the cleared state of a flag).
static uint64_t next_epoch()
{
    static std::atomic<uint64_t> ctr{[] {
        std::random_device rd;
        const uint64_t t = (uint64_t)std::chrono::steady_clock::now().time_since_epoch().count();
        return (((uint64_t)rd() << 32) ^ (uint64_t)rd()) ^ (t * 0x9E3779B97F4A7C15ull);
    }()};
    uint64_t e;
    do e = ctr.fetch_add(1, std::memory_order_relaxed);
    while (e == 0 || e == kSplitGaveUp);
    return e;
}

// Where the fused split path beats the chunk-slot GEMV (quantization
// included, HIP-graph replay on MI355X over the config shapes): from
// M = 24 on weights below 32M elements (qkv -9%, o_proj -4..-9%, down
// -10..-21% at M = 24, 32), and from M = 12 on long rows (down, K = 9728:
// -14..-23% at M = 12, 16). Larger weights at 16 < M <= 32 (gate_up) keep
// the quantizer + K-split GEMM, up to 5% faster there.
bool gemv_split_routes(int M, int N, int K)
{
    if (M > 32) return false;
    if (M >= 12 && K >= 8192) return true;
    return M >= 24 && (long)N * K < (32L << 20);
}

bool gemv_split_ready(const Fp8Operands& op)
{
    if (op.M > 32 || op.s_step == 0) return false;
    const int s = gemv_split_count(op.M, op.N, op.K, op.tune.batch_split);
    return s == 1 || (op.part && op.part_bytes >= split_scratch(s, op.M, op.N));
}

hipError_t launch_fp8_gemv_split(const Fp8Operands& op, bool fused, hipStream_t stream,
                                 const LaunchTiming& t, const char** name)
{
    Fp8Operands o = op;
    o.splits = gemv_split_count(op.M, op.N, op.K, op.tune.batch_split);
    const bool in_launch = o.splits > 1 && o.splits <= kInLaunchMaxSplits;
    o.epoch = in_launch ? next_epoch() : 0;
    const int tiles = (op.N + kSplitCols - 1) / kSplitCols;
    const dim3 grid(tiles * o.splits), block(256);
    *name = o.splits > 1 ? (fused ? "fp8_gemv_split64_fused_splitk" : "fp8_gemv_split64_splitk")
                         : (fused ? "fp8_gemv_split64_fused" : "fp8_gemv_split64");
    const LaunchTiming tk{t.start, o.splits > 1 && !in_launch ? nullptr : t.stop};
    auto go = [&](auto kernel) { return launch(kernel, grid, block, 0, stream, tk, o); };
    const int v = (op.M > 16 ? 1 : 0) + (op.w_block ? 0 : 2) + (fused ? 4 : 0);
    hipError_t e;
    switch (v) {
    case 0: e = go(fp8_gemv_split_kernel<1, 0, false>); break;
    case 1: e = go(fp8_gemv_split_kernel<2, 0, false>); break;
    case 2: e = go(fp8_gemv_split_kernel<1, 1, false>); break;
    case 3: e = go(fp8_gemv_split_kernel<2, 1, false>); break;
    case 4: e = go(fp8_gemv_split_kernel<1, 0, true>); break;
    case 5: e = go(fp8_gemv_split_kernel<2, 0, true>); break;
    case 6: e = go(fp8_gemv_split_kernel<1, 1, true>); break;
    default: e = go(fp8_gemv_split_kernel<2, 1, true>); break;
    }
    if (e != hipSuccess || o.splits == 1 || in_launch) return e;
    return launch_splitk_reduce(o, stream, LaunchTiming{nullptr, t.stop});
}

}  // namespace heph
