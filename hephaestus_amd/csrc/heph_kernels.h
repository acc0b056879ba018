// heph_kernels.h - host-side launchers of the gfx950 kernels (internal to
// the library; the public surface is include/hephfp8.h).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

#include "heph_device.h"

namespace heph {

// HEPH_OK when the current HIP device is a gfx950, else HEPH_ERR_DEVICE
// (the answer is cached per device).
int check_device();

// Optional kernel-boundary timestamps for the main kernel of a call.
struct LaunchTiming {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};

template <typename... KArgs, typename... Args>
hipError_t launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t shmem,
                  hipStream_t stream, const LaunchTiming& t, Args... args)
{
    if (t.start || t.stop)
        hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, t.start, t.stop,
                              0u, static_cast<KArgs>(args)...);
    else
        kernel<<<grid, block, shmem, stream>>>(static_cast<KArgs>(args)...);
    return hipGetLastError();
}

// Per-call launch-shape overrides (heph_fp8_linear_with; 0 = the built-in
// choice): chunk slots, waves and steps per batch of the chunk-slot GEMV,
// tile height of the large-M GEMM (1 = the 128x128 kernel), and the
// batched-decode K-split kernel (-1 never, n > 0 always with n splits).
struct Tuning {
    int gemv_ks = 0;
    int gemv_waves = 0;
    int gemv_u = 0;
    int gemm_bm = 0;
    int gemm_bn = 0;
    int batch_split = 0;
    int wide_tiles = 0;
    int wide_waves = 0;
    int split_spin_limit = 0;   // 0: the kernel's own bound
    int gemv_groups = 0;
};

// Activation scale addressing shared by the kernels: chunk j of row m uses
// s[m * s_ld + j * s_step]; group 128: s_ld = K/128, s_step = 1;
// per-token (group K): s_ld = 1, s_step = 0.
// Weight scale addressing: block-128 uses sw[(n / 128) * sw_ld + j] with
// sw_ld = K / 128; per-channel uses sw[n].
struct Fp8Operands {
    const uint8_t* w;      // [N, K] e4m3
    const float* sw;       // weight scales
    int sw_ld;
    bool w_block;          // true: 128x128 blocks, false: per-channel [N,1]
    const uint16_t* x;     // [M, K] bf16 (fused quantization only)
    uint8_t* q;            // [M, K] e4m3 codes (workspace)
    float* s;              // activation scales (workspace)
    int s_ld;
    int s_step;
    void* c;               // [M, N] bf16 or f32
    bool c_f32;
    bool residual;
    int M, N, K;
    // Large-M GEMM split over K: scratch for the fp32 partials (nullptr:
    // none) and its size, and the number of splits the launch uses.
    float* part = nullptr;
    size_t part_bytes = 0;
    int splits = 1;
    // Batched-decode K splits: the value the launch's completion flags
    // carry (unique per launch).
    uint64_t epoch = 0;
    Tuning tune;
};

hipError_t launch_quant(const uint16_t* x, uint8_t* q, float* scales, int M,
                        int K, int group_k, hipStream_t stream,
                        const LaunchTiming& t = LaunchTiming{});

// bf16 [N,K] -> e4m3 codes + f32 scale_inv [ceil(N/128), K/128].
hipError_t launch_wquant(const uint16_t* w, uint8_t* q, float* scale_inv, int N, int K,
                         hipStream_t stream);

// M <= 32 kernel with K-chunk slots in the MFMA rows. fused: quantize x
// inside the kernel (group 128); workgroup 0 also writes q/s. gamma (fused,
// M = 1 only): x is first RMS-normalized with gamma and eps, as
// heph_rmsnorm_bf16 rounds it.
// Longest row the GEMV's RMSNorm prologue holds in LDS (with gamma: 32 KB).
constexpr int kNormMaxK = 8192;
// M = 1, fused quantization (gamma: RMSNorm first), SwiGLU epilogue: the
// weight's rows [0, N/2) are the gate, [N/2, N) the up projection, and
// op.c receives act[N/2] = bf16(bf16(silu(g)) * up) from the bf16-rounded
// gate and up values, in the plain M = 1 GEMV's launch shape for N x K
// (bit for bit the GEMV then silu_mul). N % 16 == 0.
hipError_t launch_fp8_gemv_swiglu(const Fp8Operands& op, hipStream_t stream,
                                  const LaunchTiming& t, const char** name,
                                  const uint16_t* gamma, float eps);
hipError_t launch_fp8_gemv(const Fp8Operands& op, bool fused, hipStream_t stream,
                           const LaunchTiming& t, const char** name,
                           const uint16_t* gamma = nullptr, float eps = 0.0f);

// Rows per chunk slot for M rows (M rounded up to a power of two, at most
// 16), and the launch shape (chunk slots, waves, steps per batch) for
// M x N x K with the overrides of each (0 = automatic); norm: the shape of
// the RMSNorm-fused forms (M = 1), which repeat the norm in every workgroup
// and so keep fewer of them.
int gemv_rows(int M);
// Whether the chunk-slot kernel quantizes x itself for M x N x K (group 128).
bool gemv_fuses(int M, int N, int K);
// groups (when not null): column groups per workgroup, planned for the
// fused route (1 or 2; see fp8_gemv_kernel's CG).
void gemv_shape(int M, int N, int K, const Tuning& tune, int* ks, int* waves, int* u,
                bool norm = false, int* groups = nullptr);

// Compute units the launch shapes are planned for: MI355X's 256. A fixed
// count, so that shapes, summation orders and output bits do not depend on
// how many CUs a mask or partition leaves visible.
constexpr int kPlanCUs = 256;

// Tiled MFMA GEMM for any M (prefill); reads q/s from the workspace.
hipError_t launch_fp8_gemm(const Fp8Operands& op, hipStream_t stream,
                           const LaunchTiming& t, const char** name);

// Tile (bm x bn: 64, 128, 192 or 256 x 256, 256 x 192, 128 x 320) and K
// splits (1 = none) of the large-M GEMM for M x N x K, splits only if
// can_split; forced_bm / forced_bn keep only the tiles of that height /
// width (0 = automatic).
struct GemmPlan {
    int bm, bn, splits;
};
GemmPlan gemm_plan(int M, int N, int K, bool can_split, int forced_bm = 0, int forced_bn = 0);
// Scratch bytes for the partials of the split plan (0 when it does not
// split), and whether op's scratch (part) holds them for a plan of more
// than one split.
size_t gemm_split_bytes(int M, int N, int K);
bool gemm_splits_ready(const Fp8Operands& op);

// Sums op.splits fp32 partials [split][M][N] at op.part in split order, adds
// the residual and stores bf16 or f32 (M*N % 4 == 0).
hipError_t launch_splitk_reduce(const Fp8Operands& op, hipStream_t stream, const LaunchTiming& t);

// Batched decode (M <= 32, per-chunk activation scales): 64-column
// workgroups over K splits in one launch, reading q/s from the workspace;
// partials and completion flags in op.part when it splits. Split count for M x N x K (forced > 0 raises it
// to at least that), its scratch bytes (automatic count), and whether op's
// scratch holds the partials of op's count.
// fused: quantize x inside (group 128); column tile 0 writes q/s.
hipError_t launch_fp8_gemv_split(const Fp8Operands& op, bool fused, hipStream_t stream,
                                 const LaunchTiming& t, const char** name);
int gemv_split_count(int M, int N, int K, int forced = 0);
size_t gemv_split_bytes(int M, int N, int K);
bool gemv_split_ready(const Fp8Operands& op);
// Whether M x N x K takes it by default (op.tune.batch_split: -1 never,
// n > 0 always).
bool gemv_split_routes(int M, int N, int K);

// Batched decode (M <= 32): workgroups of 16*T columns over all of K
// (gemv_wide.hip), reading q/s from the workspace. Launch shape for
// M x N x K with op.tune's overrides, and whether M x N x K takes it by
// default with codes already in the workspace (codes) or bf16 rows to
// quantize first (op.tune.wide_tiles: -1 never, > 0 always).
hipError_t launch_fp8_gemv_wide(const Fp8Operands& op, hipStream_t stream,
                                const LaunchTiming& t, const char** name);
void gemv_wide_shape(int M, int N, int K, const Tuning& tune, int* tiles, int* waves, int* u);
bool gemv_wide_routes(int M, int N, int K, bool codes);

// bf16 x [M,K] @ w [N,K]^T, f32 accumulation, M > 32 (bf16_gemm.hip):
// 128x128 tiles; the residual is the output buffer's contents.
struct Bf16GemmArgs {
    void* c;
    const uint16_t* x;
    const uint16_t* w;
    int M, N, K;
    bool c_f32;
    bool residual;
};
hipError_t launch_bf16_gemm(void* c, bool c_f32, bool residual, const uint16_t* x,
                            const uint16_t* w, int M, int N, int K, hipStream_t stream,
                            const LaunchTiming& t, const char** name);

// bf16 x [M,K] @ w [N,K]^T, f32 accumulation, M <= 32.
hipError_t launch_bf16_skinny(void* c, bool c_f32, bool residual, const uint16_t* x,
                              const uint16_t* w, int M, int N, int K,
                              hipStream_t stream, const LaunchTiming& t,
                              const char** name);

}  // namespace heph
