// api.hip - the C ABI (include/hephfp8.h): argument checks and dispatch.
//
// Mirrors the reference's FP8 linear dispatch (src/hephaestus/kernels.mojo:
// 410-470 linear_fp8, :473-527 linear_add_residual_fp8, :372-407 gemv_fp8):
// M <= 32 goes to the weight-streaming kernel (the reference sends M == 1
// to its GEMV and 2..32 to its small-M kernel), larger M to the tiled GEMM;
// do_quantize=False becomes HEPH_FLAG_SKIP_QUANT. Unlike the reference,
// whose shape preconditions are debug_assert only
// (wmma_gfx12.mojo:731-732, :872-874, :996-1005), every precondition is
// checked here on every call and reported as a status code.
#include <cstring>
#include <mutex>

#include "../../include/hephfp8.h"
#include "heph_kernels.h"

using namespace heph;

namespace {

thread_local LaunchTiming g_next_timing;
thread_local const char* g_last_kernel = "none";

constexpr int kMaxDevices = 64;
int g_dev_ok[kMaxDevices];  // 0 unknown, 1 gfx950, -1 other
std::mutex g_dev_mu;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

LaunchTiming take_timing()
{
    LaunchTiming t = g_next_timing;
    g_next_timing = LaunchTiming{};
    return t;
}

int launch_status(hipError_t e) { return e == hipSuccess ? HEPH_OK : HEPH_ERR_LAUNCH; }

int check_quant_args(const void* x, const void* q, const void* s, int M, int K, int group_k)
{
    if (!x || !q || !s) return HEPH_ERR_NULL;
    if (M < 1 || K < 16 || K % 16) return HEPH_ERR_SHAPE;
    if ((long)M * K > (1L << 40)) return HEPH_ERR_SHAPE;
    if (group_k != kChunk && group_k != K) return HEPH_ERR_GROUP;
    if (group_k == kChunk && K % kChunk) return HEPH_ERR_SHAPE;
    if (!aligned16(x) || !aligned16(q)) return HEPH_ERR_ALIGN;
    return HEPH_OK;
}

}  // namespace

namespace heph {

int check_device()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return HEPH_ERR_DEVICE;
    if (dev < 0 || dev >= kMaxDevices) return HEPH_ERR_DEVICE;
    int state = __atomic_load_n(&g_dev_ok[dev], __ATOMIC_ACQUIRE);
    if (state == 0) {
        std::lock_guard<std::mutex> lk(g_dev_mu);
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, dev) != hipSuccess) return HEPH_ERR_DEVICE;
        state = strncmp(p.gcnArchName, "gfx950", 6) == 0 ? 1 : -1;
        __atomic_store_n(&g_dev_ok[dev], state, __ATOMIC_RELEASE);
    }
    return state == 1 ? HEPH_OK : HEPH_ERR_DEVICE;
}

}  // namespace heph

extern "C" {

size_t heph_fp8_q_ws_bytes(int M, int K)
{
    if (M < 1 || K < 1) return 0;
    return (size_t)M * (size_t)K;
}

size_t heph_fp8_linear_ws_bytes(int M, int N, int K)
{
    if (M < 1 || N < 1 || K < 1) return 0;
    const size_t q = ((size_t)M * (size_t)K + 255) & ~(size_t)255;
    if (check_device() != HEPH_OK) return q;
    const size_t g = gemm_split_bytes(M, N, K);
    const size_t b = M <= HEPH_SKINNY_MAX_M ? gemv_split_bytes(M, N, K) : 0;
    return q + (g > b ? g : b);
}

size_t heph_fp8_s_ws_floats(int M, int K, int group_k)
{
    if (M < 1 || K < 1 || group_k < 1 || K % group_k) return 0;
    return (size_t)M * (size_t)(K / group_k);
}

int heph_fp8_quant_act(const uint16_t* x_bf16, uint8_t* q, float* scales, int M,
                       int K, int group_k, void* stream)
{
    int st = check_quant_args(x_bf16, q, scales, M, K, group_k);
    if (st != HEPH_OK) return st;
    if ((st = check_device()) != HEPH_OK) return st;
    return launch_status(launch_quant(x_bf16, q, scales, M, K, group_k,
                                      static_cast<hipStream_t>(stream)));
}

int heph_fp8_quant_weight(const uint16_t* w_bf16, uint8_t* q, float* scale_inv, int N,
                          int K, void* stream)
{
    if (!w_bf16 || !q || !scale_inv) return HEPH_ERR_NULL;
    if (N < 1 || K < kChunk || K % kChunk || (long)N * K > (1L << 40)) return HEPH_ERR_SHAPE;
    if (!aligned16(w_bf16) || !aligned16(q)) return HEPH_ERR_ALIGN;
    int st = check_device();
    if (st != HEPH_OK) return st;
    return launch_status(launch_wquant(w_bf16, q, scale_inv, N, K,
                                       static_cast<hipStream_t>(stream)));
}

}  // extern "C"

namespace {

// Launch-shape overrides of one heph_fp8_linear_with call, checked and
// copied into the operands (no state outlives the call).
int take_overrides(const heph_launch_overrides* ov, Tuning* t)
{
    *t = Tuning{};
    if (!ov) return HEPH_OK;
    const int ks = ov->gemv_ks, w = ov->gemv_waves, u = ov->gemv_u, bm = ov->gemm_bm;
    if (ks != 0 && ks != 1 && ks != 2 && ks != 4 && ks != 8) return HEPH_ERR_FLAGS;
    if (w != 0 && w != 4 && w != 5 && w != 8 && w != 10 && w != 16) return HEPH_ERR_FLAGS;
    if (u != 0 && u != 1 && u != 2) return HEPH_ERR_FLAGS;
    if (bm != 0 && bm != 1 && bm != 64 && bm != 128 && bm != 192 && bm != 256)
        return HEPH_ERR_FLAGS;
    if (ov->batch_split < -1 || ov->batch_split > 64) return HEPH_ERR_FLAGS;
    const int wt = ov->wide_tiles, ww = ov->wide_waves;
    if (wt != -1 && wt != 0 && wt != 1 && wt != 2 && wt != 4) return HEPH_ERR_FLAGS;
    if (ww != 0 && ww != 4 && ww != 8 && ww != 16) return HEPH_ERR_FLAGS;
    if (ov->split_spin_limit < -1) return HEPH_ERR_FLAGS;
    if (ov->gemv_groups != 0 && ov->gemv_groups != 1 && ov->gemv_groups != 2)
        return HEPH_ERR_FLAGS;
    if (ov->gemm_bn != 0 && ov->gemm_bn != 192 && ov->gemm_bn != 256 && ov->gemm_bn != 320)
        return HEPH_ERR_FLAGS;
    t->gemm_bn = ov->gemm_bn;
    t->split_spin_limit = ov->split_spin_limit;
    t->gemv_groups = ov->gemv_groups;
    t->wide_tiles = wt;
    t->wide_waves = ww;
    t->gemv_ks = ks;
    t->gemv_waves = w;
    t->gemv_u = u;
    t->gemm_bm = bm;
    t->batch_split = ov->batch_split;
    return HEPH_OK;
}

}  // namespace

namespace heph {

// heph_fp8_linear, and with gamma (M = 1, group 128, fused GEMV only) the
// RMSNorm of x folded into the GEMV's quantization prologue; also the body
// of the allocation-free entry point (noalloc.hip).
int fp8_linear_impl(void* c, int c_dtype, const uint16_t* x_bf16, const uint8_t* w,
                    const float* w_scale, int w_block_n, int w_block_k, uint8_t* q_ws,
                    size_t q_ws_bytes, float* s_ws, size_t s_ws_floats, int M, int N, int K,
                    int group_k, int flags, void* stream, const uint16_t* gamma, float eps,
                    const heph_launch_overrides* ov)
{
    const int known = HEPH_FLAG_ADD_RESIDUAL | HEPH_FLAG_SKIP_QUANT | HEPH_FLAG_FORCE_GEMM |
                      HEPH_FLAG_NO_FUSE;
    if (flags & ~known) return HEPH_ERR_FLAGS;
    Tuning tune;
    if (take_overrides(ov, &tune) != HEPH_OK) return HEPH_ERR_FLAGS;
    const bool skip_quant = flags & HEPH_FLAG_SKIP_QUANT;
    if (!c || !w || !w_scale || !q_ws || !s_ws) return HEPH_ERR_NULL;
    if (!skip_quant && !x_bf16) return HEPH_ERR_NULL;
    if (c_dtype != HEPH_DTYPE_BF16 && c_dtype != HEPH_DTYPE_F32) return HEPH_ERR_DTYPE;
    if (M < 1 || N < 16 || K < 16 || N % 16 || K % 16) return HEPH_ERR_SHAPE;
    if ((long)M * K > (1L << 40) || (long)N * K > (1L << 40) || (long)M * N > (1L << 40))
        return HEPH_ERR_SHAPE;
    if (group_k != kChunk && group_k != K) return HEPH_ERR_GROUP;
    bool w_block;
    if (w_block_n == kChunk && w_block_k == kChunk) w_block = true;
    else if (w_block_n == 1 && w_block_k == K) w_block = false;
    else return HEPH_ERR_GROUP;
    // K not a multiple of 128: the reference's own granularity only
    // (per-token activations, per-channel weights; its kernels need K % 16,
    // wmma_gfx12.mojo:731-732), through the 128x128 GEMM with the last
    // chunk's missing pieces read as zeros, any M (the reference loops a
    // GEMV over the rows there, kernels.mojo:461-470)
    const bool ragged = K % kChunk != 0;
    if (ragged && (group_k != K || w_block)) return HEPH_ERR_SHAPE;
    if (q_ws_bytes < heph_fp8_q_ws_bytes(M, K) ||
        s_ws_floats < heph_fp8_s_ws_floats(M, K, group_k))
        return HEPH_ERR_WORKSPACE;
    if (!aligned16(c) || !aligned16(w) || !aligned16(q_ws) || (x_bf16 && !aligned16(x_bf16)))
        return HEPH_ERR_ALIGN;
    int st = check_device();
    if (st != HEPH_OK) return st;

    hipStream_t s = static_cast<hipStream_t>(stream);
    Fp8Operands op{};
    op.w = w;
    op.sw = w_scale;
    op.sw_ld = w_block ? K / kChunk : 1;
    op.w_block = w_block;
    op.x = x_bf16;
    op.q = q_ws;
    op.s = s_ws;
    op.s_ld = K / group_k;
    op.s_step = group_k == kChunk ? 1 : 0;
    op.c = c;
    op.c_f32 = c_dtype == HEPH_DTYPE_F32;
    op.residual = flags & HEPH_FLAG_ADD_RESIDUAL;
    op.M = M;
    op.N = N;
    op.K = K;
    op.tune = tune;
    // The part of q_ws past the codes (from the next 256-byte boundary) is
    // scratch for the large-M GEMM's split-K partials.
    const size_t qb = ((size_t)M * (size_t)K + 255) & ~(size_t)255;
    if (q_ws_bytes > qb) {
        op.part = reinterpret_cast<float*>(q_ws + qb);
        op.part_bytes = q_ws_bytes - qb;
    }

    // M <= 32 takes the chunk-slot GEMV unless the GEMM is forced. Batched
    // decode from M = 8 (codes) or 9 (bf16 rows, quantized first) takes the
    // wide-tile kernel (gemv_wide_routes), except past M = 24 on large
    // weights: there the 64-column K-split kernel where gemv_split_routes
    // holds and the caller's scratch holds its partials, else quantizer +
    // K-split GEMM on weights of >= 32M elements when scratch allows. Forced
    // K splits or chunk-slot shapes (overrides) keep the wide kernel out.
    // The RMSNorm entry point always takes the GEMV.
    const bool forced_gemm = (flags & HEPH_FLAG_FORCE_GEMM) || ragged;
    if (ragged) op.tune.gemm_bm = 1;
    const int wmode = gamma ? -1 : tune.wide_tiles;
    const int bmode = gamma ? -1 : tune.batch_split;
    const bool wide_auto = bmode <= 0 && !tune.gemv_ks && !tune.gemv_waves &&
                           gemv_wide_routes(M, N, K, skip_quant);
    const bool wide = !forced_gemm && M <= HEPH_SKINNY_MAX_M && wmode >= 0 &&
                      (wmode > 0 || wide_auto);
    const bool batch_split = !forced_gemm && !wide && M <= HEPH_SKINNY_MAX_M &&
                             group_k == kChunk && bmode >= 0 &&
                             (bmode > 0 || gemv_split_routes(M, N, K)) && gemv_split_ready(op);
    const bool split_gemm = !gamma && !wide && !batch_split && M >= 16 &&
                            (long)N * K >= (32L << 20) && gemm_splits_ready(op);
    const bool gemv =
        !forced_gemm && M <= HEPH_SKINNY_MAX_M && !split_gemm && !batch_split && !wide;
    if (gamma && !(gemv && M == 1 && group_k == kChunk)) return HEPH_ERR_UNSUPPORTED;
    const bool fuse_ok = !skip_quant && !(flags & HEPH_FLAG_NO_FUSE) && group_k == kChunk;
    const bool fused = fuse_ok && (batch_split || (gemv && gemv_fuses(M, N, K)));
    if (gamma && !fused) return HEPH_ERR_UNSUPPORTED;
    LaunchTiming t = take_timing();
    if (!skip_quant && !fused) {
        // A timed call spans both kernels: the quantizer carries the start
        // stamp and the main kernel the stop stamp.
        hipError_t e = launch_quant(x_bf16, q_ws, s_ws, M, K, group_k, s,
                                    LaunchTiming{t.start, nullptr});
        if (e != hipSuccess) return HEPH_ERR_LAUNCH;
        t.start = nullptr;
    }
    hipError_t e;
    if (wide) e = launch_fp8_gemv_wide(op, s, t, &g_last_kernel);
    else if (batch_split) e = launch_fp8_gemv_split(op, fused, s, t, &g_last_kernel);
    else if (gemv) e = launch_fp8_gemv(op, fused, s, t, &g_last_kernel, gamma, eps);
    else e = launch_fp8_gemm(op, s, t, &g_last_kernel);
    return launch_status(e);
}

}  // namespace heph

extern "C" {

int heph_fp8_linear(void* c, int c_dtype, const uint16_t* x_bf16, const uint8_t* w,
                    const float* w_scale, int w_block_n, int w_block_k, uint8_t* q_ws,
                    size_t q_ws_bytes, float* s_ws, size_t s_ws_floats, int M, int N,
                    int K, int group_k, int flags, void* stream)
{
    return fp8_linear_impl(c, c_dtype, x_bf16, w, w_scale, w_block_n, w_block_k, q_ws,
                           q_ws_bytes, s_ws, s_ws_floats, M, N, K, group_k, flags, stream,
                           nullptr, 0.0f, nullptr);
}

int heph_fp8_linear_with(void* c, int c_dtype, const uint16_t* x_bf16, const uint8_t* w,
                         const float* w_scale, int w_block_n, int w_block_k, uint8_t* q_ws,
                         size_t q_ws_bytes, float* s_ws, size_t s_ws_floats, int M, int N,
                         int K, int group_k, int flags, void* stream,
                         const heph_launch_overrides* overrides)
{
    return fp8_linear_impl(c, c_dtype, x_bf16, w, w_scale, w_block_n, w_block_k, q_ws,
                           q_ws_bytes, s_ws, s_ws_floats, M, N, K, group_k, flags, stream,
                           nullptr, 0.0f, overrides);
}

int heph_fp8_linear_rmsnorm(void* c, int c_dtype, const uint16_t* x_bf16,
                            const uint16_t* gamma_bf16, float eps, const uint8_t* w,
                            const float* w_scale, int w_block_n, int w_block_k, uint8_t* q_ws,
                            size_t q_ws_bytes, float* s_ws, size_t s_ws_floats, int N, int K,
                            int flags, void* stream)
{
    if (!gamma_bf16 || !x_bf16) return HEPH_ERR_NULL;
    if (flags & ~HEPH_FLAG_ADD_RESIDUAL) return HEPH_ERR_FLAGS;
    if (!aligned16(gamma_bf16)) return HEPH_ERR_ALIGN;     // read in 16-byte pieces
    if (K > kNormMaxK) return HEPH_ERR_UNSUPPORTED;
    return fp8_linear_impl(c, c_dtype, x_bf16, w, w_scale, w_block_n, w_block_k, q_ws,
                           q_ws_bytes, s_ws, s_ws_floats, 1, N, K, kChunk, flags, stream,
                           gamma_bf16, eps, nullptr);
}

int heph_fp8_linear_swiglu(void* act_bf16, const uint16_t* x_bf16, const uint16_t* gamma_bf16,
                           float eps, const uint8_t* w, const float* w_scale, int w_block_n,
                           int w_block_k, uint8_t* q_ws, size_t q_ws_bytes, float* s_ws,
                           size_t s_ws_floats, int N, int K, void* stream)
{
    if (!act_bf16 || !x_bf16 || !w || !w_scale || !q_ws || !s_ws) return HEPH_ERR_NULL;
    if (N < 16 || N % 16 || K < kChunk || K % kChunk) return HEPH_ERR_SHAPE;
    if ((long)N * K > (1L << 40)) return HEPH_ERR_SHAPE;
    bool w_block;
    if (w_block_n == kChunk && w_block_k == kChunk) w_block = true;
    else if (w_block_n == 1 && w_block_k == K) w_block = false;
    else return HEPH_ERR_GROUP;
    if (gamma_bf16 && K > kNormMaxK) return HEPH_ERR_UNSUPPORTED;
    if (q_ws_bytes < heph_fp8_q_ws_bytes(1, K) ||
        s_ws_floats < heph_fp8_s_ws_floats(1, K, kChunk))
        return HEPH_ERR_WORKSPACE;
    if (!aligned16(act_bf16) || !aligned16(w) || !aligned16(q_ws) || !aligned16(x_bf16) ||
        (gamma_bf16 && !aligned16(gamma_bf16)))
        return HEPH_ERR_ALIGN;
    int st = check_device();
    if (st != HEPH_OK) return st;
    Fp8Operands op{};
    op.w = w;
    op.sw = w_scale;
    op.sw_ld = w_block ? K / kChunk : 1;
    op.w_block = w_block;
    op.x = x_bf16;
    op.q = q_ws;
    op.s = s_ws;
    op.s_ld = K / kChunk;
    op.s_step = 1;
    op.c = act_bf16;
    op.M = 1;
    op.N = N;
    op.K = K;
    const hipError_t e = launch_fp8_gemv_swiglu(op, static_cast<hipStream_t>(stream),
                                                take_timing(), &g_last_kernel, gamma_bf16, eps);
    return launch_status(e);
}

int heph_bf16_linear(void* c, int c_dtype, const uint16_t* x_bf16, const uint16_t* w_bf16,
                     int M, int N, int K, int flags, void* stream)
{
    if (flags & ~HEPH_FLAG_ADD_RESIDUAL) return HEPH_ERR_FLAGS;
    if (!c || !x_bf16 || !w_bf16) return HEPH_ERR_NULL;
    if (c_dtype != HEPH_DTYPE_BF16 && c_dtype != HEPH_DTYPE_F32) return HEPH_ERR_DTYPE;
    if (M < 1 || N < 16 || N % 16 || K < kChunk || K % kChunk) return HEPH_ERR_SHAPE;
    if ((long)N * K > (1L << 40) || (long)M * K > (1L << 40) || (long)M * N > (1L << 40))
        return HEPH_ERR_SHAPE;
    if (!aligned16(c) || !aligned16(x_bf16) || !aligned16(w_bf16)) return HEPH_ERR_ALIGN;
    int st = check_device();
    if (st != HEPH_OK) return st;
    const LaunchTiming t = take_timing();
    const bool f32 = c_dtype == HEPH_DTYPE_F32, res = flags & HEPH_FLAG_ADD_RESIDUAL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // up to 32 rows the weight stream bounds the call; beyond, the MFMA GEMM
    if (M <= HEPH_SKINNY_MAX_M)
        return launch_status(launch_bf16_skinny(c, f32, res, x_bf16, w_bf16, M, N, K, s, t,
                                                &g_last_kernel));
    return launch_status(launch_bf16_gemm(c, f32, res, x_bf16, w_bf16, M, N, K, s, t,
                                          &g_last_kernel));
}

const char* heph_strerror(int status)
{
    switch (status) {
    case HEPH_OK: return "ok";
    case HEPH_ERR_NULL: return "a required pointer is NULL";
    case HEPH_ERR_SHAPE:
        return "M, N or K out of range (need M>=1, N%16==0, K%16==0, and K%128==0 unless "
               "group_k = K with per-channel weights)";
    case HEPH_ERR_ALIGN: return "pointer not 16-byte aligned";
    case HEPH_ERR_GROUP: return "unsupported activation group or weight block";
    case HEPH_ERR_DTYPE: return "unknown output dtype";
    case HEPH_ERR_WORKSPACE: return "workspace smaller than required";
    case HEPH_ERR_FLAGS: return "unknown or contradictory flags";
    case HEPH_ERR_DEVICE: return "current HIP device is not gfx950 (MI355X)";
    case HEPH_ERR_LAUNCH: return "HIP kernel launch failed";
    case HEPH_ERR_SCRATCH:
        return "codes and scales larger than the allocation-free entry point's fixed scratch "
               "(heph_noalloc_scratch_bytes)";
    case HEPH_ERR_UNSUPPORTED:
        return "shape outside this entry point's limits (fused RMSNorm linear: M = 1, "
               "group 128, K <= 8192)";
    default: return "unknown status";
    }
}

int heph_abi_version(void) { return HEPH_ABI_VERSION; }

int heph_profile_next_launch(void* start_event, void* stop_event)
{
    g_next_timing.start = static_cast<hipEvent_t>(start_event);
    g_next_timing.stop = static_cast<hipEvent_t>(stop_event);
    return HEPH_OK;
}

const char* heph_last_kernel(void) { return g_last_kernel; }

}  // extern "C"
