/*
 * hephfp8.h - C ABI of the MI355X (gfx950) W8A8 FP8 linear-layer library.
 *
 * The library replaces the matmul dispatch of the Hephaestus engine's FP8
 * linear layer. Every entry point takes caller-owned device pointers and a
 * HIP stream, allocates nothing, never synchronizes, and is reentrant.
 * Shapes are checked on the host on every call; a bad call returns a
 * negative HEPH_ERR_* code and launches nothing.
 *
 * Data layouts (all row-major, device memory):
 *   activations x    bf16 [M, K]                  (uint16_t bit patterns)
 *   weight w         OCP E4M3FN codes [N, K]      (safetensors [out, in])
 *   weight scale     f32, one of
 *                      block-128: [ceil(N/128), ceil(K/128)]
 *                                 (the weight_scale_inv dequant multiplier)
 *                      per-channel: [N, 1]  (block 1 x K)
 *   act codes q      E4M3FN [M, K]
 *   act scales s     f32 [M, K / group_k]; group_k is 128 or K
 *   output c         bf16 or f32 [M, N]
 *
 * Arithmetic: c[m,n] = sum over 128-wide K chunks j of
 *     sa[m, j*128/group_k] * sw[n/bn, j*128/bk] * sum_{k in j} q[m,k]*w[n,k]
 * with fp32 accumulation, then (ADD_RESIDUAL) + f32(c[m,n]), then the cast.
 * Activation quantization per group: scale = amax/448 (1.0 when below
 * 1e-12), q = e4m3_rne(x * (1/scale)).
 *
 * Requirements: N % 16 == 0, K % 16 == 0, M >= 1, 16-byte aligned
 * pointers for x, w, q and c; K % 128 == 0 with 1x128 activation groups or
 * 128x128 weight blocks (heph_fp8_linear below lists the domain).
 */
#ifndef HEPHFP8_H
#define HEPHFP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HEPH_ABI_VERSION 6

/* status codes */
#define HEPH_OK                 0
#define HEPH_ERR_NULL         (-1)  /* a required pointer is NULL */
#define HEPH_ERR_SHAPE        (-2)  /* M, N or K out of range / not aligned */
#define HEPH_ERR_ALIGN        (-3)  /* pointer not 16-byte aligned */
#define HEPH_ERR_GROUP        (-4)  /* group_k or weight block unsupported */
#define HEPH_ERR_DTYPE        (-5)  /* unknown output dtype */
#define HEPH_ERR_WORKSPACE    (-6)  /* workspace smaller than required */
#define HEPH_ERR_FLAGS        (-7)  /* unknown or contradictory flags */
#define HEPH_ERR_DEVICE       (-8)  /* current device is not gfx950 */
#define HEPH_ERR_LAUNCH       (-9)  /* HIP reported an error at launch */
#define HEPH_ERR_UNSUPPORTED (-10)  /* valid shape outside this entry point's limits */
#define HEPH_ERR_SCRATCH     (-11)  /* codes + scales exceed the fixed no-alloc scratch */

/* output dtypes */
#define HEPH_DTYPE_BF16 0
#define HEPH_DTYPE_F32  1

/* flags for heph_fp8_linear / heph_bf16_linear */
#define HEPH_FLAG_ADD_RESIDUAL 0x1  /* c += result (c is read, then written) */
#define HEPH_FLAG_SKIP_QUANT   0x2  /* q_ws / s_ws already hold this x's codes */
#define HEPH_FLAG_FORCE_GEMM   0x8  /* use the tiled MFMA GEMM (tests) */
#define HEPH_FLAG_NO_FUSE      0x10 /* quantize in its own kernel (tests) */

/* Largest M served by the weight-streaming kernels (chunk-slot GEMV, K-split). */
#define HEPH_SKINNY_MAX_M 32

/*
 * Dynamic activation quantization, bf16 [M,K] -> E4M3 codes + f32 scales.
 * Replaces quantize_act_rows_fp8 / quantize_act_fp8_pad
 * (reference src/hephaestus/kernels.mojo:196-211, :270-287); group_k == K is
 * the reference's per-token quantizer (K % 16 == 0), group_k == 128 the
 * 1x128 groups (K % 128 == 0). scales has M * (K / group_k) floats.
 */
int heph_fp8_quant_act(const uint16_t* x_bf16, uint8_t* q, float* scales,
                       int M, int K, int group_k, void* stream);

/*
 * Block weight quantization, bf16 [N,K] -> E4M3 codes [N,K] + f32
 * scale_inv [ceil(N/128), K/128]: per 128x128 block s = amax/448 (1.0 when
 * amax is 0 or s < 1e-12), codes = e4m3(w / s). Produces the
 * weight / weight_scale_inv format from a bf16 tensor. Replaces the
 * reference's offline per-row quantizer
 * (reference scripts/stage_tiny_fp8_from_bf16.py:59-71) with its block form.
 */
int heph_fp8_quant_weight(const uint16_t* w_bf16, uint8_t* q, float* scale_inv,
                          int N, int K, void* stream);

/*
 * W8A8 linear: c = x @ dequant(w)^T with dynamic activation quantization.
 * Replaces linear_fp8, linear_add_residual_fp8 and gemv_fp8
 * (reference src/hephaestus/kernels.mojo:372-407, :410-470, :473-527):
 *   c, c_dtype           the reference's `c` (or `residual` with
 *                        HEPH_FLAG_ADD_RESIDUAL, updated in place)
 *   x_bf16               `a`
 *   w, w_scale           `w`, `scale` (block given by w_block_n/w_block_k:
 *                        (128,128) or (1,K))
 *   q_ws, s_ws           `a_fp8_ws`, `act_scale_ws`; sizes in bytes / floats
 *   M, N, K              `m`, `n`, `k`: N % 16 == 0, K % 16 == 0; K % 128
 *                        == 0 except with the reference's own granularity
 *                        (group_k = K, w block (1,K)), which takes the
 *                        128x128 GEMM for any M with the K tail zeroed
 *   group_k              activation group: 128 or K
 *   flags                HEPH_FLAG_SKIP_QUANT is the reference's
 *                        do_quantize=False
 *   stream               the stream of the reference's DeviceContext
 * On return the workspaces hold x's codes and scales (unless SKIP_QUANT),
 * so later calls on the same x can pass SKIP_QUANT.
 * Past the codes (from the next 256-byte boundary) q_ws is K-split scratch
 * when q_ws_bytes >= heph_fp8_linear_ws_bytes(M, N, K). At M <= 32 the
 * 64-column kernel may sum 2 or 3 K splits inside one launch, where the last
 * split of each column tile waits for the others' completion flags for a
 * bounded time (~0.3 s). If a wait ever gives up, that tile's outputs are
 * NaN, the call still returns HEPH_OK (nothing waits for the device), and
 * the 64-bit word at byte HEPH_SPLIT_STATUS_OFFSET(q_ws_bytes) of q_ws is
 * incremented: a count of tiles given up since the caller last zeroed it,
 * for the caller to read after synchronizing. The flags are left ready, so
 * later calls and graph replays on the workspace are unaffected.
 */
#define HEPH_SPLIT_STATUS_OFFSET(q_ws_bytes) (((size_t)(q_ws_bytes) - 8) & ~(size_t)7)
int heph_fp8_linear(void* c, int c_dtype, const uint16_t* x_bf16,
                    const uint8_t* w, const float* w_scale, int w_block_n,
                    int w_block_k, uint8_t* q_ws, size_t q_ws_bytes,
                    float* s_ws, size_t s_ws_floats, int M, int N, int K,
                    int group_k, int flags, void* stream);

/*
 * Decode-step linear on an RMS-normalized row (M = 1, group 128): c =
 * rmsnorm(x, gamma, eps) @ dequant(w)^T, where the norm is
 * bf16(gamma * bf16(x * r)) with r = 1/sqrt(mean(x^2) + eps) summed as
 * heph_rmsnorm sums it, computed by every workgroup of the fused GEMV
 * before its quantization, so the normalized row is never written. Its
 * launch shape keeps fewer workgroups than heph_fp8_linear's at M = 1 (each
 * repeats the norm): the fewest K-chunk slots (<= 8) giving >= 256
 * workgroups, 4 waves up to 3 chunk steps, else 8 (two-step batches when
 * each wave has two steps). Bit for bit heph_rmsnorm followed by
 * heph_fp8_linear_with that shape (gemv_ks, gemv_waves, gemv_u); plain
 * heph_fp8_linear may sum in another order (within the linear's tolerance).
 * The workspaces hold the normalized row's codes and scales. Replaces the
 * pair rms_norm + linear_fp8
 * of the reference's decode step (src/hephaestus/forward.mojo:359-615,
 * kernels.mojo:653-762). flags: HEPH_FLAG_ADD_RESIDUAL only; gamma 16-byte
 * aligned (HEPH_ERR_ALIGN); K <= 8192 (the row and gamma sit in the
 * workgroup's LDS), else HEPH_ERR_UNSUPPORTED (callers with longer rows run
 * heph_rmsnorm, then heph_fp8_linear).
 */
int heph_fp8_linear_rmsnorm(void* c, int c_dtype, const uint16_t* x_bf16,
                            const uint16_t* gamma_bf16, float eps, const uint8_t* w,
                            const float* w_scale, int w_block_n, int w_block_k,
                            uint8_t* q_ws, size_t q_ws_bytes, float* s_ws,
                            size_t s_ws_floats, int N, int K, int flags, void* stream);

/*
 * Decode-step feed-forward input (M = 1, group 128): act = silu(g) * u
 * with g = xn @ dequant(w[0:N/2])^T and u = xn @ dequant(w[N/2:N])^T, xn =
 * rmsnorm(x, gamma, eps) when gamma is given (as heph_fp8_linear_rmsnorm
 * computes it; K <= 8192, else HEPH_ERR_UNSUPPORTED) or x itself when gamma
 * is NULL. w holds the gate rows then the up rows ([N, K], N % 16 == 0),
 * w_scale their 128x128 blocks (w_block_n = w_block_k = 128) or per-row
 * scales [N, 1] (1, K). act: bf16 [N/2], bf16(bf16(g / (1 + exp(-g))) * u)
 * of the bf16-rounded g and u: bit for bit the gate/up linear (bf16 output;
 * heph_fp8_linear_rmsnorm with gamma, heph_fp8_linear without) followed by
 * heph_silu_mul, in one launch whose workgroups each finish as many gate as
 * up columns. Replaces rms_norm + linear_fp8(gate_proj) +
 * linear_fp8(up_proj) + silu_mul of the reference's decode step
 * (src/hephaestus/forward.mojo:537-578; silu_mul, kernels.mojo:1243-1278).
 * The workspaces receive xn's codes and scales, as for the other M = 1
 * entry points.
 */
int heph_fp8_linear_swiglu(void* act_bf16, const uint16_t* x_bf16, const uint16_t* gamma_bf16,
                           float eps, const uint8_t* w, const float* w_scale, int w_block_n,
                           int w_block_k, uint8_t* q_ws, size_t q_ws_bytes, float* s_ws,
                           size_t s_ws_floats, int N, int K, void* stream);

/*
 * Unquantized bf16 linear with f32 accumulation: c = x @ w^T.
 * Replaces `linear` for the lm_head (reference
 * src/hephaestus/kernels.mojo:89-121, which keeps F32 logits): M <= 32
 * streams the weights (the decode rows, as the reference's gemv path),
 * M > 32 runs an MFMA GEMM (the reference's wmma_gemm_bf16 for M > 1,
 * src/hephaestus/wmma_gfx12.mojo:428-473). N % 16 == 0, K % 128 == 0.
 * flags: ADD_RESIDUAL only.
 */
int heph_bf16_linear(void* c, int c_dtype, const uint16_t* x_bf16,
                     const uint16_t* w_bf16, int M, int N, int K, int flags,
                     void* stream);

/*
 * heph_fp8_linear without workspace arguments, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference, whose
 * callers preallocate a_fp8_ws / act_scale_ws (forward.mojo:121-125).
 * The activation codes, scales and K-split partials live in one fixed
 * device array of HEPH_NOALLOC_SCRATCH_BYTES (64 MiB) that the library's
 * code object holds on every GPU it runs on until the process ends; the
 * call allocates and frees nothing. Limit: round256(M*K) +
 * round256(4*M*K/group_k) <= HEPH_NOALLOC_SCRATCH_BYTES (e.g. M = 4096 at
 * K = 9728), else HEPH_ERR_SCRATCH before any device work. All calls on
 * one GPU share the array: HEPH_FLAG_SKIP_QUANT reuses the codes the
 * previous call on that GPU left there (same M, K, group_k), and calls that
 * overlap on one GPU (several streams or threads) race on it and must be
 * serialized by the caller. Arguments and flags otherwise as
 * heph_fp8_linear; outputs are bit for bit those of heph_fp8_linear with a
 * q_ws of heph_fp8_linear_ws_bytes(M, N, K) bytes whenever the K-split
 * partials fit the array's remainder.
 */
#define HEPH_NOALLOC_SCRATCH_BYTES (64u << 20)
int heph_fp8_linear_noalloc(void* c, int c_dtype, const uint16_t* x_bf16,
                            const uint8_t* w, const float* w_scale, int w_block_n,
                            int w_block_k, int M, int N, int K, int group_k,
                            int flags, void* stream);

/* HEPH_NOALLOC_SCRATCH_BYTES of the built library. */
size_t heph_noalloc_scratch_bytes(void);

/*
 * Producer-side activation quantization: the op that feeds an FP8 linear
 * writes that linear's activation codes and scales itself (bit for bit what
 * the producer followed by heph_fp8_quant_act writes), so the linear runs
 * with HEPH_FLAG_SKIP_QUANT and the separate quantizer launch, with its pass
 * over the bf16 activations, is gone. Replaces the pairs rms_norm +
 * quantize_act_rows_fp8 and silu_mul + quantize_act_rows_fp8 of the
 * reference's prefill (src/hephaestus/forward.mojo:45-81,
 * kernels.mojo:1243-1278, :270-287; the quantization is the one linear_fp8
 * runs at kernels.mojo:449-450).
 *
 * heph_rmsnorm_quant_fp8: per row of cols, y = bf16(gamma * bf16(x * r)),
 * r = 1/sqrt(mean(x^2) + eps) summed as heph_rmsnorm sums it; q [rows, cols]
 * codes and scales [rows, cols / group_k] of y. cols % 128 == 0 and
 * cols <= 16384 (the row is staged in LDS; HEPH_ERR_UNSUPPORTED beyond).
 *
 * heph_silu_mul_quant_fp8: per row, y = bf16(bf16(g / (1 + exp(-g))) * up)
 * as heph_silu_mul computes it, over n elements of gate and up, row r at
 * gate + r * ld and up + r * ld (elements; ld % 8 == 0, e.g. the fused
 * gate|up output [rows, 2n] with up = gate + n and ld = 2n); q [rows, n] and
 * scales [rows, n / group_k]. n % 128 == 0; group_k = n needs n <= 16384.
 *
 * group_k is 128 or the row length; q, gate and up 16-byte aligned.
 */
int heph_rmsnorm_quant_fp8(uint8_t* q, float* scales, const uint16_t* x_bf16,
                           const uint16_t* gamma_bf16, int rows, int cols, float eps,
                           int group_k, void* stream);
int heph_silu_mul_quant_fp8(uint8_t* q, float* scales, const uint16_t* gate_bf16,
                            const uint16_t* up_bf16, int rows, int n, int ld, int group_k,
                            void* stream);

/* Workspace sizes heph_fp8_linear needs for (M, K, group_k). */
size_t heph_fp8_q_ws_bytes(int M, int K);
size_t heph_fp8_s_ws_floats(int M, int K, int group_k);

/*
 * Optional larger q_ws for (M, N, K): the activation codes, rounded up to
 * 256 bytes, plus scratch for the fp32 partials of the large-M GEMM when it
 * splits K (M >= 128 and few output tiles, e.g. M = 512 with N = 2560).
 * Passing a q_ws of this size (q_ws_bytes) lets heph_fp8_linear use the
 * part past the codes as that scratch; with the minimal q_ws it does not
 * split. No counterpart in the reference, whose workspaces are sized for
 * the codes and scales only (forward.mojo:121-125).
 */
size_t heph_fp8_linear_ws_bytes(int M, int N, int K);

/* Message for a status code (static storage). */
const char* heph_strerror(int status);

/* HEPH_ABI_VERSION of the built library. */
int heph_abi_version(void);

/*
 * Timing hook: the next heph_fp8_linear / heph_bf16_linear call on the
 * calling thread records start_event at the begin of its first kernel and
 * stop_event at the end of its last kernel (hipEvent_t, stamped through
 * hipExtLaunchKernel); a call that runs one kernel (fused quantization, or
 * SKIP_QUANT) times exactly that kernel. Cleared after one call.
 * No counterpart in the reference; it exists for kernel-duration
 * measurement without a profiler.
 */
int heph_profile_next_launch(void* start_event, void* stop_event);

/* Name of the main kernel the last call on this thread selected. */
const char* heph_last_kernel(void);

/*
 * Launch-shape overrides for one call, for measurement sweeps and the
 * cross-kernel tests; a zero field keeps the built-in choice. The library
 * keeps no tuning state: heph_fp8_linear_with is heph_fp8_linear with the
 * overrides applied to that call only. No counterpart in the reference.
 *   gemv_ks      K-chunk slots per MFMA of the M <= 32 chunk-slot GEMV:
 *                1, 2, 4 or 8 (capped at 16 / rows per slot, i.e. 1 for M > 8)
 *   gemv_waves   its waves per workgroup: 4, 5, 8, 10 or 16 (5 only for
 *                M = 1, 10 for M = 1 and 3 <= M <= 8, 16 only for
 *                8 < M <= 16; 8 is used otherwise)
 *   gemv_u       its steps per load batch: 1 or 2 (1 with 16 waves)
 *   gemm_bm      tile height of the large-M GEMM: 64, 128, 192, 256; 1 selects
 *                the 128x128 GEMM (otherwise used only when M*K or N*K
 *                reaches 2^31)
 *   gemm_bn      tile width of the large-M GEMM: 192, 256 or 320 (tiles
 *                64/128/192/256 x 256, 64/256 x 192, 128 x 320; a gemm_bm and
 *                gemm_bn that form none of these run gemm_bm x 256)
 *   batch_split  the 64-column K-split kernel for M <= 32 with 1x128 groups:
 *                -1 never, n in 1..64 always, with at least n K splits
 *   wide_tiles   the wide-tile batched-decode kernel for M <= 32: -1 never,
 *                1, 2 or 4 always, with 16 x that many output columns per
 *                workgroup (halved until it divides N / 16)
 *   wide_waves   its waves per workgroup: 4, 8 or 16 (16: one column tile)
 *   split_spin_limit  polls of a completion flag before the 64-column
 *                kernel's in-launch split sum gives up (that tile's outputs
 *                are then NaN, see HEPH_SPLIT_STATUS): n > 0 polls, -1 give
 *                up without polling (to exercise that path in tests)
 *   gemv_groups  column groups per workgroup of the chunk-slot GEMV at M = 1
 *                with bf16 rows and four chunk slots: 1 or 2 (2: each
 *                workgroup covers 8 columns and quantizes x once for both
 *                groups); ignored by every other shape
 * Values outside these sets give HEPH_ERR_FLAGS.
 */
typedef struct heph_launch_overrides {
    int gemv_ks;
    int gemv_waves;
    int gemv_u;
    int gemm_bm;
    int batch_split;
    int wide_tiles;
    int wide_waves;
    int split_spin_limit;
    int gemv_groups;
    int gemm_bn;
} heph_launch_overrides;

int heph_fp8_linear_with(void* c, int c_dtype, const uint16_t* x_bf16,
                         const uint8_t* w, const float* w_scale, int w_block_n,
                         int w_block_k, uint8_t* q_ws, size_t q_ws_bytes,
                         float* s_ws, size_t s_ws_floats, int M, int N, int K,
                         int group_k, int flags, void* stream,
                         const heph_launch_overrides* overrides);

#ifdef __cplusplus
}
#endif
#endif /* HEPHFP8_H */
