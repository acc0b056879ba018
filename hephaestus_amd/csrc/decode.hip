// decode.hip - the non-linear ops of one Qwen3 W8A8 decode step, so the FP8
// linear path can be checked end to end (random-init model, greedy argmax).
//
// Each op follows the reference engine's arithmetic (src/hephaestus/
// forward.mojo:359-615 and the kernels it calls); every reduction runs in a
// fixed order that the CPU restatement (oracle/heph_oracle.c) repeats, and
// every rounding step is explicit:
//   * embedding: x = bf16(scale * e4m3(code))               (kernels.mojo:530-548)
//   * RMSNorm: y = bf16(gamma * bf16(x * (1/sqrt(mean(x^2) + eps))))
//     (HF Qwen3RMSNorm, forward.mojo:45-81)
//   * RoPE: split-half pairs (p, p + D/2), cos/sin of the f32 angle rounded
//     to bf16, bf16 after every multiply and add          (kernels.mojo:709-762)
//   * attention: fp32 scores, softmax probabilities rounded to bf16 before
//     the PV product                                       (kernels.mojo:923-1035)
//   * SwiGLU: bf16(bf16(g / (1 + exp(-g))) * up)           (kernels.mojo:1243-1255)
//   * argmax over bf16-rounded logits, lowest index on ties (kernels.mojo:1376-1433)
// The KV cache holds E4M3 codes with one scale per (layer, kv head, K|V):
// new rows are quantized as code = e4m3(clamp(v * (1/s), +-448)).
#include "heph_kernels.h"
#include "../../include/hephdecode.h"

namespace heph {
namespace {

__device__ __forceinline__ float f32_of_bf16(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ float round_bf16(float f) { return f32_of_bf16(f32_to_bf16(f)); }

// OCP E4M3FN code -> float (exact; 0x7F / 0xFF are NaN).
__device__ __forceinline__ float e4m3_value(uint32_t c)
{
    const uint32_t e = (c >> 3) & 15u, m = c & 7u;
    float v = e ? __uint_as_float(((e + 120u) << 23) | (m << 20)) : (float)m * 0x1p-9f;
    if ((c & 0x7Fu) == 0x7Fu) v = __builtin_nanf("");
    return (c & 0x80u) ? -v : v;
}

// float -> E4M3FN code, saturating at +-448 (round to nearest even).
__device__ __forceinline__ uint32_t e4m3_sat(float v)
{
    v = fminf(fmaxf(v, -kE4M3Max), kE4M3Max);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v, v, 0, false) & 0xFFu;
}

// Sum over the 256 threads of a workgroup: s[t] for t < 256 in LDS, folded
// as s[t] += s[t + h] for h = 128, 64, ..., 1 (the order the CPU repeats).
__device__ __forceinline__ float block_sum256(float v, float* s)
{
    const int t = threadIdx.x;
    s[t] = v;
    __syncthreads();
    for (int h = 128; h > 0; h >>= 1) {
        if (t < h) s[t] += s[t + h];
        __syncthreads();
    }
    const float r = s[0];
    __syncthreads();
    return r;
}

// Sum over the 64 lanes of a wave, folded as v[l] += v[l + h] for
// h = 32, 16, ..., 1; the result is lane 0's.
__device__ __forceinline__ float wave_sum64(float v)
{
    for (int h = 32; h > 0; h >>= 1) v += __shfl_down(v, h, 64);
    return __shfl(v, 0, 64);
}

// A token id outside [0, vocab) gives a zero row instead of a read past
// the table (the host cannot see device-side ids).
__global__ __launch_bounds__(256) void embed_fp8_kernel(uint16_t* x, const uint8_t* emb,
                                                        const float* scale, int block,
                                                        const int32_t* tok, int vocab, int hidden)
{
    const int t = blockIdx.y;
    const int d = blockIdx.x * 256 + threadIdx.x;
    if (d >= hidden) return;
    const int32_t raw = tok[t];
    if (raw < 0 || raw >= vocab) {
        x[(size_t)t * hidden + d] = 0;
        return;
    }
    const size_t id = (size_t)raw;
    const float s = block ? scale[(id >> 7) * (size_t)(hidden >> 7) + (d >> 7)] : scale[id];
    x[(size_t)t * hidden + d] = f32_to_bf16(s * e4m3_value(emb[id * hidden + d]));
}

// One workgroup of 256 threads per row; thread t owns elements t, t + 256,
// ... Rows up to kNormMax elements are loaded into registers, x and gamma
// together, every load issued before the first use (one memory round
// trip); longer rows loop.
constexpr int kNormPer = 40;
constexpr int kNormMax = 256 * kNormPer;

__global__ __launch_bounds__(256) void rmsnorm_kernel(uint16_t* out, const uint16_t* in,
                                                      const uint16_t* gamma, int cols, float eps)
{
    __shared__ float red[256];
    const uint16_t* x = in + (size_t)blockIdx.x * cols;
    uint16_t* y = out + (size_t)blockIdx.x * cols;
    const int t = threadIdx.x;
    if (cols <= kNormMax) {
        float v[kNormPer], g[kNormPer];
#pragma unroll
        for (int e = 0; e < kNormPer; ++e) {
            const int i = t + e * 256;
            v[e] = i < cols ? f32_of_bf16(x[i]) : 0.0f;
            g[e] = i < cols ? f32_of_bf16(gamma[i]) : 0.0f;
        }
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < kNormPer; ++e)
            if (t + e * 256 < cols) ss = __builtin_fmaf(v[e], v[e], ss);
        ss = block_sum256(ss, red);
        const float r = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)cols) + eps));
#pragma unroll
        for (int e = 0; e < kNormPer; ++e) {
            const int i = t + e * 256;
            if (i < cols) y[i] = f32_to_bf16(g[e] * round_bf16(v[e] * r));
        }
        return;
    }
    float ss = 0.0f;
    for (int i = t; i < cols; i += 256) {
        const float v = f32_of_bf16(x[i]);
        ss = __builtin_fmaf(v, v, ss);
    }
    ss = block_sum256(ss, red);
    const float r = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)cols) + eps));
    for (int i = t; i < cols; i += 256)
        y[i] = f32_to_bf16(f32_of_bf16(gamma[i]) * round_bf16(f32_of_bf16(x[i]) * r));
}

// RoPE angle for pair p of a D-wide head at position pos, and its bf16 cos
// and sin: freq = f32(pos * theta^(-2p/D)) in double, cos/sin of that f32
// value rounded to f32 then bf16.
__device__ __forceinline__ void rope_cs(int pos, int p, int D, double theta, float& c, float& s)
{
    const float freq = (float)((double)pos * pow(theta, -2.0 * (double)p / (double)D));
    c = round_bf16((float)cos((double)freq));
    s = round_bf16((float)sin((double)freq));
}

// One wave per head (D = 128): lane l holds elements l and l + 64, which is
// exactly RoPE's pair (l, l + 64). Waves 0..H-1 take the q heads (normalized
// and rotated in place), H..H+KVH-1 the k heads (normalized, rotated and
// quantized into the cache slot), H+KVH.. the v heads (quantized).
__global__ __launch_bounds__(64) void qk_norm_rope_kv_kernel(
    uint16_t* qkv, const uint16_t* q_gamma, const uint16_t* k_gamma, uint8_t* k_slot,
    uint8_t* v_slot, const float* kv_inv, int n_heads, int n_kv, int pos, double theta, float eps)
{
    constexpr int D = 128;
    const int h = blockIdx.x;
    const int l = threadIdx.x;
    uint16_t* row = qkv + (size_t)h * D;     // q heads, then k heads, then v heads
    float a = f32_of_bf16(row[l]), b = f32_of_bf16(row[l + 64]);
    if (h >= n_heads + n_kv) {                // v: quantize only
        const int kh = h - n_heads - n_kv;
        const float inv = kv_inv[n_kv + kh];
        v_slot[kh * D + l] = (uint8_t)e4m3_sat(a * inv);
        v_slot[kh * D + l + 64] = (uint8_t)e4m3_sat(b * inv);
        return;
    }
    const uint16_t* gamma = h < n_heads ? q_gamma : k_gamma;
    float ss = a * a;
    ss = __builtin_fmaf(b, b, ss);
    ss = wave_sum64(ss);
    const float r = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)D) + eps));
    a = round_bf16(f32_of_bf16(gamma[l]) * round_bf16(a * r));
    b = round_bf16(f32_of_bf16(gamma[l + 64]) * round_bf16(b * r));
    float c, s;
    rope_cs(pos, l, D, theta, c, s);
    const float re_c = round_bf16(a * c), im_s = round_bf16(b * s);
    const float im_c = round_bf16(b * c), re_s = round_bf16(a * s);
    const float re = round_bf16(re_c - im_s), im = round_bf16(im_c + re_s);
    if (h < n_heads) {
        row[l] = f32_to_bf16(re);
        row[l + 64] = f32_to_bf16(im);
    } else {
        const int kh = h - n_heads;
        const float inv = kv_inv[kh];
        k_slot[kh * D + l] = (uint8_t)e4m3_sat(re * inv);
        k_slot[kh * D + l + 64] = (uint8_t)e4m3_sat(im * inv);
    }
}

// 16 E4M3 codes -> 16 floats with the hardware converter (OCP E4M3FN on
// gfx950, exact).
__device__ __forceinline__ void decode16(const uint4& w, float* f)
{
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)wd[k], false);
        const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)wd[k], true);
        f[4 * k] = lo[0];
        f[4 * k + 1] = lo[1];
        f[4 * k + 2] = hi[0];
        f[4 * k + 3] = hi[1];
    }
}

// Attention over the E4M3 cache runs as three kernels over splits of
// kAttnSplit keys, with scores and per-split sums in a caller workspace:
//   A  scores:  s_j = (sum_d q_d * k_jd, d in order) * sk / sqrt(128)
//   B  softmax: m = max s; sum of e_j = exp(s_j - m) as per-thread sums over
//      j = t, t + 256, ... in order folded across the 256 threads; p_j =
//      bf16(e_j * (1/sum)); then this split's PV: per-thread sums over its
//      keys j = t, t + 256 (in order) folded across threads -> r_split[d]
//   C  out_d = bf16((sum over splits of r_split[d], in split order) * sv)
// The order is fixed by kAttnSplit, not by the launch, and the CPU
// restatement repeats it. Workgroups are numbered so that the query heads
// sharing a kv head and a split land on the same XCD (shared L2).
constexpr int kAttnSplit = 512;

struct AttnMap {
    int h, split;
};

__device__ __forceinline__ AttnMap attn_map(int b, int n_heads, int n_kv, int n_splits)
{
    const int F = n_kv * n_splits;      // (kv head, split) pairs
    const int qi = b / F, f = b % F;
    return {(f / n_splits) * (n_heads / n_kv) + qi, f % n_splits};
}

__global__ __launch_bounds__(256) void attn_scores_kernel(
    float* scores, const uint16_t* q, const uint8_t* kc, const float* kv_scale, int n_heads,
    int n_kv, int n_keys, int n_splits)
{
    constexpr int D = 128;
    const AttnMap m = attn_map(blockIdx.x, n_heads, n_kv, n_splits);
    const int t = threadIdx.x, kh = m.h / (n_heads / n_kv);
    const size_t row = (size_t)n_kv * D;
    float qv[D];
#pragma unroll
    for (int c = 0; c < D / 8; ++c) {
        const uint4 w = ldg16u(q + (size_t)m.h * D + c * 8);
        qv[8 * c] = bf16lo(w.x); qv[8 * c + 1] = bf16hi(w.x);
        qv[8 * c + 2] = bf16lo(w.y); qv[8 * c + 3] = bf16hi(w.y);
        qv[8 * c + 4] = bf16lo(w.z); qv[8 * c + 5] = bf16hi(w.z);
        qv[8 * c + 6] = bf16lo(w.w); qv[8 * c + 7] = bf16hi(w.w);
    }
    const float qk_scale = kv_scale[kh] * 0.08838834764831845f;   // sk * f32(1/sqrt(128))
    const int j0 = m.split * kAttnSplit + t;
    uint4 w[2][8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int j = min(j0 + u * 256, n_keys - 1);
        const uint4* kp = reinterpret_cast<const uint4*>(kc + j * row + kh * D);
#pragma unroll
        for (int c = 0; c < 8; ++c) w[u][c] = kp[c];
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int j = j0 + u * 256;
        float dot = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            float k16[16];
            decode16(w[u][c], k16);
#pragma unroll
            for (int k = 0; k < 16; ++k) dot = __builtin_fmaf(qv[16 * c + k], k16[k], dot);
        }
        if (j < n_keys) scores[(size_t)m.h * n_keys + j] = dot * qk_scale;
    }
}

__global__ __launch_bounds__(256) void attn_pv_kernel(
    float* partial, const float* scores, const uint8_t* vc, int n_heads, int n_kv, int n_keys,
    int n_splits)
{
    constexpr int D = 128, FOLD = 32, PAD = FOLD + 1;
    __shared__ float red[256 * PAD];
    const AttnMap m = attn_map(blockIdx.x, n_heads, n_kv, n_splits);
    const int t = threadIdx.x, kh = m.h / (n_heads / n_kv);
    const size_t row = (size_t)n_kv * D;
    const float* sc = scores + (size_t)m.h * n_keys;

    // V rows of this thread's two keys go out first
    const int j0 = m.split * kAttnSplit + t;
    uint4 w[2][8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int j = min(j0 + u * 256, n_keys - 1);
        const uint4* vp = reinterpret_cast<const uint4*>(vc + j * row + kh * D);
#pragma unroll
        for (int c = 0; c < 8; ++c) w[u][c] = vp[c];
    }
    float mx = -3.4e38f;
    for (int j = t; j < n_keys; j += 256) mx = fmaxf(mx, sc[j]);
    red[t] = mx;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (t < s) red[t] = fmaxf(red[t], red[t + s]);
        __syncthreads();
    }
    mx = red[0];
    __syncthreads();
    float se = 0.0f;
    for (int j = t; j < n_keys; j += 256) se += expf(sc[j] - mx);
    se = block_sum256(se, red);
    const float inv = __fdiv_rn(1.0f, se);

    float acc[D];
#pragma unroll
    for (int d = 0; d < D; ++d) acc[d] = 0.0f;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int j = j0 + u * 256;
        const float pj = j < n_keys ? round_bf16(expf(sc[j] - mx) * inv) : 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            float v16[16];
            decode16(w[u][c], v16);
#pragma unroll
            for (int k = 0; k < 16; ++k) acc[16 * c + k] = __builtin_fmaf(pj, v16[k], acc[16 * c + k]);
        }
    }
    float* dst = partial + ((size_t)m.h * n_splits + m.split) * D;
#pragma unroll
    for (int d0 = 0; d0 < D; d0 += FOLD) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < FOLD; ++i) red[t * PAD + i] = acc[d0 + i];
        __syncthreads();
        for (int s = 128; s > 0; s >>= 1) {
            for (int k = t; k < s * FOLD; k += 256) {
                const int r = k / FOLD, i = k % FOLD;
                red[r * PAD + i] += red[(r + s) * PAD + i];
            }
            __syncthreads();
        }
        if (t < FOLD) dst[d0 + t] = red[t];
    }
}

__global__ __launch_bounds__(128) void attn_combine_kernel(
    uint16_t* out, const float* partial, const float* kv_scale, int n_heads, int n_kv, int n_splits)
{
    const int h = blockIdx.x, d = threadIdx.x;
    const float* p = partial + (size_t)h * n_splits * 128 + d;
    float v = 0.0f;
    for (int s = 0; s < n_splits; ++s) v += p[s * 128];
    out[(size_t)h * 128 + d] = f32_to_bf16(v * kv_scale[n_kv + h / (n_heads / n_kv)]);
}

__global__ __launch_bounds__(256) void silu_mul_kernel(uint16_t* out, const uint16_t* gate,
                                                       const uint16_t* up, int n)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float g = f32_of_bf16(gate[i]);
    const float s = round_bf16(__fdiv_rn(g, 1.0f + expf(-g)));
    out[i] = f32_to_bf16(s * f32_of_bf16(up[i]));
}

// One workgroup of 1024 threads: thread t scans i = t, t + 1024, ... keeping
// the first maximum; then a tree keeps the larger value, or on a tie the
// lower index.
__global__ __launch_bounds__(1024) void argmax_bf16_kernel(int32_t* out, const float* logits, int n)
{
    __shared__ float bv[1024];
    __shared__ int bi[1024];
    const int t = threadIdx.x;
    float best = -3.4e38f;
    int idx = -1;
    for (int i = t; i < n; i += 1024) {
        const float v = round_bf16(logits[i]);
        if (v > best) { best = v; idx = i; }
    }
    bv[t] = best;
    bi[t] = idx;
    __syncthreads();
    for (int h = 512; h > 0; h >>= 1) {
        if (t < h) {
            const float ov = bv[t + h];
            const int oi = bi[t + h];
            if (ov > bv[t] || (ov == bv[t] && oi >= 0 && (bi[t] < 0 || oi < bi[t]))) {
                bv[t] = ov;
                bi[t] = oi;
            }
        }
        __syncthreads();
    }
    if (t == 0) out[0] = bi[0];
}

int status_of(hipError_t e) { return e == hipSuccess ? HEPH_OK : HEPH_ERR_LAUNCH; }

}  // namespace
}  // namespace heph

using namespace heph;

extern "C" {

int heph_embed_fp8(void* x_bf16, const uint8_t* emb, const float* emb_scale, int block,
                   const int32_t* tokens, int n_tok, int vocab, int hidden, void* stream)
{
    if (!x_bf16 || !emb || !emb_scale || !tokens) return HEPH_ERR_NULL;
    if (n_tok < 1 || vocab < 1 || hidden < 128 || hidden % 128) return HEPH_ERR_SHAPE;
    if (int st = check_device()) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    embed_fp8_kernel<<<dim3((hidden + 255) / 256, n_tok), 256, 0, s>>>(
        static_cast<uint16_t*>(x_bf16), emb, emb_scale, block, tokens, vocab, hidden);
    return status_of(hipGetLastError());
}

int heph_rmsnorm(void* out_bf16, const void* in_bf16, const void* gamma_bf16, int rows, int cols,
                 float eps, void* stream)
{
    if (!out_bf16 || !in_bf16 || !gamma_bf16) return HEPH_ERR_NULL;
    if (rows < 1 || cols < 1) return HEPH_ERR_SHAPE;
    if (int st = check_device()) return st;
    rmsnorm_kernel<<<rows, 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<uint16_t*>(out_bf16), static_cast<const uint16_t*>(in_bf16),
        static_cast<const uint16_t*>(gamma_bf16), cols, eps);
    return status_of(hipGetLastError());
}

int heph_qk_norm_rope_kv(void* qkv_bf16, const void* q_gamma, const void* k_gamma,
                         uint8_t* k_slot, uint8_t* v_slot, const float* kv_inv_scale,
                         int n_heads, int n_kv_heads, int head_dim, int pos, double theta,
                         float eps, void* stream)
{
    if (!qkv_bf16 || !q_gamma || !k_gamma || !k_slot || !v_slot || !kv_inv_scale)
        return HEPH_ERR_NULL;
    if (head_dim != 128 || n_kv_heads < 1 || n_heads < n_kv_heads || n_heads % n_kv_heads ||
        pos < 0)
        return HEPH_ERR_SHAPE;
    if (int st = check_device()) return st;
    qk_norm_rope_kv_kernel<<<n_heads + 2 * n_kv_heads, 64, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<uint16_t*>(qkv_bf16), static_cast<const uint16_t*>(q_gamma),
        static_cast<const uint16_t*>(k_gamma), k_slot, v_slot, kv_inv_scale, n_heads,
        n_kv_heads, pos, theta, eps);
    return status_of(hipGetLastError());
}

size_t heph_attention_ws_bytes(int n_heads, int n_keys)
{
    if (n_heads < 1 || n_keys < 1) return 0;
    const size_t splits = (size_t)(n_keys + kAttnSplit - 1) / kAttnSplit;
    return 4 * (size_t)n_heads * ((size_t)n_keys + splits * 128);
}

int heph_attention_fp8kv(void* out_bf16, const void* q_bf16, const uint8_t* k_cache,
                         const uint8_t* v_cache, const float* kv_scale, int n_heads,
                         int n_kv_heads, int head_dim, int n_keys, void* ws, size_t ws_bytes,
                         void* stream)
{
    if (!out_bf16 || !q_bf16 || !k_cache || !v_cache || !kv_scale || !ws) return HEPH_ERR_NULL;
    if (head_dim != 128 || n_kv_heads < 1 || n_heads < n_kv_heads || n_heads % n_kv_heads ||
        n_keys < 1 || n_keys > HEPH_ATTN_MAX_KEYS)
        return HEPH_ERR_SHAPE;
    if (ws_bytes < heph_attention_ws_bytes(n_heads, n_keys)) return HEPH_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(k_cache) % 16 || reinterpret_cast<uintptr_t>(v_cache) % 16 ||
        reinterpret_cast<uintptr_t>(q_bf16) % 16 || reinterpret_cast<uintptr_t>(ws) % 16)
        return HEPH_ERR_ALIGN;
    if (int st = check_device()) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int splits = (n_keys + kAttnSplit - 1) / kAttnSplit;
    float* scores = static_cast<float*>(ws);
    float* partial = scores + (size_t)n_heads * n_keys;
    const int blocks = n_heads * splits;
    attn_scores_kernel<<<blocks, 256, 0, s>>>(scores, static_cast<const uint16_t*>(q_bf16),
                                              k_cache, kv_scale, n_heads, n_kv_heads, n_keys,
                                              splits);
    attn_pv_kernel<<<blocks, 256, 0, s>>>(partial, scores, v_cache, n_heads, n_kv_heads, n_keys,
                                          splits);
    attn_combine_kernel<<<n_heads, 128, 0, s>>>(static_cast<uint16_t*>(out_bf16), partial,
                                                kv_scale, n_heads, n_kv_heads, splits);
    return status_of(hipGetLastError());
}

int heph_silu_mul(void* out_bf16, const void* gate_bf16, const void* up_bf16, int n, void* stream)
{
    if (!out_bf16 || !gate_bf16 || !up_bf16) return HEPH_ERR_NULL;
    if (n < 1) return HEPH_ERR_SHAPE;
    if (int st = check_device()) return st;
    silu_mul_kernel<<<(n + 255) / 256, 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<uint16_t*>(out_bf16), static_cast<const uint16_t*>(gate_bf16),
        static_cast<const uint16_t*>(up_bf16), n);
    return status_of(hipGetLastError());
}

int heph_argmax_bf16(int32_t* out_idx, const float* logits, int n, void* stream)
{
    if (!out_idx || !logits) return HEPH_ERR_NULL;
    if (n < 1) return HEPH_ERR_SHAPE;
    if (int st = check_device()) return st;
    argmax_bf16_kernel<<<1, 1024, 0, static_cast<hipStream_t>(stream)>>>(out_idx, logits, n);
    return status_of(hipGetLastError());
}

}  // extern "C"
