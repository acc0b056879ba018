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

// One workgroup of 256 threads per row.
__global__ __launch_bounds__(256) void rmsnorm_kernel(uint16_t* out, const uint16_t* in,
                                                      const uint16_t* gamma, int cols, float eps)
{
    __shared__ float red[256];
    const uint16_t* x = in + (size_t)blockIdx.x * cols;
    uint16_t* y = out + (size_t)blockIdx.x * cols;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < cols; i += 256) {
        const float v = f32_of_bf16(x[i]);
        ss = __builtin_fmaf(v, v, ss);
    }
    ss = block_sum256(ss, red);
    const float r = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)cols) + eps));
    for (int i = threadIdx.x; i < cols; i += 256) {
        const float v = round_bf16(f32_of_bf16(x[i]) * r);
        y[i] = f32_to_bf16(f32_of_bf16(gamma[i]) * v);
    }
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

// One workgroup (256 threads) per query head; scores live in LDS.
__global__ __launch_bounds__(256) void attention_fp8kv_kernel(
    uint16_t* out, const uint16_t* q, const uint8_t* kc, const uint8_t* vc, const float* kv_scale,
    int n_heads, int n_kv, int n_keys)
{
    constexpr int D = 128;
    __shared__ float qs[D];
    __shared__ float p[HEPH_ATTN_MAX_KEYS];
    __shared__ float red[256];
    __shared__ float part[2][D];
    const int h = blockIdx.x, t = threadIdx.x;
    const int kh = h / (n_heads / n_kv);
    if (t < D) qs[t] = f32_of_bf16(q[(size_t)h * D + t]);
    __syncthreads();
    const size_t row = (size_t)n_kv * D;
    const float qk_scale = kv_scale[kh] * 0.08838834764831845f;   // sk * f32(1/sqrt(128))

    // scores: key j = t, t + 256, ...; dot over d = 0..127 in order
    float mx = -3.4e38f;
    for (int j = t; j < n_keys; j += 256) {
        const uint4* kp = reinterpret_cast<const uint4*>(kc + j * row + kh * D);
        float dot = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint4 w = kp[c];
            const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int k = 0; k < 16; ++k)
                dot = __builtin_fmaf(qs[c * 16 + k], e4m3_value((wd[k >> 2] >> (8 * (k & 3))) & 0xFFu), dot);
        }
        const float sc = dot * qk_scale;
        p[j] = sc;
        mx = fmaxf(mx, sc);
    }
    red[t] = mx;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (t < w) red[t] = fmaxf(red[t], red[t + w]);
        __syncthreads();
    }
    mx = red[0];
    __syncthreads();
    float se = 0.0f;
    for (int j = t; j < n_keys; j += 256) {
        const float e = expf(p[j] - mx);
        p[j] = e;
        se += e;
    }
    se = block_sum256(se, red);
    const float inv = __fdiv_rn(1.0f, se);
    for (int j = t; j < n_keys; j += 256) p[j] = round_bf16(p[j] * inv);
    __syncthreads();

    // PV: thread (d, half) sums keys [half * n/2 ... ) in order
    const int d = t & (D - 1), hf = t >> 7;
    const int mid = (n_keys + 1) >> 1;
    const int j0 = hf ? mid : 0, j1 = hf ? n_keys : mid;
    float acc = 0.0f;
    for (int j = j0; j < j1; ++j)
        acc = __builtin_fmaf(p[j], e4m3_value(vc[j * row + kh * D + d]), acc);
    part[hf][d] = acc;
    __syncthreads();
    if (t < D) out[(size_t)h * D + t] = f32_to_bf16((part[0][t] + part[1][t]) * kv_scale[n_kv + kh]);
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

int heph_attention_fp8kv(void* out_bf16, const void* q_bf16, const uint8_t* k_cache,
                         const uint8_t* v_cache, const float* kv_scale, int n_heads,
                         int n_kv_heads, int head_dim, int n_keys, void* stream)
{
    if (!out_bf16 || !q_bf16 || !k_cache || !v_cache || !kv_scale) return HEPH_ERR_NULL;
    if (head_dim != 128 || n_kv_heads < 1 || n_heads < n_kv_heads || n_heads % n_kv_heads ||
        n_keys < 1 || n_keys > HEPH_ATTN_MAX_KEYS)
        return HEPH_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(k_cache) % 16) return HEPH_ERR_ALIGN;
    if (int st = check_device()) return st;
    attention_fp8kv_kernel<<<n_heads, 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<uint16_t*>(out_bf16), static_cast<const uint16_t*>(q_bf16), k_cache, v_cache,
        kv_scale, n_heads, n_kv_heads, n_keys);
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
