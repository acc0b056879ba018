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

// Sum over the 64 lanes of a wave, folded as v[l] += v[l + h] for
// h = 32, 16, ..., 1; the result is lane 0's.
__device__ __forceinline__ float wave_sum64(float v) { return wave_fold_sum64(v); }

// Max over the 64 lanes of a wave (exact in any order), in every lane.
__device__ __forceinline__ float wave_max64(float v) { return wave_fold_max64(v); }

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
// ... and sums their squares in that order (fma); the 256 sums are folded
// as s[t] += s[t + h] for h = 128, 64, ..., 1. The first two levels are read
// by wave 0 from LDS as (s[t] + s[t+128]) + (s[t+64] + s[t+192]), the rest
// move between its lanes: two barriers in all. Rows up to 256 * PER
// elements hold x and gamma in registers, every load issued before the
// first use; longer rows loop.
template <int PER>
__global__ __launch_bounds__(256) void rmsnorm_kernel(uint16_t* out, const uint16_t* in,
                                                      const uint16_t* gamma, int cols, float eps)
{
    __shared__ float red[256];
    __shared__ float res;
    const uint16_t* x = in + (size_t)blockIdx.x * cols;
    uint16_t* y = out + (size_t)blockIdx.x * cols;
    const int t = threadIdx.x;
    if constexpr (PER > 0) {
        float v[PER], g[PER];
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int i = t + e * 256;
            v[e] = i < cols ? f32_of_bf16(x[i]) : 0.0f;
            g[e] = i < cols ? f32_of_bf16(gamma[i]) : 0.0f;
        }
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < PER; ++e)
            if (t + e * 256 < cols) ss = __builtin_fmaf(v[e], v[e], ss);
        const float r = rms_inv(fold256_wave0(ss, red, &res), cols, eps);
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int i = t + e * 256;
            if (i < cols) y[i] = f32_to_bf16(g[e] * round_bf16(v[e] * r));
        }
    } else {
        float ss = 0.0f;
        for (int i = t; i < cols; i += 256) {
            const float v = f32_of_bf16(x[i]);
            ss = __builtin_fmaf(v, v, ss);
        }
        const float r = rms_inv(fold256_wave0(ss, red, &res), cols, eps);
        for (int i = t; i < cols; i += 256)
            y[i] = f32_to_bf16(f32_of_bf16(gamma[i]) * round_bf16(f32_of_bf16(x[i]) * r));
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

// The RoPE table: row pos holds (cos, sin) of pairs 0..D/2-1 as bf16
// patterns, the values rope_cs gives. One thread per (pos, pair).
__global__ __launch_bounds__(256) void rope_table_kernel(uint16_t* table, int n_pos, int D,
                                                         double theta)
{
    const int half = D / 2;
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)n_pos * half) return;
    const int pos = (int)(i / half), p = (int)(i % half);
    float c, s;
    rope_cs(pos, p, D, theta, c, s);
    table[2 * i] = f32_to_bf16(c);
    table[2 * i + 1] = f32_to_bf16(s);
}

// Per-head RMSNorm and RoPE of a 128-wide head over one wave: lane l holds
// elements a = x[l] and b = x[l + 64], which is exactly RoPE's pair
// (l, l + 64); (c, s) are that pair's bf16 cos and sin. On return a and b
// hold the rotated pair (bf16 values): y = bf16(gamma * bf16(x * r)) with
// r = 1/sqrt(mean(x^2) + eps), then re = bf16(bf16(a c) - bf16(b s)),
// im = bf16(bf16(b c) + bf16(a s)).
// head_norm_rope after the sum of squares: ss = the wave's fold of
// a*a + b*b (fma), as wave_sum64 forms it.
__device__ __forceinline__ void head_finish(float& a, float& b, float g_lo, float g_hi,
                                            float c, float s, float eps, float ss)
{
    constexpr int D = 128;
    const float r = __fdiv_rn(1.0f, sqrt_rn(__fdiv_rn(ss, (float)D) + eps));
    a = round_bf16(g_lo * round_bf16(a * r));
    b = round_bf16(g_hi * round_bf16(b * r));
    const float re_c = round_bf16(a * c), im_s = round_bf16(b * s);
    const float im_c = round_bf16(b * c), re_s = round_bf16(a * s);
    a = round_bf16(re_c - im_s);
    b = round_bf16(im_c + re_s);
}

__device__ __forceinline__ void head_norm_rope(float& a, float& b, float g_lo, float g_hi,
                                               float c, float s, float eps)
{
    float ss = a * a;
    ss = __builtin_fmaf(b, b, ss);
    head_finish(a, b, g_lo, g_hi, c, s, eps, wave_sum64(ss));
}

// The V cache in 64-key blocks: key j, kv head kh, dim d at byte
//   ((j / 64 * n_kv + kh) * 8 + d / 16) * 1024 + (j % 64) * 16 + d % 16,
// i.e. [n_keys / 64][n_kv][8 dim chunks][64 keys][16 dims]: the 64 keys of
// one block and one 16-dim chunk are 1 KB in a row, which one wave of the
// values kernel reads with one 16-byte load per lane. Whole blocks are
// allocated (the keys of the last block past n_keys are padding).
constexpr int kVBlock = 64;
__host__ __device__ __forceinline__ size_t vblk_off(int j, int kh, int d, int n_kv)
{
    return ((((size_t)(j / kVBlock) * n_kv + kh) * 8 + d / 16) << 10) + (j % kVBlock) * 16 + d % 16;
}

// One wave per head (D = 128), lane l holding elements l and l + 64. Waves
// 0..H-1 take the q heads (normalized and rotated in place), H..H+KVH-1 the
// k heads (normalized, rotated and quantized into K cache row pos),
// H+KVH.. the v heads (quantized into V cache position pos).
__global__ __launch_bounds__(64) void qk_norm_rope_kv_kernel(
    uint16_t* qkv, const uint16_t* q_gamma, const uint16_t* k_gamma, uint8_t* k_cache,
    uint8_t* v_cache, const float* kv_inv, int n_heads, int n_kv, int pos, double theta, float eps)
{
    constexpr int D = 128;
    const int h = blockIdx.x;
    const int l = threadIdx.x;
    uint16_t* row = qkv + (size_t)h * D;     // q heads, then k heads, then v heads
    float a = f32_of_bf16(row[l]), b = f32_of_bf16(row[l + 64]);
    if (h >= n_heads + n_kv) {                // v: quantize only
        const int kh = h - n_heads - n_kv;
        const float inv = kv_inv[n_kv + kh];
        v_cache[vblk_off(pos, kh, l, n_kv)] = (uint8_t)e4m3_sat(a * inv);
        v_cache[vblk_off(pos, kh, l + 64, n_kv)] = (uint8_t)e4m3_sat(b * inv);
        return;
    }
    const uint16_t* gamma = h < n_heads ? q_gamma : k_gamma;
    float c, s;
    rope_cs(pos, l, D, theta, c, s);
    head_norm_rope(a, b, f32_of_bf16(gamma[l]), f32_of_bf16(gamma[l + 64]), c, s, eps);
    if (h < n_heads) {
        row[l] = f32_to_bf16(a);
        row[l + 64] = f32_to_bf16(b);
    } else {
        const int kh = h - n_heads;
        const float inv = kv_inv[kh];
        uint8_t* k_slot = k_cache + (size_t)pos * n_kv * D;
        k_slot[kh * D + l] = (uint8_t)e4m3_sat(a * inv);
        k_slot[kh * D + l + 64] = (uint8_t)e4m3_sat(b * inv);
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

// Attention over the E4M3 cache in two kernels:
//   A  scores, one workgroup per (kv head, split of kAttnSplit keys) serving
//      the G query heads that share the kv head (every K byte read once):
//      thread t holds dims 16c .. 16c+15 (c = t & 7) of keys
//      j = kAttnSplit*split + (t >> 3) + (kAttnSplit/kAttnKPT)*i
//      (i < kAttnKPT), one 16-byte load each (eight lanes read a key's
//      128-byte row). Per head g:
//        part_c = sum over those 16 dims in order (fma), then
//        s_j = (((p0+p1)+(p2+p3)) + ((p4+p5)+(p6+p7))) * (sk * f32(1/sqrt(128)))
//      written to the workspace
//   B  values, one workgroup per (query head, 16-dim chunk) over all keys
//      (attn_values_kernel): the global max m and sum of exp(s_j - m) over
//      the head's keys, p_j = bf16(exp(s_j - m) * (1/sum)) (the reference's
//      probability, kernels.mojo:1003-1019, global max and sum), and
//      out_d = bf16(sum over keys of p_j * v_j[d] * sv), in the orders that
//      kernel states.
// A workgroup of B reads the scores of one head and one 16-byte chunk of
// each of its kv head's V rows; the softmax statistics and each output need
// every key, and finishing them in one workgroup replaces per-split
// statistics and a third launch that summed per-split partial outputs. The
// CPU restatement repeats every order above.
// Keys per split and per thread of the scores kernel: the split's keys sit
// in kAttnSplit / kAttnKPT key slots of 8 lanes, a workgroup of
// 8 * kAttnSplit / kAttnKPT threads; a score's arithmetic does not depend
// on either. On MI355X at 4097 keys (graph-replayed decode step, ms per
// token): 256 keys x 2 per thread (136 workgroups of 1024 threads) 1.682,
// 256 x 4 1.687, 128 x 4 1.727, 64 x 2 1.712, 512 x 4 1.743, 256 x 8 1.727:
// fewer workgroups each prepare the query heads once for more keys.
constexpr int kAttnSplit = 256;
constexpr int kAttnKPT = 2;

// The workspace holds the scores [n_heads][n_keys] (fp32).

// Sum of 16 per-wave values: pairs (2u, 2u + 1), then
// ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7)).
__device__ __forceinline__ float sum16_waves(const float* r)
{
    float r8[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) r8[u] = r[2 * u] + r[2 * u + 1];
    return ((r8[0] + r8[1]) + (r8[2] + r8[3])) + ((r8[4] + r8[5]) + (r8[6] + r8[7]));
}

// x + (the value of lane l ^ 1, l ^ 2 or l ^ 4 within each 8-lane group),
// i.e. one level of the 8-lane butterfly (quad_perm [1,0,3,2], [2,3,0,1],
// row_half_mirror: lane l pairs with 7 - l, the other quad).
template <int CTRL>
__device__ __forceinline__ float dpp_add(float x)
{
    return x + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}

// The token's q/k/v preparation done by the scores kernel in its QKV form
// (heph_attention_qkv_fp8kv): the raw projection row, the per-head norm
// gammas, the cache rows of the new key (position n_keys - 1) and the
// inverse K|V scales.
struct QkvPrep {
    const uint16_t* qkv;     // [n_heads + 2 n_kv, 128] bf16: q heads, k heads, v heads
    const uint16_t* q_gamma;
    const uint16_t* k_gamma;
    uint8_t* k_slot;         // [n_kv, 128] codes of the new key (its K cache row)
    uint8_t* v_cache;        // the blocked V cache; the new key is position n_keys - 1
    const float* kv_inv;     // n_kv K entries, then n_kv V entries
    const uint16_t* rope;    // (cos, sin) bf16 of the 64 pairs at the new key's
                             // position, or nullptr: computed here (rope_cs)
    int n_heads;
    double theta;
    float eps;
};

// QKV form: the workgroup first prepares what qk_norm_rope_kv_kernel would
// have left in memory, with the same arithmetic (head_norm_rope): its G
// query heads, and in the split holding the new key (the last) that key's
// k and v rows, quantized into the cache (the values kernel reads v from
// there). The G q heads and the new key's k go round-robin to the NW
// waves, every raw load issued before the first reduction, a wave's heads
// folded together; v takes one element per thread; the rotated
// q heads and the new key's codes meet in LDS after one barrier, and the
// new key's score uses those codes instead of the cache row loaded at the
// start. All of it runs while the cache loads are in flight.
template <int G, bool QKV, int KPT>
__global__ __launch_bounds__(8 * kAttnSplit / KPT) void attn_scores_kernel(
    float* ws, const uint16_t* q, const uint8_t* kc, const float* kv_scale, int n_kv,
    int n_keys, int n_splits, QkvPrep prep)
{
    constexpr int D = 128;
    constexpr int SLOTS = kAttnSplit / KPT, NW = SLOTS / 8;   // key slots, waves
    const int kh = blockIdx.x % n_kv, split = blockIdx.x / n_kv;
    const int t = threadIdx.x, ks = t >> 3, c = t & 7;
    const size_t row = (size_t)n_kv * D;
    const int j0 = split * kAttnSplit + ks;
    // The cache rows go out after the loads of q (or of the raw projection
    // row and the norm gammas): a wave's loads complete in issue order, and
    // the q preparation, which needs only those, then runs while the cache
    // rows are in flight.
    uint4 kv[KPT];
    auto load_keys = [&]() {
#pragma unroll
        for (int i = 0; i < KPT; ++i)
            kv[i] = ldg16u(kc + (size_t)min(j0 + SLOTS * i, n_keys - 1) * row + kh * D + 16 * c);
    };
    float qv[G][16];
    if constexpr (QKV) {
        // normalized heads: items 0..G-1 the q heads kh*G + g, item G the
        // new key's k row (last split only), round-robin over the NW
        // waves; a wave's heads fold their sums of squares together (the
        // same per-head order as wave_sum64). The new key's v row is
        // quantized one element per thread.
        constexpr int NI = (G + 1 + NW - 1) / NW;
        __shared__ __attribute__((aligned(16))) uint16_t qs[G][D];
        __shared__ __attribute__((aligned(16))) uint8_t knew[D];
        const int wave = t >> 6, l = t & 63;
        const bool last = split == n_splits - 1;
        const int items = last ? G + 1 : G;
        uint32_t rcs = 0;
        if (prep.rope) rcs = reinterpret_cast<const uint32_t*>(prep.rope)[l];
        float vx = 0.0f;
        if (last && t < D) vx = f32_of_bf16(prep.qkv[(size_t)(prep.n_heads + n_kv + kh) * D + t]);
        float xa[NI], xb[NI], ga[NI], gb[NI];
#pragma unroll
        for (int k = 0; k < NI; ++k) {
            const int it = wave + NW * k;
            xa[k] = xb[k] = ga[k] = gb[k] = 0.0f;
            if (it < items) {
                const int h = it < G ? kh * G + it : prep.n_heads + kh;
                const uint16_t* r = prep.qkv + (size_t)h * D;
                const uint16_t* gm = it < G ? prep.q_gamma : prep.k_gamma;
                xa[k] = f32_of_bf16(r[l]);
                xb[k] = f32_of_bf16(r[l + 64]);
                ga[k] = f32_of_bf16(gm[l]);
                gb[k] = f32_of_bf16(gm[l + 64]);
            }
        }
        load_keys();
        float cs, sn;
        if (prep.rope) {
            cs = bf16lo(rcs);
            sn = bf16hi(rcs);
        } else {
            rope_cs(n_keys - 1, l, D, prep.theta, cs, sn);
        }
        float ss[NI];
#pragma unroll
        for (int k = 0; k < NI; ++k)
            ss[k] = wave_sum64(__builtin_fmaf(xb[k], xb[k], xa[k] * xa[k]));
#pragma unroll
        for (int k = 0; k < NI; ++k) {
            const int it = wave + NW * k;
            if (it >= items) break;
            float a = xa[k], b = xb[k];
            head_finish(a, b, ga[k], gb[k], cs, sn, prep.eps, ss[k]);
            if (it < G) {
                qs[it][l] = f32_to_bf16(a);
                qs[it][l + 64] = f32_to_bf16(b);
            } else {
                const float inv = prep.kv_inv[kh];
                const uint8_t lo = (uint8_t)e4m3_sat(a * inv), hi = (uint8_t)e4m3_sat(b * inv);
                prep.k_slot[kh * D + l] = lo;
                prep.k_slot[kh * D + l + 64] = hi;
                knew[l] = lo;
                knew[l + 64] = hi;
            }
        }
        if (last && t < D)
            prep.v_cache[vblk_off(n_keys - 1, kh, t, n_kv)] =
                (uint8_t)e4m3_sat(vx * prep.kv_inv[n_kv + kh]);
        __syncthreads();
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const uint4 a = *reinterpret_cast<const uint4*>(&qs[g][16 * c]);
            const uint4 b = *reinterpret_cast<const uint4*>(&qs[g][16 * c + 8]);
            const uint32_t d[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                qv[g][2 * e] = bf16lo(d[e]);
                qv[g][2 * e + 1] = bf16hi(d[e]);
            }
        }
        // the new key (and the clamped indices past it) takes the codes
        // just computed, not the cache row read before they were written
        if (last) {
#pragma unroll
            for (int i = 0; i < KPT; ++i)
                if (j0 + SLOTS * i >= n_keys - 1)
                    kv[i] = *reinterpret_cast<const uint4*>(&knew[16 * c]);
        }
    } else {
        uint4 qa[G], qb[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const uint16_t* qp = q + (size_t)(kh * G + g) * D + 16 * c;
            qa[g] = ldg16u(qp);
            qb[g] = ldg16u(qp + 8);
        }
        load_keys();
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const uint4 a = qa[g], b = qb[g];
            const uint32_t d[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                qv[g][2 * e] = bf16lo(d[e]);
                qv[g][2 * e + 1] = bf16hi(d[e]);
            }
        }
    }
    const float qk_scale = kv_scale[kh] * 0.08838834764831845f;   // sk * f32(1/sqrt(128))
    float sc[KPT][G];
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
        float k16[16];
        decode16(kv[i], k16);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float part = 0.0f;
#pragma unroll
            for (int e = 0; e < 16; ++e) part = __builtin_fmaf(qv[g][e], k16[e], part);
            part = dpp_add<0xB1>(part);
            part = dpp_add<0x4E>(part);
            part = dpp_add<0x141>(part);
            sc[i][g] = part * qk_scale;
        }
    }
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
        const int j = j0 + SLOTS * i;
#pragma unroll
        for (int g = 0; g < G; ++g)
            if (c == g && j < n_keys) ws[(size_t)(kh * G + g) * n_keys + j] = sc[i][g];
    }
}

// Values: one workgroup per (query head, 16-dim chunk) over all the keys,
// so each output is finished inside the workgroup. Wave w takes the 64-key
// blocks b = w, w + 16, w + 32, ... (lane l key 64b + l, one 16-byte load
// of the block's chunk), kValBlocks blocks per pass with every load of a
// pass in flight, the next pass issued before the current one is used.
constexpr int kValWaves = 16;
constexpr int kValBlocks = 5;
static_assert(kValWaves == 16, "sum16_waves folds 16 waves");

// ONE: n_keys <= kValWaves * kValBlocks * 64, one pass (its own kernel, so
// that the register allocation of the common case is its own).
template <int G, bool ONE>
__global__ __launch_bounds__(64 * kValWaves) void attn_values_kernel(
    uint16_t* out, const float* ws, const uint8_t* vc, const float* kv_scale, int n_kv,
    int n_keys)
{
    constexpr int NW = kValWaves, NB = kValBlocks;
    // kv head kh's workgroups are blockIdx kh + n_kv * i: with 8 kv heads
    // they share one XCD (and its L2) with each other and with the scores
    // kernel's workgroups of kh, which use the same rule
    const int kh = blockIdx.x % n_kv, i = blockIdx.x / n_kv;
    const int g = i % G, c = i / G, h = kh * G + g;
    const int t = threadIdx.x, l = t & 63, wave = t >> 6;
    const int n_blocks = (n_keys + kVBlock - 1) / kVBlock;
    const int n_pass = ONE ? 1 : (n_blocks + NW * NB - 1) / (NW * NB);
    const float* sh = ws + (size_t)h * n_keys;
    const uint8_t* vh = vc + vblk_off(l, kh, 16 * c, n_kv);
    const size_t vstep = (size_t)n_kv * 8 * 1024;   // bytes per 64-key block

    // Loads in the order their data is needed (a wave's loads complete in
    // issue order): the scores (written by the scores kernel, near in the
    // cache hierarchy), then the V blocks (HBM).
    float sa[NB], sb[NB];
    uint4 va[NB], vb[NB];
    auto issue = [&](int pass, float (&sj)[NB], uint4 (&vv)[NB]) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            const int b = (pass * NB + k) * NW + wave;
            if (b < n_blocks) sj[k] = sh[min(kVBlock * b + l, n_keys - 1)];
        }
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            const int b = (pass * NB + k) * NW + wave;
            if (b < n_blocks) vv[k] = ldg16u(vh + b * vstep);
        }
    };
    if (ONE) issue(0, sa, va);

    // The head's max m and sum of exp(s_j - m) over all its keys: per lane
    // over its keys in block order (the sum by plain adds), then over the
    // wave (wave_max64 / wave_sum64), then over the 16 waves in LDS (the sum
    // as sum16_waves). With one pass (n_keys <= 16 * 5 * 64) every score is
    // already in registers; longer contexts read the scores again.
    __shared__ float red[2][NW];
    float mx = -3.4e38f;
    if (ONE) {
#pragma unroll
        for (int k = 0; k < NB; ++k)
            if (kVBlock * (k * NW + wave) + l < n_keys) mx = fmaxf(mx, sa[k]);
    } else {
        for (int j = kVBlock * wave + l; j < n_keys; j += kVBlock * NW) mx = fmaxf(mx, sh[j]);
    }
    mx = wave_max64(mx);
    if (l == 0) red[0][wave] = mx;
    __syncthreads();
    float m = red[0][0];
#pragma unroll
    for (int v = 1; v < NW; ++v) m = fmaxf(m, red[0][v]);
    float a = 0.0f;
    if (ONE) {   // sa then holds exp(s_j - m)
#pragma unroll
        for (int k = 0; k < NB; ++k)
            if (kVBlock * (k * NW + wave) + l < n_keys) {
                sa[k] = expf(sa[k] - m);
                a += sa[k];
            }
    } else {
        for (int j = kVBlock * wave + l; j < n_keys; j += kVBlock * NW) a += expf(sh[j] - m);
    }
    a = wave_sum64(a);
    if (l == 0) red[1][wave] = a;
    __syncthreads();
    const float inv = __fdiv_rn(1.0f, sum16_waves(red[1]));

    // p_j = bf16(exp(s_j - m) * inv) (the reference's probability,
    // kernels.mojo:1003-1019); per lane an fma chain over its keys in block
    // order; keys past n_keys (the last block's padding) are skipped
    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
    // (have_e: sj holds exp(s_j - m) already)
    auto consume = [&](int pass, const float (&sj)[NB], const uint4 (&vv)[NB], bool have_e)
        __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            const int j = kVBlock * ((pass * NB + k) * NW + wave) + l;
            if (j < n_keys) {
                const float pj = round_bf16((have_e ? sj[k] : expf(sj[k] - m)) * inv);
                float v16[16];
                decode16(vv[k], v16);
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[e] = __builtin_fmaf(pj, v16[e], acc[e]);
            }
        }
    };
    if (ONE) {
        consume(0, sa, va, true);
    } else {
        issue(0, sa, va);
        for (int p = 0; p < n_pass; p += 2) {
            if (p + 1 < n_pass) issue(p + 1, sb, vb);
            consume(p, sa, va, false);
            if (p + 1 >= n_pass) break;
            if (p + 2 < n_pass) issue(p + 2, sa, va);
            consume(p + 1, sb, vb, false);
        }
    }

    // Sum of the 16 values over the 64 lanes, halving the values per lane at
    // each level: lanes l, l ^ 32 by v_permlane32_swap (the lower half keeps
    // values 0-7), l ^ 16 by v_permlane16_swap (even rows keep the first
    // half), l ^ 8 by row_ror:8 and l, 7 - l within 8 lanes by
    // row_half_mirror (each lane sending the half its partner keeps), then
    // l ^ 2 and l ^ 1 on the one value left. Lane l ends with value
    // 8*bit5 + 4*bit4 + 2*bit3 + bit2 of l, summed (with x_k the lane sums
    // and T_q = ((x_q + x_q+32) + (x_q+16 + x_q+48)) + ((x_q+8 + x_q+40) +
    // (x_q+24 + x_q+56))) as ((T0 + T7) + (T2 + T5)) + ((T1 + T6) + (T3 + T4)).
    float h8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[e]),
                                                        __float_as_uint(acc[e + 8]), false, false);
        h8[e] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    float h4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(h8[e]),
                                                        __float_as_uint(h8[e + 4]), false, false);
        h4[e] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    const bool b3 = l & 8, b2 = l & 4;
    float h2[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const float send = b3 ? h4[e] : h4[e + 2], keep = b3 ? h4[e + 2] : h4[e];
        h2[e] = keep + __int_as_float(
                           __builtin_amdgcn_mov_dpp(__float_as_int(send), 0x128, 0xf, 0xf, false));
    }
    float h1;
    {
        const float send = b2 ? h2[0] : h2[1], keep = b2 ? h2[1] : h2[0];
        h1 = keep + __int_as_float(
                        __builtin_amdgcn_mov_dpp(__float_as_int(send), 0x141, 0xf, 0xf, false));
    }
    h1 = dpp_add<0x4E>(h1);
    h1 = dpp_add<0xB1>(h1);
    // the 16 waves: pairs (2u, 2u + 1), then ((r0 + r1) + (r2 + r3)) +
    // ((r4 + r5) + (r6 + r7)); times the V scale, bf16
    __shared__ float wsum[NW][16];
    if ((l & 3) == 0) wsum[wave][8 * (l >> 5) + 4 * ((l >> 4) & 1) + 2 * b3 + b2] = h1;
    __syncthreads();
    if (t < 16) {
        float r[NW];
#pragma unroll
        for (int v = 0; v < NW; ++v) r[v] = wsum[v][t];
        out[(size_t)h * 128 + 16 * c + t] = f32_to_bf16(sum16_waves(r) * kv_scale[n_kv + kh]);
    }
}

__global__ __launch_bounds__(256) void silu_mul_kernel(uint16_t* out, const uint16_t* gate,
                                                       const uint16_t* up, int n)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    out[i] = (uint16_t)swiglu_bits(gate[i], up[i]);
}

// argmax over bf16-rounded logits, lowest index on ties, in two kernels:
// workgroup b of the first takes the kArgChunk logits from b * kArgChunk
// (thread t: b * kArgChunk + t + 256k, k < 8, in order, keeping the first
// maximum) and leaves its (value, index) in the workspace; the second
// reduces those. A pair beats another with a larger value, or an equal one
// and a lower index (index -1: nothing found, e.g. all NaN); the rule is
// associative and commutative, so any reduction order gives the same pair.
constexpr int kArgChunk = 2048;

struct ArgPair {
    float v;
    int i;
};

__device__ __forceinline__ ArgPair arg_better(ArgPair a, ArgPair b)
{
    if (b.v > a.v || (b.v == a.v && b.i >= 0 && (a.i < 0 || b.i < a.i))) return b;
    return a;
}

__device__ __forceinline__ ArgPair arg_block256(ArgPair p, ArgPair* lds)
{
    for (int h = 32; h > 0; h >>= 1) {
        ArgPair o;
        o.v = __shfl_xor(p.v, h, 64);
        o.i = __shfl_xor(p.i, h, 64);
        p = arg_better(p, o);
    }
    const int t = threadIdx.x;
    if ((t & 63) == 0) lds[t >> 6] = p;
    __syncthreads();
    return arg_better(arg_better(lds[0], lds[1]), arg_better(lds[2], lds[3]));
}

__global__ __launch_bounds__(256) void argmax_part_kernel(ArgPair* part, const float* logits, int n)
{
    __shared__ ArgPair lds[4];
    const int base = blockIdx.x * kArgChunk + threadIdx.x;
    float x[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = logits[min(base + 256 * k, n - 1)];
    ArgPair p{-3.4e38f, -1};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float v = round_bf16(x[k]);
        if (base + 256 * k < n && v > p.v) p = ArgPair{v, base + 256 * k};
    }
    p = arg_block256(p, lds);
    if (threadIdx.x == 0) part[blockIdx.x] = p;
}

__global__ __launch_bounds__(256) void argmax_final_kernel(int32_t* out, const ArgPair* part, int nb)
{
    __shared__ ArgPair lds[4];
    ArgPair p{-3.4e38f, -1};
    for (int b = threadIdx.x; b < nb; b += 256) p = arg_better(p, part[b]);
    p = arg_block256(p, lds);
    if (threadIdx.x == 0) out[0] = p.i;
}

int status_of(hipError_t e) { return e == hipSuccess ? HEPH_OK : HEPH_ERR_LAUNCH; }

// prep.qkv set: the QKV form of the scores kernel (q, k and v prepared
// inside; q is then not read).
template <int G>
hipError_t launch_attention(uint16_t* out, const uint16_t* q, const uint8_t* kc, const uint8_t* vc,
                            const float* kv_scale, int n_kv, int n_keys, float* ws, hipStream_t s,
                            const QkvPrep& prep = QkvPrep{})
{
    const int splits = (n_keys + kAttnSplit - 1) / kAttnSplit;
    const int blocks = n_kv * splits;
    constexpr int NT = 8 * kAttnSplit / kAttnKPT;
    if (prep.qkv)
        attn_scores_kernel<G, true, kAttnKPT><<<blocks, NT, 0, s>>>(ws, q, kc, kv_scale, n_kv,
                                                                   n_keys, splits, prep);
    else
        attn_scores_kernel<G, false, kAttnKPT><<<blocks, NT, 0, s>>>(ws, q, kc, kv_scale, n_kv,
                                                                    n_keys, splits, prep);
    if (n_keys <= kValWaves * kValBlocks * kVBlock)
        attn_values_kernel<G, true><<<n_kv * G * 8, 64 * kValWaves, 0, s>>>(out, ws, vc, kv_scale,
                                                                            n_kv, n_keys);
    else
        attn_values_kernel<G, false><<<n_kv * G * 8, 64 * kValWaves, 0, s>>>(out, ws, vc, kv_scale,
                                                                             n_kv, n_keys);
    return hipGetLastError();
}

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
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint16_t* o = static_cast<uint16_t*>(out_bf16);
    const uint16_t* x = static_cast<const uint16_t*>(in_bf16);
    const uint16_t* g = static_cast<const uint16_t*>(gamma_bf16);
    const int per = (cols + 255) / 256;      // elements per thread
    if (per <= 1) rmsnorm_kernel<1><<<rows, 256, 0, s>>>(o, x, g, cols, eps);
    else if (per <= 2) rmsnorm_kernel<2><<<rows, 256, 0, s>>>(o, x, g, cols, eps);
    else if (per <= 4) rmsnorm_kernel<4><<<rows, 256, 0, s>>>(o, x, g, cols, eps);
    else if (per <= 10) rmsnorm_kernel<10><<<rows, 256, 0, s>>>(o, x, g, cols, eps);
    else if (per <= 16) rmsnorm_kernel<16><<<rows, 256, 0, s>>>(o, x, g, cols, eps);
    else if (per <= 40) rmsnorm_kernel<40><<<rows, 256, 0, s>>>(o, x, g, cols, eps);
    else rmsnorm_kernel<0><<<rows, 256, 0, s>>>(o, x, g, cols, eps);
    return status_of(hipGetLastError());
}

int heph_qk_norm_rope_kv(void* qkv_bf16, const void* q_gamma, const void* k_gamma,
                         uint8_t* k_cache, uint8_t* v_cache, const float* kv_inv_scale,
                         int n_heads, int n_kv_heads, int head_dim, int pos, double theta,
                         float eps, void* stream)
{
    if (!qkv_bf16 || !q_gamma || !k_gamma || !k_cache || !v_cache || !kv_inv_scale)
        return HEPH_ERR_NULL;
    if (head_dim != 128 || n_kv_heads < 1 || n_heads < n_kv_heads || n_heads % n_kv_heads ||
        pos < 0)
        return HEPH_ERR_SHAPE;
    if (int st = check_device()) return st;
    qk_norm_rope_kv_kernel<<<n_heads + 2 * n_kv_heads, 64, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<uint16_t*>(qkv_bf16), static_cast<const uint16_t*>(q_gamma),
        static_cast<const uint16_t*>(k_gamma), k_cache, v_cache, kv_inv_scale, n_heads,
        n_kv_heads, pos, theta, eps);
    return status_of(hipGetLastError());
}

int heph_rope_table_bf16(void* table_bf16, int n_pos, int head_dim, double theta, void* stream)
{
    if (!table_bf16) return HEPH_ERR_NULL;
    if (n_pos < 1 || n_pos > HEPH_ATTN_MAX_KEYS || head_dim != 128) return HEPH_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(table_bf16) % 4) return HEPH_ERR_ALIGN;
    if (int st = check_device()) return st;
    const long n = (long)n_pos * (head_dim / 2);
    rope_table_kernel<<<(unsigned)((n + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<uint16_t*>(table_bf16), n_pos, head_dim, theta);
    return status_of(hipGetLastError());
}

size_t heph_attention_ws_bytes(int n_heads, int n_keys)
{
    if (n_heads < 1 || n_keys < 1) return 0;
    return 4 * (size_t)n_heads * (size_t)n_keys;
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
    const int G = n_heads / n_kv_heads;
    if (G != 1 && G != 2 && G != 4 && G != 8) return HEPH_ERR_SHAPE;
    if (ws_bytes < heph_attention_ws_bytes(n_heads, n_keys)) return HEPH_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(k_cache) % 16 || reinterpret_cast<uintptr_t>(v_cache) % 16 ||
        reinterpret_cast<uintptr_t>(q_bf16) % 16 || reinterpret_cast<uintptr_t>(ws) % 16)
        return HEPH_ERR_ALIGN;
    if (int st = check_device()) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint16_t* out = static_cast<uint16_t*>(out_bf16);
    const uint16_t* q = static_cast<const uint16_t*>(q_bf16);
    float* w = static_cast<float*>(ws);
    hipError_t e;
    switch (G) {
    case 1: e = launch_attention<1>(out, q, k_cache, v_cache, kv_scale, n_kv_heads, n_keys, w, s); break;
    case 2: e = launch_attention<2>(out, q, k_cache, v_cache, kv_scale, n_kv_heads, n_keys, w, s); break;
    case 4: e = launch_attention<4>(out, q, k_cache, v_cache, kv_scale, n_kv_heads, n_keys, w, s); break;
    default: e = launch_attention<8>(out, q, k_cache, v_cache, kv_scale, n_kv_heads, n_keys, w, s); break;
    }
    return status_of(e);
}

int heph_attention_qkv_fp8kv(void* out_bf16, const void* qkv_bf16, const void* q_gamma,
                             const void* k_gamma, uint8_t* k_cache, uint8_t* v_cache,
                             const float* kv_scale, const float* kv_inv_scale,
                             const void* rope_table, int n_rope_pos, int n_heads,
                             int n_kv_heads, int head_dim, int pos, double theta, float eps,
                             void* ws, size_t ws_bytes, void* stream)
{
    if (!out_bf16 || !qkv_bf16 || !q_gamma || !k_gamma || !k_cache || !v_cache || !kv_scale ||
        !kv_inv_scale || !ws)
        return HEPH_ERR_NULL;
    if (head_dim != 128 || n_kv_heads < 1 || n_heads < n_kv_heads || n_heads % n_kv_heads ||
        pos < 0 || pos >= HEPH_ATTN_MAX_KEYS)
        return HEPH_ERR_SHAPE;
    // the table's row pos is read on the device: it must exist
    if (rope_table && pos >= n_rope_pos) return HEPH_ERR_SHAPE;
    const int G = n_heads / n_kv_heads;
    if (G != 1 && G != 2 && G != 4 && G != 8) return HEPH_ERR_SHAPE;
    const int n_keys = pos + 1;
    if (ws_bytes < heph_attention_ws_bytes(n_heads, n_keys)) return HEPH_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(k_cache) % 16 || reinterpret_cast<uintptr_t>(v_cache) % 16 ||
        reinterpret_cast<uintptr_t>(ws) % 16 || reinterpret_cast<uintptr_t>(rope_table) % 4)
        return HEPH_ERR_ALIGN;
    if (int st = check_device()) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t slot = (size_t)pos * n_kv_heads * 128;
    QkvPrep prep;
    prep.qkv = static_cast<const uint16_t*>(qkv_bf16);
    prep.q_gamma = static_cast<const uint16_t*>(q_gamma);
    prep.k_gamma = static_cast<const uint16_t*>(k_gamma);
    prep.k_slot = k_cache + slot;
    prep.v_cache = v_cache;
    prep.kv_inv = kv_inv_scale;
    prep.rope = rope_table ? static_cast<const uint16_t*>(rope_table) + (size_t)pos * 128
                           : nullptr;
    prep.n_heads = n_heads;
    prep.theta = theta;
    prep.eps = eps;
    uint16_t* out = static_cast<uint16_t*>(out_bf16);
    float* w = static_cast<float*>(ws);
    hipError_t e;
    switch (G) {
    case 1: e = launch_attention<1>(out, nullptr, k_cache, v_cache, kv_scale, n_kv_heads, n_keys, w, s, prep); break;
    case 2: e = launch_attention<2>(out, nullptr, k_cache, v_cache, kv_scale, n_kv_heads, n_keys, w, s, prep); break;
    case 4: e = launch_attention<4>(out, nullptr, k_cache, v_cache, kv_scale, n_kv_heads, n_keys, w, s, prep); break;
    default: e = launch_attention<8>(out, nullptr, k_cache, v_cache, kv_scale, n_kv_heads, n_keys, w, s, prep); break;
    }
    return status_of(e);
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

size_t heph_argmax_ws_bytes(int n)
{
    if (n < 1) return 0;
    return sizeof(ArgPair) * (size_t)((n + kArgChunk - 1) / kArgChunk);
}

int heph_argmax_bf16(int32_t* out_idx, const float* logits, int n, void* ws, size_t ws_bytes,
                     void* stream)
{
    if (!out_idx || !logits || !ws) return HEPH_ERR_NULL;
    if (n < 1) return HEPH_ERR_SHAPE;
    if (ws_bytes < heph_argmax_ws_bytes(n)) return HEPH_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(ws) % 8) return HEPH_ERR_ALIGN;
    if (int st = check_device()) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int nb = (n + kArgChunk - 1) / kArgChunk;
    ArgPair* part = static_cast<ArgPair*>(ws);
    argmax_part_kernel<<<nb, 256, 0, s>>>(part, logits, n);
    argmax_final_kernel<<<1, 256, 0, s>>>(out_idx, part, nb);
    return status_of(hipGetLastError());
}

}  // extern "C"
