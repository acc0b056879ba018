/*
 * heph_decode_oracle.c - CPU restatement of the non-linear ops of one Qwen3
 * W8A8 decode step (TEST INFRASTRUCTURE ONLY; see heph_oracle.h).
 *
 * Each function follows the reference engine's arithmetic and repeats the
 * fixed reduction order of the HIP kernels in hephaestus_amd/csrc/decode.hip
 * (partial sums over a stride, then a pairwise fold), so the only expected
 * differences against the GPU are the last bit of expf / cos / sin from two
 * different math libraries. Compiled with -ffp-contract=off: every fused
 * multiply-add below is an explicit fmaf.
 *   embed          src/hephaestus/kernels.mojo:530-548
 *   rmsnorm        HF Qwen3RMSNorm as the engine calls it, forward.mojo:45-81
 *   qk_norm_rope   forward.mojo:474-500, rope kernels.mojo:709-762
 *   attention      kernels.mojo:923-1035 (fp32 scores, bf16 probabilities
 *                  from the global max and sum), the sum of exponentials and
 *                  the value sums in the lane and wave order of decode.hip's
 *                  values kernel
 *   silu_mul       kernels.mojo:1243-1255
 *   argmax         kernels.mojo:1376-1433 (bf16 logits, lowest index on ties)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "heph_oracle.h"

static inline float bf(uint16_t b) { return heph_oracle_bf16_to_f32(b); }
static inline uint16_t tob(float f) { return heph_oracle_f32_to_bf16(f); }
static inline float rb(float f) { return bf(tob(f)); }

static inline uint8_t e4m3_sat(float v)
{
    if (v > 448.0f) v = 448.0f;
    if (v < -448.0f) v = -448.0f;
    return heph_oracle_e4m3_encode(v);
}

/* v[0..n) folded as v[t] += v[t + h] for h = n/2, ..., 1 (n a power of 2). */
static float fold(float* v, int n)
{
    for (int h = n / 2; h > 0; h >>= 1)
        for (int t = 0; t < h; ++t) v[t] += v[t + h];
    return v[0];
}

void heph_oracle_embed_fp8(uint16_t* x, const uint8_t* emb, const float* scale, int block,
                           const int32_t* tokens, int n_tok, int hidden)
{
    for (int t = 0; t < n_tok; ++t) {
        const size_t id = (size_t)tokens[t];
        for (int d = 0; d < hidden; ++d) {
            const float s = block ? scale[(id >> 7) * (size_t)(hidden >> 7) + (d >> 7)] : scale[id];
            x[(size_t)t * hidden + d] = tob(s * heph_oracle_e4m3_decode(emb[id * hidden + d]));
        }
    }
}

static float rms_factor(float ss, int n, float eps)
{
    return 1.0f / sqrtf(ss / (float)n + eps);
}

void heph_oracle_rmsnorm(uint16_t* out, const uint16_t* in, const uint16_t* gamma, int rows,
                         int cols, float eps)
{
    float part[256];
    for (int r = 0; r < rows; ++r) {
        const uint16_t* x = in + (size_t)r * cols;
        uint16_t* y = out + (size_t)r * cols;
        for (int t = 0; t < 256; ++t) {
            float ss = 0.0f;
            for (int i = t; i < cols; i += 256) ss = fmaf(bf(x[i]), bf(x[i]), ss);
            part[t] = ss;
        }
        const float f = rms_factor(fold(part, 256), cols, eps);
        for (int i = 0; i < cols; ++i) y[i] = tob(bf(gamma[i]) * rb(bf(x[i]) * f));
    }
}

void heph_oracle_rope_cs(int pos, int p, int D, double theta, float* c, float* s)
{
    const float freq = (float)((double)pos * pow(theta, -2.0 * (double)p / (double)D));
    *c = rb((float)cos((double)freq));
    *s = rb((float)sin((double)freq));
}

void heph_oracle_qk_norm_rope_kv(uint16_t* qkv, const uint16_t* q_gamma, const uint16_t* k_gamma,
                                 uint8_t* k_slot, uint8_t* v_slot, const float* kv_inv,
                                 int n_heads, int n_kv, int pos, double theta, float eps)
{
    enum { D = 128, L = 64 };
    for (int h = 0; h < n_heads + 2 * n_kv; ++h) {
        uint16_t* row = qkv + (size_t)h * D;
        if (h >= n_heads + n_kv) {
            const int kh = h - n_heads - n_kv;
            const float inv = kv_inv[n_kv + kh];
            for (int i = 0; i < D; ++i) v_slot[kh * D + i] = e4m3_sat(bf(row[i]) * inv);
            continue;
        }
        const uint16_t* g = h < n_heads ? q_gamma : k_gamma;
        float part[L];
        for (int l = 0; l < L; ++l) {
            const float a = bf(row[l]), b = bf(row[l + L]);
            part[l] = fmaf(b, b, a * a);
        }
        const float f = rms_factor(fold(part, L), D, eps);
        float re[L], im[L];
        for (int l = 0; l < L; ++l) {
            const float a = rb(bf(g[l]) * rb(bf(row[l]) * f));
            const float b = rb(bf(g[l + L]) * rb(bf(row[l + L]) * f));
            float c, s;
            heph_oracle_rope_cs(pos, l, D, theta, &c, &s);
            const float re_c = rb(a * c), im_s = rb(b * s), im_c = rb(b * c), re_s = rb(a * s);
            re[l] = rb(re_c - im_s);
            im[l] = rb(im_c + re_s);
        }
        if (h < n_heads) {
            for (int l = 0; l < L; ++l) {
                row[l] = tob(re[l]);
                row[l + L] = tob(im[l]);
            }
        } else {
            const int kh = h - n_heads;
            const float inv = kv_inv[kh];
            for (int l = 0; l < L; ++l) {
                k_slot[kh * D + l] = e4m3_sat(re[l] * inv);
                k_slot[kh * D + l + L] = e4m3_sat(im[l] * inv);
            }
        }
    }
}

/* The values kernel's sum of 64 lane values x[l] (decode.hip,
 * attn_values_kernel): T_q over the lanes q + 8m, then the eight T_q. */
static float lanes64(const float* x)
{
    float T[8];
    for (int q = 0; q < 8; ++q)
        T[q] = ((x[q] + x[q + 32]) + (x[q + 16] + x[q + 48])) +
               ((x[q + 8] + x[q + 40]) + (x[q + 24] + x[q + 56]));
    return ((T[0] + T[7]) + (T[2] + T[5])) + ((T[1] + T[6]) + (T[3] + T[4]));
}

/* The values kernel's sum of its 16 waves' values: pairs, then a tree. */
static float waves16(const float* r)
{
    float r8[8];
    for (int u = 0; u < 8; ++u) r8[u] = r[2 * u] + r[2 * u + 1];
    return ((r8[0] + r8[1]) + (r8[2] + r8[3])) + ((r8[4] + r8[5]) + (r8[6] + r8[7]));
}

int heph_oracle_attention_fp8kv(uint16_t* out, const uint16_t* q, const uint8_t* kc,
                                const uint8_t* vc, const float* kv_scale, int n_heads, int n_kv,
                                int n_keys)
{
    /* Orders (decode.hip runs the same), with 16 waves w x 64 lanes l
     * holding the keys j = 64(w + 16k) + l, k = 0, 1, ... (in that order):
     *   score: per 16-dim chunk c an fma chain over its dims, then
     *          ((c0+c1)+(c2+c3)) + ((c4+c5)+(c6+c7)), times sk/sqrt(128)
     *   softmax: m = max over all keys; per lane the sum of exp(s_j - m)
     *          over its keys by plain adds, fold64 per wave, waves16;
     *          p = bf16(exp(s - m) * (1/sum))
     *   values: per dim, per lane an fma chain of p_j v_j over its keys,
     *          lanes64 per wave, waves16; times sv, bf16 */
    enum { D = 128 };
    float* sc = malloc(sizeof(float) * (size_t)n_keys);
    if (!sc) return -1;
    float dec[256];
    for (int c = 0; c < 256; ++c) dec[c] = heph_oracle_e4m3_decode((uint8_t)c);
    const size_t row = (size_t)n_kv * D;
    const int G = n_heads / n_kv;
    for (int h = 0; h < n_heads; ++h) {
        const int kh = h / G;
        float qs[D];
        for (int d = 0; d < D; ++d) qs[d] = bf(q[(size_t)h * D + d]);
        const float qk_scale = kv_scale[kh] * 0.08838834764831845f;
        for (int j = 0; j < n_keys; ++j) {
            const uint8_t* k = kc + j * row + kh * D;
            float pc[8];
            for (int c = 0; c < 8; ++c) {
                float part = 0.0f;
                for (int e = 0; e < 16; ++e) part = fmaf(qs[16 * c + e], dec[k[16 * c + e]], part);
                pc[c] = part;
            }
            const float s = ((pc[0] + pc[1]) + (pc[2] + pc[3])) + ((pc[4] + pc[5]) + (pc[6] + pc[7]));
            sc[j] = s * qk_scale;
        }
        float m = -3.4e38f;
        for (int j = 0; j < n_keys; ++j) m = fmaxf(m, sc[j]);
        for (int j = 0; j < n_keys; ++j) sc[j] = expf(sc[j] - m);
        float sw[16];
        for (int w = 0; w < 16; ++w) {
            float x[64];
            for (int l = 0; l < 64; ++l) {
                float a = 0.0f;
                for (int j = 64 * w + l; j < n_keys; j += 64 * 16) a += sc[j];
                x[l] = a;
            }
            sw[w] = fold(x, 64);
        }
        const float inv = 1.0f / waves16(sw);
        for (int j = 0; j < n_keys; ++j) sc[j] = rb(sc[j] * inv);
        for (int d = 0; d < D; ++d) {
            float wv[16];
            for (int w = 0; w < 16; ++w) {
                float x[64];
                for (int l = 0; l < 64; ++l) {
                    float a = 0.0f;
                    for (int j = 64 * w + l; j < n_keys; j += 64 * 16)
                        a = fmaf(sc[j], dec[vc[j * row + kh * D + d]], a);
                    x[l] = a;
                }
                wv[w] = lanes64(x);
            }
            out[(size_t)h * D + d] = tob(waves16(wv) * kv_scale[n_kv + kh]);
        }
    }
    free(sc);
    return 0;
}

void heph_oracle_silu_mul(uint16_t* out, const uint16_t* gate, const uint16_t* up, size_t n)
{
    for (size_t i = 0; i < n; ++i) {
        const float g = bf(gate[i]);
        const float s = rb(g / (1.0f + expf(-g)));
        out[i] = tob(s * bf(up[i]));
    }
}

int heph_oracle_argmax_bf16(const float* logits, size_t n)
{
    int best = -1;
    float bv = -3.4e38f;
    for (size_t i = 0; i < n; ++i) {
        const float v = rb(logits[i]);
        if (v > bv) {
            bv = v;
            best = (int)i;
        }
    }
    return best;
}
