/*
 * heph_oracle.h - CPU restatement of the Hephaestus W8A8 FP8 linear path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP library
 * (hephaestus_amd/libhephfp8.so) and the CPU baseline that bench.py times.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it. The product path never calls it.
 *
 * What each function restates (paths relative to the reference tree):
 *   e4m3 codec        OCP 8-bit FP spec, E4M3FN variant (bias 7, no Inf,
 *                     NaN = S.1111.111, max 448). The reference names the
 *                     type at src/hephaestus/wmma_gfx12.mojo:631-633 and
 *                     converts with .cast[FP8]() (kernels.mojo:186, :266).
 *   quant_act         src/hephaestus/kernels.mojo:151-186 (absmax, /448,
 *                     1e-12 floor, f32 reciprocal, x*inv, cast), applied per
 *                     group of group_k elements of one row. group_k == K
 *                     is exactly the reference's per-token quantizer
 *                     (kernels.mojo:214-267).
 *   quant_weight      scripts/stage_tiny_fp8_from_bf16.py:59-71 (absmax/448,
 *                     1.0 floor, row / s), applied per bn x bk block; the
 *                     block-128 layout is the weight/weight_scale_inv format.
 *   linear            experiments/exp4b_wmma_gemm/oracle.py:113-126
 *                     (dequantize, f32 accumulate, C = A @ W^T) with the
 *                     per-block scales of the block-scaled format.
 *   bf16_linear       src/hephaestus/kernels.mojo:89-121 (lm_head, f32 out).
 *   decode-step ops   heph_decode_oracle.c: embedding, RMSNorm, q/k norm +
 *                     RoPE + KV-cache quantization, attention over an E4M3
 *                     KV cache, SwiGLU, argmax (forward.mojo:359-615).
 */
#ifndef HEPH_ORACLE_H
#define HEPH_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar codecs ---------------------------------------------------- */
float    heph_oracle_e4m3_decode(uint8_t code);
uint8_t  heph_oracle_e4m3_encode(float x);          /* RNE, NaN on overflow */
float    heph_oracle_bf16_to_f32(uint16_t b);
uint16_t heph_oracle_f32_to_bf16(float x);          /* RNE */

void heph_oracle_e4m3_encode_array(const float* x, uint8_t* q, size_t n);
void heph_oracle_e4m3_decode_array(const uint8_t* q, float* x, size_t n);
void heph_oracle_f32_to_bf16_array(const float* x, uint16_t* b, size_t n);
void heph_oracle_bf16_to_f32_array(const uint16_t* b, float* x, size_t n);

/* ---- quantizers ------------------------------------------------------- */
/* x: bf16 [M,K]; q: e4m3 [M,K]; scales: f32 [M, K/group_k] row-major.
 * Returns 0, or -1 when group_k does not divide K. */
int heph_oracle_quant_act(const uint16_t* x, int M, int K, int group_k,
                          uint8_t* q, float* scales);

/* w: f32 [N,K]; q: e4m3 [N,K]; scale_inv: f32 [ceil(N/bn), ceil(K/bk)].
 * Block (bn,bk) = (128,128) gives weight_scale_inv; (1,K) gives the
 * reference's per-output-channel [N,1] scale. */
int heph_oracle_quant_weight(const float* w, int N, int K, int bn, int bk,
                             uint8_t* q, float* scale_inv);

/* ---- dequant-matmul --------------------------------------------------- */
/* out[m,n] = sum_k (dec(qa[m,k]) * sa[m, k/group_k]) *
 *                  (dec(qw[n,k]) * sw[n/bn, k/bk])
 * f32 products, f32 accumulation (16 interleaved partial sums, then a
 * fixed pairwise fold), f32 output. nthreads <= 0 uses every core. */
int heph_oracle_linear(const uint8_t* qa, const float* sa, int group_k,
                       const uint8_t* qw, const float* sw, int bn, int bk,
                       int M, int N, int K, float* out, int nthreads);

/* Same sum accumulated in f64 (the pinning reference for tolerance tests). */
int heph_oracle_linear_f64(const uint8_t* qa, const float* sa, int group_k,
                           const uint8_t* qw, const float* sw, int bn, int bk,
                           int M, int N, int K, double* out, int nthreads);

/* Whole CPU path: quant_act(x) then linear. Uses caller scratch q/s. */
int heph_oracle_quant_linear(const uint16_t* x, int group_k,
                             const uint8_t* qw, const float* sw, int bn, int bk,
                             int M, int N, int K, uint8_t* q_scratch,
                             float* s_scratch, float* out, int nthreads);

/* bf16 x [M,K] times bf16 w [N,K]^T, f32 accumulate, f32 out. */
int heph_oracle_bf16_linear(const uint16_t* x, const uint16_t* w, int M, int N,
                            int K, float* out, int nthreads);

/* ---- deterministic synthetic inputs ----------------------------------- */
/* out[i] = mean + std * N(0,1) for element (offset + i) of stream `seed`,
 * from splitmix64 counters and Box-Muller in double precision. */
void heph_oracle_gen_normal(uint64_t seed, uint64_t offset, size_t n,
                            float mean, float std, float* out);
/* out[i] = uniform [0,1) double for element (offset + i) of stream seed. */
void heph_oracle_gen_uniform(uint64_t seed, uint64_t offset, size_t n,
                             double* out);
/* bf16 activations ~N(0,1); when outlier_p > 0 an entry whose uniform draw
 * (stream seed ^ 0x5eed) is below outlier_p is multiplied by outlier_mul
 * before rounding to bf16. */
void heph_oracle_gen_act_bf16(uint64_t seed, size_t n, double outlier_p,
                              float outlier_mul, uint16_t* out);

/* ---- one Qwen3 decode step: the non-linear ops (heph_decode_oracle.c) --- */
/* Same arithmetic and reduction order as hephaestus_amd/csrc/decode.hip;
 * head size 128. */
void heph_oracle_embed_fp8(uint16_t* x, const uint8_t* emb, const float* scale, int block,
                           const int32_t* tokens, int n_tok, int hidden);
void heph_oracle_rmsnorm(uint16_t* out, const uint16_t* in, const uint16_t* gamma, int rows,
                         int cols, float eps);
void heph_oracle_rope_cs(int pos, int p, int D, double theta, float* c, float* s);
void heph_oracle_qk_norm_rope_kv(uint16_t* qkv, const uint16_t* q_gamma,
                                 const uint16_t* k_gamma, uint8_t* k_slot, uint8_t* v_slot,
                                 const float* kv_inv, int n_heads, int n_kv, int pos,
                                 double theta, float eps);
int heph_oracle_attention_fp8kv(uint16_t* out, const uint16_t* q, const uint8_t* kc,
                                const uint8_t* vc, const float* kv_scale, int n_heads,
                                int n_kv, int n_keys);
void heph_oracle_silu_mul(uint16_t* out, const uint16_t* gate, const uint16_t* up, size_t n);
int heph_oracle_argmax_bf16(const float* logits, size_t n);

/* FNV-1a 64 digest, used for committed input/output digests. */
uint64_t heph_oracle_fnv1a64(const void* data, size_t n);

int heph_oracle_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
