/*
 * hephdecode.h - the non-linear ops of one Qwen3 W8A8 decode step
 * (random-init end-to-end check of the FP8 linear path). Same conventions as
 * hephfp8.h: device pointers, a hipStream_t as void* (NULL = default
 * stream), HEPH_* status codes, no allocation, no synchronization.
 *
 * bf16 tensors are passed as their 16-bit patterns. Head size is 128.
 */
#ifndef HEPHDECODE_H
#define HEPHDECODE_H

#include <stddef.h>
#include <stdint.h>

#include "hephfp8.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Longest context the attention op takes. */
#define HEPH_ATTN_MAX_KEYS 262144

/*
 * x[t, :] = bf16(scale * e4m3(emb[tokens[t], :])) for t < n_tok.
 * block != 0: emb_scale is [ceil(vocab/128), hidden/128] (128x128 blocks);
 * block == 0: one scale per row, [vocab]. A token id outside [0, vocab)
 * gives a zero row.
 * Replaces embed_lookup_fp8 (src/hephaestus/kernels.mojo:530-570).
 */
int heph_embed_fp8(void* x_bf16, const uint8_t* emb, const float* emb_scale, int block,
                   const int32_t* tokens, int n_tok, int vocab, int hidden, void* stream);

/*
 * out = bf16(gamma * bf16(in * 1/sqrt(mean(in^2) + eps))) per row of cols;
 * out may alias in. Replaces _rms_norm (src/hephaestus/forward.mojo:45-81).
 */
int heph_rmsnorm(void* out_bf16, const void* in_bf16, const void* gamma_bf16, int rows,
                 int cols, float eps, void* stream);

/*
 * The KV cache layouts (E4M3 codes, head_dim 128):
 *   K: rows [n_keys][n_kv_heads][128]; key j's row at j * n_kv_heads * 128.
 *   V: 64-key blocks [ceil(n_keys/64)][n_kv_heads][8][64][16]: key j, kv
 *      head h, dim d at ((j/64 * n_kv_heads + h) * 8 + d/16) * 1024 +
 *      (j%64) * 16 + d%16. Whole blocks are allocated: a V cache of
 *      n_keys keys holds ceil(n_keys/64) * 64 * n_kv_heads * 128 bytes (the
 *      padding keys of the last block are never used as values).
 * The reference's cache is [MAX_KEYS, kv_out] rows (kernels.mojo:917); V's
 * blocks let one 64-lane load read 64 keys of one 16-dim chunk.
 */

/*
 * On the qkv output of one token ([n_heads + 2*n_kv_heads, 128] bf16):
 * per-head RMSNorm of q (q_gamma) and k (k_gamma), RoPE of both at `pos`
 * (theta), q written back in place; k and v quantized to E4M3 with
 * code = e4m3(clamp(x * kv_inv_scale[h], +-448)) into key `pos` of
 * k_cache / v_cache (the layouts above). kv_inv_scale: n_kv_heads K
 * entries, then n_kv_heads V entries. Replaces the q/k _rms_norm calls and
 * apply_rope_qk_inplace of forward.mojo:474-500 (kernels.mojo:709-796) and
 * the cache write of k/v (forward.mojo:415-431).
 */
int heph_qk_norm_rope_kv(void* qkv_bf16, const void* q_gamma, const void* k_gamma,
                         uint8_t* k_cache, uint8_t* v_cache, const float* kv_inv_scale,
                         int n_heads, int n_kv_heads, int head_dim, int pos, double theta,
                         float eps, void* stream);

/*
 * One query token over n_keys cached keys: out[h] = sum_j p_j * v_j with
 * p = bf16(softmax(q.k_j * sk / sqrt(128))), K and V E4M3 codes in the
 * layouts above scaled by kv_scale (K entries, then V), in two launches.
 * n_heads / n_kv_heads (query heads per kv head) must be 1, 2, 4 or 8.
 * ws: device scratch of heph_attention_ws_bytes(n_heads, n_keys) bytes
 * (the fp32 scores), 16-byte aligned.
 * Replaces attention (src/hephaestus/kernels.mojo:923-1035, :1183-1240).
 */
size_t heph_attention_ws_bytes(int n_heads, int n_keys);
int heph_attention_fp8kv(void* out_bf16, const void* q_bf16, const uint8_t* k_cache,
                         const uint8_t* v_cache, const float* kv_scale, int n_heads,
                         int n_kv_heads, int head_dim, int n_keys, void* ws, size_t ws_bytes,
                         void* stream);

/*
 * RoPE table: table_bf16[pos][p] = (cos, sin) of pair p < head_dim/2 at
 * position pos < n_pos as bf16 patterns (2 * n_pos * head_dim/2 values,
 * 4-byte aligned): exactly the values heph_qk_norm_rope_kv computes,
 * freq = f32(pos * theta^(-2p/head_dim)) in double, cos/sin of it rounded
 * to f32, then bf16. head_dim 128. The cos/sin of kernels.mojo:709-762,
 * computed once per position instead of per call.
 */
int heph_rope_table_bf16(void* table_bf16, int n_pos, int head_dim, double theta, void* stream);

/*
 * heph_qk_norm_rope_kv on qkv_bf16 into key `pos` of k_cache / v_cache,
 * then heph_attention_fp8kv over pos + 1 keys with the rotated q: the same
 * out, the same cache bytes, in the attention's two launches (the scores
 * kernel prepares q and the new key's k and v itself). q in qkv_bf16 is left as it was (not
 * rotated in place). ws: heph_attention_ws_bytes(n_heads, pos + 1) bytes.
 * rope_table: a heph_rope_table_bf16 table of n_rope_pos rows (for this
 * theta and head_dim), or NULL to compute pos's cos/sin in the call
 * (n_rope_pos is then ignored); HEPH_ERR_SHAPE when pos >= n_rope_pos.
 * Replaces the q/k norms, RoPE, K/V write and attention call of
 * src/hephaestus/forward.mojo:474-520 (kernels.mojo:709-796, :923-1035).
 */
int heph_attention_qkv_fp8kv(void* out_bf16, const void* qkv_bf16, const void* q_gamma,
                             const void* k_gamma, uint8_t* k_cache, uint8_t* v_cache,
                             const float* kv_scale, const float* kv_inv_scale,
                             const void* rope_table, int n_rope_pos, int n_heads,
                             int n_kv_heads, int head_dim, int pos, double theta, float eps,
                             void* ws, size_t ws_bytes, void* stream);

/*
 * out = bf16(bf16(g / (1 + exp(-g))) * up). Replaces silu_mul
 * (src/hephaestus/kernels.mojo:1243-1278).
 */
int heph_silu_mul(void* out_bf16, const void* gate_bf16, const void* up_bf16, int n,
                  void* stream);

/*
 * out_idx[0] = argmax_i bf16(logits[i]), lowest index on ties (-1 when no
 * logit compares above -3.4e38, e.g. all NaN). ws: device scratch of
 * heph_argmax_ws_bytes(n) bytes, 8-byte aligned (one (value, index) pair per
 * 2048 logits). Replaces argmax_logits (src/hephaestus/kernels.mojo:1376-1463).
 */
size_t heph_argmax_ws_bytes(int n);
int heph_argmax_bf16(int32_t* out_idx, const float* logits, int n, void* ws, size_t ws_bytes,
                     void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HEPHDECODE_H */
