/*
 * heph_oracle.c - CPU restatement of the Hephaestus W8A8 FP8 linear path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP library and the CPU
 * baseline bench.py times. Nothing in the product path links it.
 * Each function cites the reference file:line it restates (paths relative
 * to the reference tree); the header lists the same map.
 */
#include "heph_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------
 * Bit casts
 * --------------------------------------------------------------------- */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------
 * OCP E4M3FN codec (reference type: wmma_gfx12.mojo:631-633).
 *   code = S EEEE MMM, bias 7.
 *   E == 0          : subnormal, value = M * 2^-9
 *   E == 15, M == 7 : NaN (no infinities)
 *   otherwise       : (1 + M/8) * 2^(E-7); max finite 0x7E = 448.
 * --------------------------------------------------------------------- */
float heph_oracle_e4m3_decode(uint8_t code)
{
    const int s = code >> 7;
    const int e = (code >> 3) & 0xF;
    const int m = code & 0x7;
    float v;
    if (e == 15 && m == 7)
        return s ? -NAN : NAN;
    if (e == 0)
        v = ldexpf((float)m, -9);
    else
        v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return s ? -v : v;
}

/* f32 -> E4M3FN, round to nearest even. A finite input whose rounded
 * magnitude exceeds 448 (|x| > 464, or the tie 464 going even) and +-Inf
 * become NaN, the OCP non-saturating conversion. */
uint8_t heph_oracle_e4m3_encode(float x)
{
    const uint32_t u = f2u(x);
    const uint8_t sign = (uint8_t)((u >> 24) & 0x80);
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u)                      /* Inf or NaN */
        return sign | 0x7F;
    const float ax = u2f(a);
    if (ax < 0.015625f) {                      /* below 2^-6: subnormal grid */
        /* ax * 2^9 is exact; rint rounds half to even in the default mode.
         * A result of 8 is the smallest normal, code 0x08. */
        const float t = rintf(ax * 512.0f);
        return sign | (uint8_t)t;
    }
    /* Normal: keep 3 mantissa bits with RNE, carrying into the exponent. */
    const uint32_t lsb = (a >> 20) & 1u;
    const uint32_t r = (a + 0x7FFFFu + lsb) >> 20;        /* exp8:mant3 */
    const int e = (int)(r >> 3) - 127 + 7;
    const uint32_t code = ((uint32_t)e << 3) | (r & 7u);
    if (code > 0x7Eu)
        return sign | 0x7F;
    return sign | (uint8_t)code;
}

float heph_oracle_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

uint16_t heph_oracle_f32_to_bf16(float x)
{
    uint32_t u = f2u(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u)       /* NaN: keep quiet NaN */
        return (uint16_t)((u >> 16) | 0x40);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void heph_oracle_e4m3_encode_array(const float* x, uint8_t* q, size_t n)
{
#pragma omp parallel for schedule(static) if (n > (1u << 20))
    for (size_t i = 0; i < n; ++i) q[i] = heph_oracle_e4m3_encode(x[i]);
}

void heph_oracle_e4m3_decode_array(const uint8_t* q, float* x, size_t n)
{
    float lut[256];
    for (int c = 0; c < 256; ++c) lut[c] = heph_oracle_e4m3_decode((uint8_t)c);
    for (size_t i = 0; i < n; ++i) x[i] = lut[q[i]];
}

void heph_oracle_f32_to_bf16_array(const float* x, uint16_t* b, size_t n)
{
#pragma omp parallel for schedule(static) if (n > (1u << 20))
    for (size_t i = 0; i < n; ++i) b[i] = heph_oracle_f32_to_bf16(x[i]);
}

void heph_oracle_bf16_to_f32_array(const uint16_t* b, float* x, size_t n)
{
    for (size_t i = 0; i < n; ++i) x[i] = heph_oracle_bf16_to_f32(b[i]);
}

/* ------------------------------------------------------------------------
 * Dynamic activation quantizer.
 * Restates kernels.mojo:151-186 for one group of g consecutive elements:
 *   v = f32(x); if v < 0: v = -v; if v > amax: amax = v      (:151-159)
 *   scale = amax / 448; if scale < 1e-12: scale = 1          (:173-177)
 *   inv = 1 / scale; q = e4m3(f32(x) * inv)                  (:182-186)
 * The order of the max fold does not matter: max is exact and the
 * comparison ignores NaN the same way in any order.
 * --------------------------------------------------------------------- */
static void quant_group(const uint16_t* x, int g, uint8_t* q, float* scale_out)
{
    float amax = 0.0f;
    for (int i = 0; i < g; ++i) {
        float v = heph_oracle_bf16_to_f32(x[i]);
        if (v < 0.0f) v = -v;
        if (v > amax) amax = v;
    }
    float scale = amax / 448.0f;
    if (scale < 1e-12f) scale = 1.0f;
    const float inv = 1.0f / scale;
    for (int i = 0; i < g; ++i)
        q[i] = heph_oracle_e4m3_encode(heph_oracle_bf16_to_f32(x[i]) * inv);
    *scale_out = scale;
}

int heph_oracle_quant_act(const uint16_t* x, int M, int K, int group_k,
                          uint8_t* q, float* scales)
{
    if (M < 0 || K <= 0 || group_k <= 0 || K % group_k) return -1;
    const int G = K / group_k;
#pragma omp parallel for schedule(static) if ((long)M * K > (1L << 18))
    for (int m = 0; m < M; ++m)
        for (int g = 0; g < G; ++g)
            quant_group(x + (size_t)m * K + (size_t)g * group_k, group_k,
                        q + (size_t)m * K + (size_t)g * group_k,
                        scales + (size_t)m * G + g);
    return 0;
}

/* ------------------------------------------------------------------------
 * Weight quantizer. Restates scripts/stage_tiny_fp8_from_bf16.py:59-71
 *   amax = max|row|; s = amax/448 if amax > 0 else 1; if s < 1e-12: s = 1
 *   q = e4m3(row / s)        (numpy: f32 array / scalar -> f32 division)
 * over bn x bk blocks instead of whole rows.
 * --------------------------------------------------------------------- */
int heph_oracle_quant_weight(const float* w, int N, int K, int bn, int bk,
                             uint8_t* q, float* scale_inv)
{
    if (N <= 0 || K <= 0 || bn <= 0 || bk <= 0) return -1;
    const int NB = (N + bn - 1) / bn, KB = (K + bk - 1) / bk;
#pragma omp parallel for schedule(dynamic) collapse(2)
    for (int ib = 0; ib < NB; ++ib)
        for (int jb = 0; jb < KB; ++jb) {
            const int n0 = ib * bn, n1 = n0 + bn < N ? n0 + bn : N;
            const int k0 = jb * bk, k1 = k0 + bk < K ? k0 + bk : K;
            float amax = 0.0f;
            for (int n = n0; n < n1; ++n)
                for (int k = k0; k < k1; ++k) {
                    /* np.max propagates NaN; a NaN amax then fails
                     * `amax > 0` below and takes s = 1 */
                    const float v = fabsf(w[(size_t)n * K + k]);
                    if (v > amax || v != v) amax = v;
                }
            float s = amax > 0.0f ? amax / 448.0f : 1.0f;
            if (s < 1e-12f) s = 1.0f;
            scale_inv[(size_t)ib * KB + jb] = s;
            for (int n = n0; n < n1; ++n)
                for (int k = k0; k < k1; ++k)
                    q[(size_t)n * K + k] =
                        heph_oracle_e4m3_encode(w[(size_t)n * K + k] / s);
        }
    return 0;
}

/* ------------------------------------------------------------------------
 * Dequant-matmul. Restates experiments/exp4b_wmma_gemm/oracle.py:113-126
 * (A and W to f32, C = A @ W^T with f32 accumulation) on the dequantized
 * operands dec(q) * scale of the block-scaled format.
 * --------------------------------------------------------------------- */
static int check_linear_args(int group_k, int bn, int bk, int M, int N, int K)
{
    if (M <= 0 || N <= 0 || K <= 0) return -1;
    if (group_k <= 0 || K % group_k) return -1;
    if (bn <= 0 || bk <= 0) return -1;
    return 0;
}

static void dequant_act(const uint8_t* qa, const float* sa, int group_k, int M,
                        int K, float* A, const float* lut)
{
    const int G = K / group_k;
    for (int m = 0; m < M; ++m)
        for (int k = 0; k < K; ++k)
            A[(size_t)m * K + k] =
                lut[qa[(size_t)m * K + k]] * sa[(size_t)m * G + k / group_k];
}

static inline void dequant_wrow(const uint8_t* qw, const float* sw, int bn,
                                int bk, int K, int n, float* row,
                                const float* lut)
{
    const int KB = (K + bk - 1) / bk;
    const float* srow = sw + (size_t)(n / bn) * KB;
    const uint8_t* q = qw + (size_t)n * K;
    for (int k = 0; k < K; ++k) row[k] = lut[q[k]] * srow[k / bk];
}

/* 16 interleaved partial sums, folded pairwise in a fixed order. */
static inline float dot_f32(const float* a, const float* b, int K)
{
    float acc[16] = {0};
    int k = 0;
    for (; k + 16 <= K; k += 16)
        for (int j = 0; j < 16; ++j) acc[j] += a[k + j] * b[k + j];
    for (; k < K; ++k) acc[k & 15] += a[k] * b[k];
    for (int w = 8; w >= 1; w >>= 1)
        for (int j = 0; j < w; ++j) acc[j] += acc[j + w];
    return acc[0];
}

static void set_threads(int nthreads)
{
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
    else omp_set_num_threads(omp_get_num_procs());
#else
    (void)nthreads;
#endif
}

int heph_oracle_linear(const uint8_t* qa, const float* sa, int group_k,
                       const uint8_t* qw, const float* sw, int bn, int bk,
                       int M, int N, int K, float* out, int nthreads)
{
    if (check_linear_args(group_k, bn, bk, M, N, K)) return -1;
    float lut[256];
    for (int c = 0; c < 256; ++c) lut[c] = heph_oracle_e4m3_decode((uint8_t)c);
    float* A = (float*)malloc(sizeof(float) * (size_t)M * K);
    if (!A) return -2;
    dequant_act(qa, sa, group_k, M, K, A, lut);
    set_threads(nthreads);
    int fail = 0;
#pragma omp parallel
    {
        float* row = (float*)malloc(sizeof(float) * (size_t)K);
        if (!row) {
#pragma omp atomic write
            fail = 1;
        } else {
#pragma omp for schedule(static)
            for (int n = 0; n < N; ++n) {
                dequant_wrow(qw, sw, bn, bk, K, n, row, lut);
                for (int m = 0; m < M; ++m)
                    out[(size_t)m * N + n] = dot_f32(A + (size_t)m * K, row, K);
            }
            free(row);
        }
    }
    free(A);
    return fail ? -2 : 0;
}

int heph_oracle_linear_f64(const uint8_t* qa, const float* sa, int group_k,
                           const uint8_t* qw, const float* sw, int bn, int bk,
                           int M, int N, int K, double* out, int nthreads)
{
    if (check_linear_args(group_k, bn, bk, M, N, K)) return -1;
    float lut[256];
    for (int c = 0; c < 256; ++c) lut[c] = heph_oracle_e4m3_decode((uint8_t)c);
    float* A = (float*)malloc(sizeof(float) * (size_t)M * K);
    if (!A) return -2;
    dequant_act(qa, sa, group_k, M, K, A, lut);
    set_threads(nthreads);
    int fail = 0;
#pragma omp parallel
    {
        float* row = (float*)malloc(sizeof(float) * (size_t)K);
        if (!row) {
#pragma omp atomic write
            fail = 1;
        } else {
#pragma omp for schedule(static)
            for (int n = 0; n < N; ++n) {
                dequant_wrow(qw, sw, bn, bk, K, n, row, lut);
                for (int m = 0; m < M; ++m) {
                    const float* a = A + (size_t)m * K;
                    double s = 0.0;
                    for (int k = 0; k < K; ++k) s += (double)a[k] * (double)row[k];
                    out[(size_t)m * N + n] = s;
                }
            }
            free(row);
        }
    }
    free(A);
    return fail ? -2 : 0;
}

int heph_oracle_quant_linear(const uint16_t* x, int group_k,
                             const uint8_t* qw, const float* sw, int bn, int bk,
                             int M, int N, int K, uint8_t* q_scratch,
                             float* s_scratch, float* out, int nthreads)
{
    set_threads(nthreads);
    if (heph_oracle_quant_act(x, M, K, group_k, q_scratch, s_scratch)) return -1;
    return heph_oracle_linear(q_scratch, s_scratch, group_k, qw, sw, bn, bk,
                              M, N, K, out, nthreads);
}

int heph_oracle_bf16_linear(const uint16_t* x, const uint16_t* w, int M, int N,
                            int K, float* out, int nthreads)
{
    if (M <= 0 || N <= 0 || K <= 0) return -1;
    float* A = (float*)malloc(sizeof(float) * (size_t)M * K);
    if (!A) return -2;
    heph_oracle_bf16_to_f32_array(x, A, (size_t)M * K);
    set_threads(nthreads);
    int fail = 0;
#pragma omp parallel
    {
        float* row = (float*)malloc(sizeof(float) * (size_t)K);
        if (!row) {
#pragma omp atomic write
            fail = 1;
        } else {
#pragma omp for schedule(static)
            for (int n = 0; n < N; ++n) {
                heph_oracle_bf16_to_f32_array(w + (size_t)n * K, row, (size_t)K);
                for (int m = 0; m < M; ++m)
                    out[(size_t)m * N + n] = dot_f32(A + (size_t)m * K, row, K);
            }
            free(row);
        }
    }
    free(A);
    return fail ? -2 : 0;
}

/* ------------------------------------------------------------------------
 * Synthetic inputs: counter-based splitmix64, Box-Muller in double.
 * --------------------------------------------------------------------- */
static inline uint64_t splitmix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline double uniform01(uint64_t seed, uint64_t i)
{
    const uint64_t z = splitmix64(splitmix64(seed) ^ (i * 0xD1B54A32D192ED03ull));
    return (double)(z >> 11) * (1.0 / 9007199254740992.0);  /* [0,1) */
}

void heph_oracle_gen_uniform(uint64_t seed, uint64_t offset, size_t n, double* out)
{
#pragma omp parallel for schedule(static) if (n > (1u << 20))
    for (size_t i = 0; i < n; ++i) out[i] = uniform01(seed, offset + i);
}

void heph_oracle_gen_normal(uint64_t seed, uint64_t offset, size_t n,
                            float mean, float std, float* out)
{
    const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static) if (n > (1u << 20))
    for (size_t i = 0; i < n; ++i) {
        const uint64_t idx = offset + i;
        const uint64_t pair = idx >> 1;
        double u1 = uniform01(seed, 2 * pair);
        const double u2 = uniform01(seed, 2 * pair + 1);
        if (u1 < 1e-300) u1 = 1e-300;
        const double r = sqrt(-2.0 * log(u1));
        const double z = (idx & 1) ? r * sin(two_pi * u2) : r * cos(two_pi * u2);
        out[i] = (float)((double)mean + (double)std * z);
    }
}

void heph_oracle_gen_act_bf16(uint64_t seed, size_t n, double outlier_p,
                              float outlier_mul, uint16_t* out)
{
    const size_t chunk = 1u << 16;
#pragma omp parallel
    {
        float* tmp = (float*)malloc(sizeof(float) * chunk);
#pragma omp for schedule(static)
        for (size_t c0 = 0; c0 < n; c0 += chunk) {
            const size_t len = n - c0 < chunk ? n - c0 : chunk;
            heph_oracle_gen_normal(seed, c0, len, 0.0f, 1.0f, tmp);
            for (size_t i = 0; i < len; ++i) {
                float v = tmp[i];
                if (outlier_p > 0.0 && uniform01(seed ^ 0x5eedull, c0 + i) < outlier_p)
                    v *= outlier_mul;
                out[c0 + i] = heph_oracle_f32_to_bf16(v);
            }
        }
        free(tmp);
    }
}

uint64_t heph_oracle_fnv1a64(const void* data, size_t n)
{
    const uint8_t* p = (const uint8_t*)data;
    uint64_t h = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < n; ++i) { h ^= p[i]; h *= 0x100000001b3ull; }
    return h;
}

int heph_oracle_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
