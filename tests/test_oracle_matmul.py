"""Pins the oracle's dequant-matmul, bf16 matmul and input generator.

Checks: numpy float64 matmul of independently dequantized operands
(catches a transposed operand or a swapped scale index); exact-integer
inputs with power-of-two scales, compared with Python integer arithmetic;
the reference's all-ones KATs (16 per 16-wide K step,
experiments/exp3g_fp8_wmma_gfx12.mojo:27-36; 1280 at N=K=2560 with scale
0.5, bench/1b-fp8-decode.md:83); determinism digests of the synthetic inputs.
"""
import json
import os

import numpy as np
import pytest


def smoke_codes(oracle, n, seed):
    """The reference smoke test's exact-in-E4M3 pattern
    ((i*17 + seed*31) % 17 - 8) * 0.25 (src/qwen_small_m_gemm_smoke.mojo:26-31)."""
    i = np.arange(n, dtype=np.int64)
    v = (((i * 17 + seed * 31) % 17) - 8).astype(np.float32) * 0.25
    return oracle.e4m3_encode(v)


def dequant(oracle, q, s, rows_per, cols_per):
    """dec(q) * scale rounded to f32 (the dequantized operand), as f64."""
    t = oracle.e4m3_decode_table()
    R, C = q.shape
    sx = np.repeat(np.repeat(s, rows_per, axis=0), cols_per, axis=1)[:R, :C]
    return (t[q] * sx).astype(np.float32).astype(np.float64)


@pytest.mark.parametrize("M,N,K", [(1, 256, 384), (5, 144, 640), (33, 272, 256)])
def test_linear_vs_numpy_f64(oracle, M, N, K):
    from oracle import oracle as O
    rng = np.random.default_rng(M * N + K)
    x = O.gen_act_bf16(M + 17, M, K)
    qa, sa = oracle.quant_act(x, 128)
    qw, sw = O.gen_weight(N + K, N, K)
    # distinct power-of-two factors per block expose a swapped scale index
    sw = (sw * (2.0 ** rng.integers(-3, 4, sw.shape))).astype(np.float32)
    A = dequant(oracle, qa, sa, 1, 128)
    W = dequant(oracle, qw, sw, 128, 128)
    ref = A @ W.T
    got32 = oracle.linear(qa, sa, qw, sw)
    got64 = oracle.linear_f64(qa, sa, qw, sw)
    scale = np.abs(ref).max()
    assert np.abs(got64 - ref).max() <= 1e-12 * scale * K
    assert np.abs(got32 - ref).max() <= 1e-5 * scale
    # a transposed-scale variant must not pass
    if sw.shape[0] != sw.shape[1]:
        Wt = dequant(oracle, qw, np.ascontiguousarray(sw[::-1]), 128, 128)
        assert np.abs(A @ Wt.T - ref).max() > 1e-3 * scale


def test_linear_per_channel_vs_numpy(oracle):
    from oracle import oracle as O
    M, N, K = 3, 160, 512
    x = O.gen_act_bf16(2, M, K)
    qa, sa = oracle.quant_act(x, K)
    w = O.gen_normal(9, N * K, 0, 0.02).reshape(N, K)
    qw, sw = oracle.quant_weight(w, 1, K)
    A = dequant(oracle, qa, sa, 1, K)
    W = dequant(oracle, qw, sw, 1, K)
    got = oracle.linear_f64(qa, sa, qw, sw, bn=1, bk=K)
    assert np.allclose(got, A @ W.T, rtol=0, atol=1e-12 * np.abs(A @ W.T).max() * K)


@pytest.mark.parametrize("M,N,K", [(1, 64, 2560), (7, 48, 9728), (32, 128, 1024)])
def test_exact_integer_case(oracle, M, N, K):
    qa = smoke_codes(oracle, M * K, 1).reshape(M, K)
    qw = smoke_codes(oracle, N * K, 2).reshape(N, K)
    sa = np.full((M, K // 128), 2.0 ** -3, np.float32)
    sw = np.full((-(-N // 128), K // 128), 2.0 ** -2, np.float32)
    ia = (((np.arange(M * K) * 17 + 31) % 17) - 8).reshape(M, K).astype(np.int64)
    iw = (((np.arange(N * K) * 17 + 62) % 17) - 8).reshape(N, K).astype(np.int64)
    exact = (ia @ iw.T).astype(np.float64) * (0.25 * 0.25) * 2.0 ** -5
    got = oracle.linear(qa, sa, qw, sw)
    assert np.array_equal(got.astype(np.float64), exact)


def test_all_ones_kat(oracle):
    # 16 per 16-wide K step in the reference KAT; 128 per 128-wide chunk here.
    K = 128
    qa = np.full((1, K), 0x38, np.uint8)
    qw = np.full((16, K), 0x38, np.uint8)
    got = oracle.linear(qa, np.ones((1, 1), np.float32), qw, np.ones((1, 1), np.float32))
    assert np.all(got == 128.0)
    qa16 = np.full((1, 16), 0x38, np.uint8)
    got16 = oracle.linear(qa16, np.ones((1, 1), np.float32), np.full((16, 16), 0x38, np.uint8),
                          np.ones((16, 1), np.float32), bn=1, bk=16)
    assert np.all(got16 == 16.0)


def test_kat_1280(oracle):
    # scale * sum(fp8(1) * bf16(1)) over K = 2560 with scale 0.5 -> 1280.
    N = K = 2560
    x = oracle.f32_to_bf16(np.ones((1, K), np.float32))
    qw = np.full((N, K), 0x38, np.uint8)
    sw = np.full((N // 128, K // 128), 0.5, np.float32)
    out = oracle.quant_linear(x, qw, sw)
    assert np.all(oracle.f32_to_bf16(out) == oracle.f32_to_bf16(np.float32([1280.0]))[0])


def test_bf16_linear_vs_numpy(oracle):
    from oracle import oracle as O
    x = O.gen_act_bf16(1, 3, 640)
    w = oracle.f32_to_bf16(O.gen_normal(2, 1000 * 640, 0, 0.05)).reshape(1000, 640)
    ref = oracle.bf16_to_f32(x).astype(np.float64) @ oracle.bf16_to_f32(w).astype(np.float64).T
    got = oracle.bf16_linear(x, w)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


def test_generator_statistics(oracle):
    from oracle import oracle as O
    z = O.gen_normal(0, 1 << 20)
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1) < 5e-3
    assert np.array_equal(z[1000:2000], O.gen_normal(0, 1000, offset=1000))
    x = O.gen_act_bf16(3, 512, 2560, outlier_p=1e-3)
    big = np.abs(oracle.bf16_to_f32(x)) > 8
    assert 0.5e-3 < big.mean() < 1.5e-3


def test_synthetic_input_digests(oracle, golden_dir):
    from oracle import oracle as O
    d = json.load(open(os.path.join(golden_dir, "digests.json")))
    qw, sw = O.gen_weight(seed=1000 + 4096 + 2560, N=4096, K=2560)
    assert O.digest(qw) == d["q_proj_w"] and O.digest(sw) == d["q_proj_scale_inv"]
    assert O.digest(O.gen_act_bf16(0, 1, 2560)) == d["x_config0"]
