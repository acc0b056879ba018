"""heph_fp8_linear_noalloc (the allocation-free entry point) against
heph_fp8_linear on the GPU, through the C ABI: the same kernels on the same
inputs must give the same bits (the workspace only moves into the library's
fixed device array), and the oracle's tolerance holds."""
import ctypes

import numpy as np
import pytest
import torch

from hephaestus_amd import _lib as L
from hephaestus_amd import kernels as HK
from oracle import oracle as O
from tests._gpu import dev, f32_of_bf16, host_bf16, max_abs_rel

pytestmark = pytest.mark.gpu


def noalloc(c, x, w, sw, M, N, K, flags=0):
    st = L.lib().heph_fp8_linear_noalloc(
        c.data_ptr(), L.HEPH_DTYPE_BF16 if c.dtype == torch.bfloat16 else L.HEPH_DTYPE_F32,
        x.data_ptr() if x is not None else None, w.data_ptr(), sw.data_ptr(), 128, 128,
        M, N, K, 128, flags, torch.cuda.current_stream().cuda_stream)
    assert st == L.HEPH_OK, L.strerror(st)
    return HK.last_kernel()


def test_noalloc_matches_linear_two_calls_second_smaller():
    # call 1: M = 512 o_proj (the large-M GEMM with its K split, partials in
    # the fixed scratch); call 2: M = 1 qkv (the fused GEMV), smaller; call
    # 3: SKIP_QUANT on call 2's codes with other weights
    runs = []
    for M, N, K, seed in ((512, 2560, 4096, 1), (1, 6144, 2560, 2)):
        x = O.gen_act_bf16(seed, M, K, outlier_p=1e-3)
        qw, sw = O.gen_weight(seed + 10, N, K)
        xd, wd, sd = dev(x), dev(qw), dev(sw)
        ref = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
        q_ws, s_ws = HK.workspace(M, K, n=N)
        HK.linear_fp8(ref, xd, wd, sd, q_ws, s_ws, M, N, K)
        want_kernel = HK.last_kernel()
        got = torch.zeros_like(ref)
        got_kernel = noalloc(got, xd, wd, sd, M, N, K)
        torch.cuda.synchronize()
        print(f"noalloc M={M} N={N} K={K}: {got_kernel} (linear: {want_kernel})", flush=True)
        assert got_kernel == want_kernel
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (M, N, K)
        r = max_abs_rel(f32_of_bf16(host_bf16(got)), O.quant_linear(x, qw, sw))
        assert r <= 1e-2, (M, r)
        runs.append((x, M, K))
    x, M, K = runs[-1]
    N = 2560
    qw, sw = O.gen_weight(99, N, K)
    wd, sd = dev(qw), dev(sw)
    got = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
    noalloc(got, None, wd, sd, M, N, K, flags=L.FLAG_SKIP_QUANT)
    ref = torch.zeros_like(got)
    q_ws, s_ws = HK.workspace(M, K)
    HK.linear_fp8(ref, dev(x), wd, sd, q_ws, s_ws, M, N, K)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
