"""Producer-side quantization (heph_rmsnorm_quant_fp8, heph_silu_mul_quant_fp8)
on the GPU: codes and scales bit for bit those of the producer followed by
heph_fp8_quant_act, the RMSNorm form also bit for bit the oracle's
rmsnorm + quantizer (at M = 512 and the full configs[3] M = 4096), and the
linear run with SKIP_QUANT on them equal to the unfused path."""
import numpy as np
import pytest
import torch

from hephaestus_amd import _lib as L
from hephaestus_amd import decode as DEC
from hephaestus_amd import kernels as HK
from oracle import oracle as O
from tests._gpu import bf16_of, dev, host_bf16

pytestmark = pytest.mark.gpu


def rows_bf16(seed, rows, cols, scale=1.0, outliers=0.0):
    x = O.gen_act_bf16(seed, rows, cols, outlier_p=outliers)
    if scale != 1.0:
        x = bf16_of(O.bf16_to_f32(x) * np.float32(scale))
    return x


@pytest.mark.parametrize("rows,cols,scale", [(1, 2560, 1.0), (3, 4096, 40.0), (7, 9728, 1e-3),
                                             (2, 128, 1.0), (2, 16384, 1.0), (512, 2560, 1.0)])
@pytest.mark.parametrize("group", ["g128", "token"])
def test_rmsnorm_quant_bit_exact(rows, cols, scale, group):
    g = 128 if group == "g128" else cols
    x = rows_bf16(cols + rows, rows, cols, scale, outliers=1e-3)
    gam = bf16_of(1.0 + 0.1 * O.gen_normal(5, cols))
    xd, gd = dev(x), dev(gam)
    q1 = torch.zeros(rows * cols, dtype=torch.uint8, device="cuda")
    s1 = torch.zeros(rows * (cols // g), dtype=torch.float32, device="cuda")
    HK.rmsnorm_quant_fp8(q1, s1, xd, gd, rows, cols, 1e-6, group_k=g)
    y = torch.empty(rows, cols, dtype=torch.bfloat16, device="cuda")
    DEC.rmsnorm(y, xd.view(rows, cols), gd)
    q2, s2 = torch.zeros_like(q1), torch.zeros_like(s1)
    HK.quantize_act_rows_fp8(q2, s2, y, rows, cols, group_k=g)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(s1, s2)
    yo = O.rmsnorm(x, gam)
    qo, so = O.quant_act(yo.reshape(rows, cols), g)
    assert np.array_equal(q1.cpu().numpy().reshape(rows, cols), qo)
    assert np.array_equal(s1.cpu().numpy().reshape(so.shape), so)


def test_rmsnorm_quant_config3_m4096_codes_vs_oracle():
    rows, cols = 4096, 2560
    x = rows_bf16(33, rows, cols, outliers=1e-3)
    gam = bf16_of(1.0 + 0.1 * O.gen_normal(6, cols))
    q = torch.zeros(rows * cols, dtype=torch.uint8, device="cuda")
    s = torch.zeros(rows * (cols // 128), dtype=torch.float32, device="cuda")
    HK.rmsnorm_quant_fp8(q, s, dev(x), dev(gam), rows, cols, 1e-6)
    torch.cuda.synchronize()
    qo, so = O.quant_act(O.rmsnorm(x, gam).reshape(rows, cols), 128)
    assert np.array_equal(q.cpu().numpy().reshape(rows, cols), qo)
    assert np.array_equal(s.cpu().numpy().reshape(so.shape), so)


@pytest.mark.parametrize("rows,n,ld", [(1, 9728, 19456), (5, 2560, 2560), (512, 9728, 19456),
                                       (4096, 9728, 19456), (3, 128, 136)])
@pytest.mark.parametrize("group", ["g128", "token"])
def test_silu_mul_quant_bit_exact(rows, n, ld, group):
    g = 128 if group == "g128" else n
    gu = rows_bf16(n + rows, rows, ld, 3.0).reshape(rows, ld)
    gud = dev(np.ascontiguousarray(gu))
    gate, up = gud.view(-1), gud.view(-1)[n:] if ld >= 2 * n else gud.view(-1)
    if ld < 2 * n:      # a separate up tensor with the same stride
        upt = dev(np.ascontiguousarray(rows_bf16(n + rows + 1, rows, ld)))
        up = upt.view(-1)
    q1 = torch.zeros(rows * n, dtype=torch.uint8, device="cuda")
    s1 = torch.zeros(rows * (n // g), dtype=torch.float32, device="cuda")
    HK.silu_mul_quant_fp8(q1, s1, gate, up, rows, n, ld, group_k=g)
    # reference composition on the GPU: silu_mul row by row, then the quantizer
    act = torch.empty(rows, n, dtype=torch.bfloat16, device="cuda")
    for r in range(rows):
        DEC.silu_mul(act[r], gate[r * ld:r * ld + n], up[r * ld:r * ld + n], n)
    q2, s2 = torch.zeros_like(q1), torch.zeros_like(s1)
    HK.quantize_act_rows_fp8(q2, s2, act, rows, n, group_k=g)
    torch.cuda.synchronize()
    assert torch.equal(s1, s2)
    assert torch.equal(q1, q2)


def test_prefill_path_with_producers_equals_unfused():
    # RMSNorm -> qkv and SwiGLU -> down at M = 512: the producer's codes fed
    # to the linear with SKIP_QUANT give the unfused path's bits.
    M, H, I = 512, 2560, 9728
    x = dev(rows_bf16(40, M, H))
    gam = dev(bf16_of(1.0 + 0.1 * O.gen_normal(7, H)))
    for N, K, kind in ((6144, H, "norm"), (2560, I, "swiglu")):
        qw, sw = O.gen_weight(41 + N, N, K)
        wd, sd = dev(qw), dev(sw)
        q_ws, s_ws = HK.workspace(M, K, n=N)
        c1 = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
        c2 = torch.zeros_like(c1)
        if kind == "norm":
            HK.rmsnorm_quant_fp8(q_ws, s_ws, x, gam, M, K)
            HK.linear_fp8(c1, None, wd, sd, q_ws, s_ws, M, N, K, do_quantize=False)
            y = torch.empty(M, K, dtype=torch.bfloat16, device="cuda")
            DEC.rmsnorm(y, x, gam)
        else:
            gu = dev(rows_bf16(42, M, 2 * I, 3.0))
            HK.silu_mul_quant_fp8(q_ws, s_ws, gu.view(-1), gu.view(-1)[I:], M, I, 2 * I)
            HK.linear_fp8(c1, None, wd, sd, q_ws, s_ws, M, N, K, do_quantize=False)
            y = torch.empty(M, K, dtype=torch.bfloat16, device="cuda")
            for r in range(M):
                DEC.silu_mul(y[r], gu[r, :I], gu[r, I:], I)
        q2, s2 = HK.workspace(M, K, n=N)
        HK.linear_fp8(c2, y, wd, sd, q2, s2, M, N, K)
        torch.cuda.synchronize()
        assert torch.equal(c1.view(torch.int16), c2.view(torch.int16)), kind
