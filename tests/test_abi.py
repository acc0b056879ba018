"""C-ABI checks that need no GPU: the library loads, exports every function
include/hephfp8.h declares, and rejects bad calls with status codes before
touching a device (the reference only debug_asserts its preconditions,
src/hephaestus/wmma_gfx12.mojo:731-732, :872-874, :996-1005)."""
import ctypes

import pytest

from hephaestus_amd import _lib as L

FAKE = 0x10000          # 16-byte aligned, never dereferenced by validation
ODD = 0x10001


@pytest.fixture(scope="module")
def lib():
    return L.lib()


def test_exports_every_declared_symbol(lib):
    names = L.header_functions()
    assert len(names) >= 9
    for n in names:
        assert hasattr(lib, n), n
    assert set(L.SIGNATURES) == set(names)


def test_version_and_strerror(lib):
    assert lib.heph_abi_version() == 6 == L.ABI_VERSION
    # the header's define, the built library and the Python binding agree
    import re
    hdr = open(L.HEADERS[0]).read()
    assert int(re.search(r"#define HEPH_ABI_VERSION (\d+)", hdr).group(1)) == L.ABI_VERSION
    for code in range(0, -12, -1):
        msg = L.strerror(code)
        assert msg and msg != "unknown status", code
    assert L.strerror(-99) == "unknown status"


def test_workspace_sizes(lib):
    assert lib.heph_fp8_q_ws_bytes(4, 2560) == 4 * 2560
    assert lib.heph_fp8_s_ws_floats(4, 2560, 128) == 4 * 20
    assert lib.heph_fp8_s_ws_floats(4, 2560, 2560) == 4
    assert lib.heph_fp8_s_ws_floats(4, 2560, 100) == 0
    assert lib.heph_fp8_q_ws_bytes(0, 2560) == 0


def lin(lib, **kw):
    a = dict(c=FAKE, c_dtype=0, x=FAKE, w=FAKE, sw=FAKE, bn=128, bk=128, q=FAKE,
             qn=1 << 30, s=FAKE, sn=1 << 30, M=1, N=256, K=2560, g=128, flags=0)
    a.update(kw)
    return lib.heph_fp8_linear(a["c"], a["c_dtype"], a["x"], a["w"], a["sw"], a["bn"],
                               a["bk"], a["q"], a["qn"], a["s"], a["sn"], a["M"], a["N"],
                               a["K"], a["g"], a["flags"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(c=None), L.HEPH_ERR_NULL),
    (dict(w=None), L.HEPH_ERR_NULL),
    (dict(sw=None), L.HEPH_ERR_NULL),
    (dict(q=None), L.HEPH_ERR_NULL),
    (dict(s=None), L.HEPH_ERR_NULL),
    (dict(x=None), L.HEPH_ERR_NULL),
    (dict(M=0), L.HEPH_ERR_SHAPE),
    (dict(N=8), L.HEPH_ERR_SHAPE),
    (dict(N=264), L.HEPH_ERR_SHAPE),
    (dict(K=2500), L.HEPH_ERR_SHAPE),
    (dict(K=64, g=64), L.HEPH_ERR_SHAPE),
    (dict(K=2624), L.HEPH_ERR_SHAPE),                  # K % 128 with 1x128 groups
    (dict(K=2624, g=2624), L.HEPH_ERR_SHAPE),          # ... or block weights
    (dict(K=2616, g=2616, bn=1, bk=2616, sn=1), L.HEPH_ERR_SHAPE),   # K % 16
    (dict(g=64), L.HEPH_ERR_GROUP),
    (dict(g=256), L.HEPH_ERR_GROUP),
    (dict(bn=64, bk=64), L.HEPH_ERR_GROUP),
    (dict(bn=1, bk=128), L.HEPH_ERR_GROUP),
    (dict(c_dtype=7), L.HEPH_ERR_DTYPE),
    (dict(qn=2559), L.HEPH_ERR_WORKSPACE),
    (dict(sn=19), L.HEPH_ERR_WORKSPACE),
    (dict(M=3, qn=3 * 2560, sn=3), L.HEPH_ERR_WORKSPACE),
    (dict(flags=0x100), L.HEPH_ERR_FLAGS),
    (dict(flags=0x4), L.HEPH_ERR_FLAGS),
    (dict(c=ODD), L.HEPH_ERR_ALIGN),
    (dict(w=ODD), L.HEPH_ERR_ALIGN),
    (dict(x=ODD), L.HEPH_ERR_ALIGN),
    (dict(q=ODD), L.HEPH_ERR_ALIGN),
])
def test_linear_rejects(lib, kw, status):
    assert lin(lib, **kw) == status


def test_skip_quant_allows_null_x(lib):
    # do_quantize=False needs no activation pointer; with every argument
    # valid, a machine without a gfx950 device reports HEPH_ERR_DEVICE.
    st = lin(lib, x=None, flags=L.FLAG_SKIP_QUANT)
    assert st in (L.HEPH_ERR_DEVICE, L.HEPH_OK)


def test_valid_call_without_gpu_reports_device(lib):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert lin(lib) == L.HEPH_ERR_DEVICE
    assert lin(lib, bn=1, bk=2560, g=2560, sn=1) == L.HEPH_ERR_DEVICE
    # K % 128 != 0 at the reference's own granularity (per-token, per-channel)
    assert lin(lib, K=2624, bn=1, bk=2624, g=2624, sn=1) == L.HEPH_ERR_DEVICE
    assert lin(lib, K=16, bn=1, bk=16, g=16, sn=40, M=40) == L.HEPH_ERR_DEVICE
    q = lib.heph_fp8_quant_act
    assert q(FAKE, FAKE, FAKE, 3, 2624, 2624, None) == L.HEPH_ERR_DEVICE
    assert q(FAKE, FAKE, FAKE, 3, 2624, 128, None) == L.HEPH_ERR_SHAPE


def test_quant_rejects(lib):
    q = lib.heph_fp8_quant_act
    assert q(None, FAKE, FAKE, 1, 2560, 128, None) == L.HEPH_ERR_NULL
    assert q(FAKE, FAKE, FAKE, 0, 2560, 128, None) == L.HEPH_ERR_SHAPE
    assert q(FAKE, FAKE, FAKE, 1, 2600, 128, None) == L.HEPH_ERR_SHAPE
    assert q(FAKE, FAKE, FAKE, 1, 2560, 512, None) == L.HEPH_ERR_GROUP
    assert q(ODD, FAKE, FAKE, 1, 2560, 128, None) == L.HEPH_ERR_ALIGN


def test_bf16_rejects(lib):
    b = lib.heph_bf16_linear
    assert b(None, 1, FAKE, FAKE, 1, 151936, 2560, 0, None) == L.HEPH_ERR_NULL
    assert b(FAKE, 1, FAKE, FAKE, 0, 151936, 2560, 0, None) == L.HEPH_ERR_SHAPE
    assert b(FAKE, 1, FAKE, FAKE, 33, 151936, 2600, 0, None) == L.HEPH_ERR_SHAPE
    # M > 32 is the MFMA GEMM: valid arguments reach the device check
    assert b(FAKE, 1, FAKE, FAKE, 4096, 151936, 2560, 0, None) == L.HEPH_ERR_DEVICE
    assert b(FAKE, 1, FAKE, FAKE, 1, 151930, 2560, 0, None) == L.HEPH_ERR_SHAPE
    assert b(FAKE, 3, FAKE, FAKE, 1, 151936, 2560, 0, None) == L.HEPH_ERR_DTYPE
    assert b(FAKE, 1, FAKE, FAKE, 1, 151936, 2560, L.FLAG_SKIP_QUANT, None) == L.HEPH_ERR_FLAGS
    assert b(FAKE, 1, FAKE, ODD, 1, 151936, 2560, 0, None) == L.HEPH_ERR_ALIGN


def with_overrides(lib, **ov):
    o = L.LaunchOverrides(**ov)
    return lib.heph_fp8_linear_with(FAKE, 0, FAKE, FAKE, FAKE, 128, 128, FAKE, 1 << 30, FAKE,
                                    1 << 30, 1, 256, 2560, 128, 0, None, ctypes.byref(o))


def test_launch_overrides_validate(lib):
    # heph_fp8_linear_with checks every override before anything else; a
    # valid set leaves the call to the device check (no GPU here).
    ok = [dict(gemv_ks=8), dict(gemv_waves=4), dict(gemv_waves=5), dict(gemv_waves=10),
          dict(gemv_waves=16), dict(gemv_u=2),
          dict(gemm_bm=192), dict(gemm_bm=64), dict(gemm_bm=1), dict(batch_split=-1),
          dict(batch_split=64), dict(wide_tiles=-1), dict(wide_tiles=4),
          dict(wide_tiles=2, wide_waves=16), dict(split_spin_limit=-1),
          dict(split_spin_limit=1000), dict(gemv_groups=1), dict(gemv_groups=2),
          dict(gemm_bn=192), dict(gemm_bn=320), dict(gemm_bm=128, gemm_bn=320), dict()]
    bad = [dict(gemv_ks=16), dict(gemv_ks=3), dict(gemv_waves=2), dict(gemv_waves=6),
           dict(gemv_u=4),
           dict(gemm_bm=96), dict(batch_split=-2), dict(batch_split=65), dict(wide_tiles=3),
           dict(wide_tiles=8), dict(wide_tiles=-2), dict(wide_waves=2), dict(wide_waves=12),
           dict(split_spin_limit=-2), dict(gemv_groups=3), dict(gemv_groups=-1),
           dict(gemm_bn=128), dict(gemm_bn=64)]
    for ov in ok:
        assert with_overrides(lib, **ov) != L.HEPH_ERR_FLAGS, ov
    for ov in bad:
        assert with_overrides(lib, **ov) == L.HEPH_ERR_FLAGS, ov
    # a NULL overrides pointer is the plain call
    assert lib.heph_fp8_linear_with(FAKE, 0, FAKE, FAKE, FAKE, 128, 128, FAKE, 1 << 30, FAKE,
                                    1 << 30, 1, 256, 2560, 128, 0, None, None) == lin(lib)


def test_library_keeps_no_tuning_state(lib):
    # the process-wide setter of earlier versions is gone
    assert not hasattr(lib, "heph_set_tuning")


def test_rmsnorm_linear_rejects(lib):
    f = lib.heph_fp8_linear_rmsnorm
    args = lambda K, flags=0, gamma=FAKE: (FAKE, 0, FAKE, gamma, 1e-6, FAKE, FAKE, 128, 128,
                                           FAKE, 1 << 30, FAKE, 1 << 30, 256, K, flags, None)
    # rows longer than the fused norm's LDS row (8192) are refused before any
    # device work, with their own status
    assert f(*args(8320)) == L.HEPH_ERR_UNSUPPORTED
    assert f(*args(2560, flags=L.FLAG_SKIP_QUANT)) == L.HEPH_ERR_FLAGS
    assert f(*args(2560, gamma=None)) == L.HEPH_ERR_NULL
    # gamma is read in 16-byte pieces
    assert f(*args(2560, gamma=FAKE + 2)) == L.HEPH_ERR_ALIGN
    assert f(*args(8192)) in (L.HEPH_ERR_DEVICE, L.HEPH_OK)


def test_profile_hook_and_last_kernel(lib):
    assert lib.heph_profile_next_launch(None, None) == 0
    assert isinstance(lib.heph_last_kernel(), bytes)


def test_python_mirror_rejects_host_tensors():
    import torch
    from hephaestus_amd import kernels as K
    c = torch.zeros(1, 256, dtype=torch.bfloat16)
    a = torch.zeros(1, 2560, dtype=torch.bfloat16)
    w = torch.zeros(256, 2560, dtype=torch.uint8)
    s = torch.ones(2, 20)
    qws = torch.zeros(2560, dtype=torch.uint8)
    sws = torch.zeros(20)
    with pytest.raises(ValueError, match="device memory"):
        K.linear_fp8(c, a, w, s, qws, sws, 1, 256, 2560)
    with pytest.raises(ValueError, match="neither"):
        K.linear_fp8(c, a, w, torch.ones(3, 20), qws, sws, 1, 256, 2560)


def test_decode_ops_reject(lib):
    assert lib.heph_embed_fp8(None, FAKE, FAKE, 1, FAKE, 1, 100, 256, None) == L.HEPH_ERR_NULL
    assert lib.heph_embed_fp8(FAKE, FAKE, FAKE, 1, FAKE, 1, 100, 200, None) == L.HEPH_ERR_SHAPE
    assert lib.heph_rmsnorm(FAKE, FAKE, None, 1, 2560, 1e-6, None) == L.HEPH_ERR_NULL
    assert lib.heph_rmsnorm(FAKE, FAKE, FAKE, 0, 2560, 1e-6, None) == L.HEPH_ERR_SHAPE
    q = lib.heph_qk_norm_rope_kv
    assert q(FAKE, FAKE, FAKE, FAKE, None, FAKE, 32, 8, 128, 0, 1e6, 1e-6, None) == L.HEPH_ERR_NULL
    assert q(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 32, 8, 64, 0, 1e6, 1e-6, None) == L.HEPH_ERR_SHAPE
    assert q(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 30, 8, 128, 0, 1e6, 1e-6, None) == L.HEPH_ERR_SHAPE
    a = lib.heph_attention_fp8kv
    ws = lib.heph_attention_ws_bytes(32, 4097)
    # the fp32 scores
    assert ws == 4 * 32 * 4097
    # query heads per kv head: 1, 2, 4 or 8
    assert a(FAKE, FAKE, FAKE, FAKE, FAKE, 24, 8, 128, 10, FAKE, ws, None) == L.HEPH_ERR_SHAPE
    assert a(FAKE, FAKE, FAKE, FAKE, FAKE, 32, 2, 128, 10, FAKE, ws, None) == L.HEPH_ERR_SHAPE
    assert a(FAKE, FAKE, FAKE, FAKE, FAKE, 32, 8, 128, L.ATTN_MAX_KEYS + 1, FAKE, 1 << 40,
             None) == L.HEPH_ERR_SHAPE
    assert a(FAKE, FAKE, FAKE, FAKE, FAKE, 32, 8, 128, 0, FAKE, ws, None) == L.HEPH_ERR_SHAPE
    assert a(FAKE, FAKE, FAKE, FAKE, FAKE, 32, 8, 128, 4097, None, ws, None) == L.HEPH_ERR_NULL
    assert a(FAKE, FAKE, FAKE, FAKE, FAKE, 32, 8, 128, 4097, FAKE, ws - 4, None) == \
        L.HEPH_ERR_WORKSPACE
    assert a(FAKE, FAKE, ODD, FAKE, FAKE, 32, 8, 128, 10, FAKE, ws, None) == L.HEPH_ERR_ALIGN
    # q/k norm + RoPE + K/V write + attention: the union of both ops' checks,
    # over pos + 1 keys
    qa = lib.heph_attention_qkv_fp8kv
    args = [FAKE] * 9
    NR = 1 << 20          # rows of the RoPE table
    assert qa(*args, NR, 32, 8, 128, 4096, 1e6, 1e-6, FAKE, ws, None) in \
        (L.HEPH_ERR_DEVICE, L.HEPH_OK)
    assert qa(*args[:7], None, FAKE, NR, 32, 8, 128, 4096, 1e6, 1e-6, FAKE, ws, None) == \
        L.HEPH_ERR_NULL
    # no table: the call computes the cos/sin of pos itself
    assert qa(*args[:8], None, 0, 32, 8, 128, 4096, 1e6, 1e-6, FAKE, ws, None) in \
        (L.HEPH_ERR_DEVICE, L.HEPH_OK)
    assert qa(*args[:8], FAKE + 2, NR, 32, 8, 128, 4096, 1e6, 1e-6, FAKE, ws, None) == \
        L.HEPH_ERR_ALIGN
    assert qa(*args, NR, 32, 8, 128, 4096, 1e6, 1e-6, None, ws, None) == L.HEPH_ERR_NULL
    assert qa(*args, NR, 32, 8, 64, 4096, 1e6, 1e-6, FAKE, ws, None) == L.HEPH_ERR_SHAPE
    assert qa(*args, NR, 24, 8, 128, 4096, 1e6, 1e-6, FAKE, ws, None) == L.HEPH_ERR_SHAPE
    assert qa(*args, NR, 32, 2, 128, 4096, 1e6, 1e-6, FAKE, ws, None) == L.HEPH_ERR_SHAPE
    assert qa(*args, NR, 32, 8, 128, -1, 1e6, 1e-6, FAKE, ws, None) == L.HEPH_ERR_SHAPE
    assert qa(*args, NR, 32, 8, 128, L.ATTN_MAX_KEYS, 1e6, 1e-6, FAKE, 1 << 40, None) == \
        L.HEPH_ERR_SHAPE
    assert qa(*args, NR, 32, 8, 128, 4096, 1e6, 1e-6, FAKE, ws - 4, None) == L.HEPH_ERR_WORKSPACE
    assert qa(*args[:4], ODD, *args[5:], NR, 32, 8, 128, 4096, 1e6, 1e-6, FAKE, ws, None) == \
        L.HEPH_ERR_ALIGN
    rt = lib.heph_rope_table_bf16
    assert rt(None, 4097, 128, 1e6, None) == L.HEPH_ERR_NULL
    assert rt(FAKE, 0, 128, 1e6, None) == L.HEPH_ERR_SHAPE
    assert rt(FAKE, 4097, 64, 1e6, None) == L.HEPH_ERR_SHAPE
    assert rt(FAKE, L.ATTN_MAX_KEYS + 1, 128, 1e6, None) == L.HEPH_ERR_SHAPE
    assert rt(FAKE + 2, 4097, 128, 1e6, None) == L.HEPH_ERR_ALIGN
    assert rt(FAKE, 4097, 128, 1e6, None) in (L.HEPH_ERR_DEVICE, L.HEPH_OK)
    assert lib.heph_silu_mul(FAKE, FAKE, FAKE, 0, None) == L.HEPH_ERR_SHAPE
    aw = lib.heph_argmax_ws_bytes(151936)
    assert aw == 8 * 75                              # one (value, index) per 2048 logits
    assert lib.heph_argmax_bf16(None, FAKE, 10, FAKE, aw, None) == L.HEPH_ERR_NULL
    assert lib.heph_argmax_bf16(FAKE, FAKE, 10, None, aw, None) == L.HEPH_ERR_NULL
    assert lib.heph_argmax_bf16(FAKE, FAKE, 0, FAKE, aw, None) == L.HEPH_ERR_SHAPE
    assert lib.heph_argmax_bf16(FAKE, FAKE, 151936, FAKE, aw - 8, None) == L.HEPH_ERR_WORKSPACE
    # a table without row pos is refused before anything reads it
    assert qa(*args, 4096, 32, 8, 128, 4096, 1e6, 1e-6, FAKE, ws, None) == L.HEPH_ERR_SHAPE
    assert qa(*args, 4097, 32, 8, 128, 4096, 1e6, 1e-6, FAKE, ws, None) in \
        (L.HEPH_ERR_DEVICE, L.HEPH_OK)


def test_noalloc_limits(lib):
    # the allocation-free entry point has a fixed 64 MiB scratch: codes plus
    # scales past it are refused before any device work, with their own status
    assert lib.heph_noalloc_scratch_bytes() == 64 << 20
    na = lib.heph_fp8_linear_noalloc
    assert na(FAKE, 0, FAKE, FAKE, FAKE, 128, 128, 8192, 256, 9728, 128, 0, None) == \
        L.HEPH_ERR_SCRATCH
    assert na(FAKE, 0, FAKE, FAKE, FAKE, 128, 128, 1, 256, 2500, 128, 0, None) == L.HEPH_ERR_SHAPE
    # M = 4096 at K = 9728 fits (40 MB of codes, 1.2 MB of scales)
    assert na(FAKE, 0, FAKE, FAKE, FAKE, 128, 128, 4096, 256, 9728, 128, 0, None) in \
        (L.HEPH_ERR_DEVICE, L.HEPH_OK)


def test_producer_quant_rejects(lib):
    rq, sq = lib.heph_rmsnorm_quant_fp8, lib.heph_silu_mul_quant_fp8
    assert rq(None, FAKE, FAKE, FAKE, 1, 2560, 1e-6, 128, None) == L.HEPH_ERR_NULL
    assert rq(FAKE, FAKE, FAKE, FAKE, 1, 2500, 1e-6, 128, None) == L.HEPH_ERR_SHAPE
    assert rq(FAKE, FAKE, FAKE, FAKE, 1, 2560, 1e-6, 256, None) == L.HEPH_ERR_GROUP
    assert rq(FAKE, FAKE, FAKE, FAKE, 1, 16512, 1e-6, 128, None) == L.HEPH_ERR_UNSUPPORTED
    assert rq(ODD, FAKE, FAKE, FAKE, 1, 2560, 1e-6, 128, None) == L.HEPH_ERR_ALIGN
    assert sq(FAKE, FAKE, FAKE, None, 1, 9728, 19456, 128, None) == L.HEPH_ERR_NULL
    assert sq(FAKE, FAKE, FAKE, FAKE, 1, 9728, 9000, 128, None) == L.HEPH_ERR_SHAPE
    assert sq(FAKE, FAKE, FAKE, FAKE, 1, 9728, 19460, 128, None) == L.HEPH_ERR_SHAPE
    assert sq(FAKE, FAKE, FAKE, FAKE, 1, 9728, 19456, 64, None) == L.HEPH_ERR_GROUP
    assert sq(FAKE, FAKE, FAKE, FAKE, 1, 32768, 32768, 32768, None) == L.HEPH_ERR_UNSUPPORTED
    assert sq(FAKE, FAKE, ODD, FAKE, 1, 9728, 19456, 128, None) == L.HEPH_ERR_ALIGN


def test_swiglu_linear_rejects(lib):
    # heph_fp8_linear_swiglu: M = 1, N % 16, K % 128, the fused norm's 8192
    # limit, weight granularity and workspace sizes, before any device work
    sg = lib.heph_fp8_linear_swiglu
    ok = dict(N=19456, K=2560)

    def call(act=FAKE, x=FAKE, gamma=FAKE, N=19456, K=2560, bn=128, bk=128, qb=1 << 20,
             sf=1 << 20):
        return sg(act, x, gamma, 1e-6, FAKE, FAKE, bn, bk, FAKE, qb, FAKE, sf, N, K, None)

    assert call(**ok) in (L.HEPH_ERR_DEVICE, L.HEPH_OK)
    assert call(gamma=None) in (L.HEPH_ERR_DEVICE, L.HEPH_OK)
    assert call(act=None) == L.HEPH_ERR_NULL
    assert call(x=None) == L.HEPH_ERR_NULL
    assert call(N=19448) == L.HEPH_ERR_SHAPE
    assert call(K=2500) == L.HEPH_ERR_SHAPE
    assert call(K=9728) == L.HEPH_ERR_UNSUPPORTED          # fused norm: K <= 8192
    assert call(K=9728, gamma=None) in (L.HEPH_ERR_DEVICE, L.HEPH_OK)
    assert call(bn=64, bk=128) == L.HEPH_ERR_GROUP
    assert call(bn=1, bk=2560) in (L.HEPH_ERR_DEVICE, L.HEPH_OK)
    assert call(qb=100) == L.HEPH_ERR_WORKSPACE
    assert call(sf=10) == L.HEPH_ERR_WORKSPACE
    assert call(act=ODD) == L.HEPH_ERR_ALIGN


def test_v_cache_block_layout():
    # decode.v_blocks / v_rows against the V cache byte formula of
    # hephdecode.h: key j, kv head h, dim d at
    # ((j/64 * n_kv + h) * 8 + d/16) * 1024 + (j%64) * 16 + d%16
    import numpy as np
    import torch
    from hephaestus_amd import decode as DEC
    rng = np.random.default_rng(7)
    for n, n_kv in ((1, 2), (64, 8), (65, 8), (300, 4)):
        rows = rng.integers(0, 256, size=(n, n_kv, 128), dtype=np.uint8)
        blk = DEC.v_blocks(rows)
        assert blk.shape == (-(-n // 64), n_kv, 8, 64, 16)
        flat = blk.reshape(-1)
        j, h, d = (rng.integers(0, n, 500), rng.integers(0, n_kv, 500), rng.integers(0, 128, 500))
        off = ((j // 64 * n_kv + h) * 8 + d // 16) * 1024 + (j % 64) * 16 + d % 16
        assert np.array_equal(flat[off], rows[j, h, d])
        assert np.array_equal(DEC.v_rows(blk, n), rows)
        assert not DEC.v_rows(blk)[n:].any()                  # zero padding keys
        tb = DEC.v_blocks(torch.from_numpy(rows))
        assert np.array_equal(tb.numpy(), blk)
        assert np.array_equal(DEC.v_rows(tb, n).numpy(), rows)
