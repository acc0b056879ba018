"""Pins the oracle's activation and weight quantizers.

The golden cases (tests/golden/quant_cases.npz) were evaluated with numpy
float32 arithmetic and torch's E4M3 cast, independently of the C oracle,
from the reference formula (src/hephaestus/kernels.mojo:151-186).
Further checks target plausible mistakes: dividing by the scale instead of
multiplying by its reciprocal, dropping the 1e-12 floor, taking the amax
over the row instead of the group, or letting one group's outlier leak into
its neighbours.
"""
import os

import numpy as np
import pytest
import torch


@pytest.fixture(scope="module")
def cases(golden_dir):
    z = np.load(os.path.join(golden_dir, "quant_cases.npz"))
    return {k: z[k] for k in z.files}


def _names(cases):
    return sorted({k.split("__")[0] for k in cases})


def test_golden_quant_cases(oracle, cases):
    for name in _names(cases):
        x = cases[f"{name}__x"]
        for tag, group in (("g128", 128), ("token", x.shape[1])):
            q, s = oracle.quant_act(x, group)
            assert np.array_equal(s, cases[f"{name}__{tag}__s"]), (name, tag)
            assert np.array_equal(q, cases[f"{name}__{tag}__q"]), (name, tag)


def test_scale_one_groups_are_plain_conversion(oracle, cases):
    # Every group of "all_bf16" holds the anchor 448, so scale == 1 and the
    # codes are exactly the RNE conversion of the bf16 values.
    x = cases["all_bf16__x"]
    q, s = oracle.quant_act(x, 128)
    assert np.all(s == 1.0)   # anchor groups: 448/448; zero padding: floor
    direct = oracle.e4m3_encode(oracle.bf16_to_f32(x))
    assert np.array_equal(q, direct)


def _divide_form(oracle, x, group):
    """The same quantizer with x / scale instead of x * (1/scale)."""
    M, K = x.shape
    xf = oracle.bf16_to_f32(x).reshape(M, K // group, group)
    amax = np.abs(xf).max(axis=2).astype(np.float32)
    s = (amax / np.float32(448)).astype(np.float32)
    s = np.where(s < np.float32(1e-12), np.float32(1), s).astype(np.float32)
    y = (xf / s[:, :, None]).astype(np.float32).reshape(M, K)
    return torch.from_numpy(y).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_reciprocal_multiply_not_division(oracle):
    # x*(1/s) and x/s round differently for some inputs; the reference
    # multiplies by the reciprocal (kernels.mojo:182-186).
    from oracle import oracle as O
    x = O.gen_act_bf16(11, 64, 4096)
    q, _ = oracle.quant_act(x, 128)
    qd = _divide_form(oracle, x, 128)
    n_diff = int((q != qd).sum())
    assert n_diff > 0, "seeded data must discriminate multiply from divide"
    assert n_diff < q.size * 1e-2


def test_zero_and_floor_groups(oracle):
    x = np.zeros((1, 384), np.uint16)
    tiny = oracle.f32_to_bf16(np.full(128, 1e-13, np.float32))
    x[0, 128:256] = tiny
    x[0, 256:384] = oracle.f32_to_bf16(np.linspace(-2, 2, 128).astype(np.float32))
    q, s = oracle.quant_act(x, 128)
    assert s[0, 0] == 1.0 and not q[0, :128].any()
    # amax/448 < 1e-12 -> scale 1, codes are the values themselves (here 0)
    assert s[0, 1] == 1.0
    assert np.array_equal(q[0, 128:256], oracle.e4m3_encode(oracle.bf16_to_f32(tiny)))
    assert s[0, 2] == np.float32(2.0) / np.float32(448)


def test_amax_element_maps_to_448(oracle):
    from oracle import oracle as O
    x = O.gen_act_bf16(5, 16, 2560, outlier_p=1e-2)
    q, s = oracle.quant_act(x, 128)
    xf = oracle.bf16_to_f32(x).reshape(16, 20, 128)
    qi = q.reshape(16, 20, 128)
    idx = np.abs(xf).argmax(axis=2)
    amax_codes = np.take_along_axis(qi, idx[:, :, None], axis=2)[:, :, 0]
    assert np.all((amax_codes & 0x7F) == 0x7E)


def test_groups_are_independent(oracle):
    from oracle import oracle as O
    x = O.gen_act_bf16(6, 2, 1024)
    q0, s0 = oracle.quant_act(x, 128)
    y = x.copy()
    y[1, 300] = oracle.f32_to_bf16(np.float32([500.0]))[0]   # outlier in group (1, 2)
    q1, s1 = oracle.quant_act(y, 128)
    changed = np.argwhere(s0 != s1)
    assert changed.tolist() == [[1, 2]]
    assert np.array_equal(q0[:, :256], q1[:, :256]) and np.array_equal(q0[0], q1[0])
    assert np.array_equal(q0[1, 384:], q1[1, 384:])


def test_token_group_is_reference_per_row(oracle):
    # group_k == K reproduces the reference's per-token quantizer: one scale
    # per row from the whole row's amax (kernels.mojo:214-267).
    from oracle import oracle as O
    x = O.gen_act_bf16(8, 5, 2560)
    q, s = oracle.quant_act(x, 2560)
    xf = oracle.bf16_to_f32(x)
    assert s.shape == (5, 1)
    assert np.array_equal(s[:, 0], (np.abs(xf).max(axis=1) / np.float32(448)).astype(np.float32))
    qg, sg = oracle.quant_act(x, 128)
    assert not np.array_equal(q, qg)   # granularity matters


def test_act_quant_skips_nan(oracle):
    # The reference's `if v > local: local = v` never takes a NaN
    # (kernels.mojo:153-160): the amax is numpy's nanmax of |x|; quiet and
    # signalling NaN of both signs, beside the group's largest value.
    from oracle import oracle as O
    x = O.gen_act_bf16(11, 2, 512).copy()
    x[0, 5], x[0, 9] = 0x7FC0, 0x4400             # qNaN and 512 in group 0
    x[0, 130], x[0, 131] = 0xFF81, 0xC3F0         # -sNaN and -480 in group 1
    x[1, 300] = 0x7F81                            # +sNaN alone in group 2
    q, s = oracle.quant_act(x, 128)
    xf = oracle.bf16_to_f32(x).reshape(2, 4, 128)
    want = (np.nanmax(np.abs(xf), axis=2) / np.float32(448)).astype(np.float32)
    assert np.array_equal(s, want)
    assert s[0, 0] == np.float32(512) / np.float32(448)
    assert s[0, 1] == np.float32(480) / np.float32(448)
    nan = np.isnan(oracle.bf16_to_f32(x))
    assert np.all((q[nan] & 0x7F) == 0x7F) and not np.any((q[~nan] & 0x7F) == 0x7F)


def test_weight_quant_matches_independent_numpy(oracle):
    from oracle import oracle as O
    w = O.gen_normal(3, 300 * 384, 0.0, 0.02).reshape(300, 384)
    # numpy's max propagates NaN, so a block holding one takes s = 1
    # (scripts/stage_tiny_fp8_from_bf16.py:65-68); an infinity gives s = inf
    w[5, 7] = np.nan
    w[140, 300] = np.inf
    for bn, bk in ((128, 128), (1, 384)):
        q, s = oracle.quant_weight(w, bn, bk)
        nb, kb = -(-300 // bn), -(-384 // bk)
        assert s.shape == (nb, kb)
        for i in range(nb):
            for j in range(kb):
                blk = w[i * bn:(i + 1) * bn, j * bk:(j + 1) * bk]
                amax = np.float32(np.abs(blk).max())
                sc = amax / np.float32(448) if amax > 0 else np.float32(1)
                assert s[i, j] == sc
                ref = torch.from_numpy((blk / sc).astype(np.float32)).to(torch.float8_e4m3fn)
                got = q[i * bn:(i + 1) * bn, j * bk:(j + 1) * bk]
                ref = ref.view(torch.uint8).numpy()
                nan = (ref & 0x7F) == 0x7F          # NaN codes: sign not compared
                assert np.array_equal((got & 0x7F) == 0x7F, nan)
                assert np.array_equal(got[~nan], ref[~nan])
        assert s[5 // bn, 7 // bk] == 1.0 and np.isinf(s[140 // bn, 300 // bk])
