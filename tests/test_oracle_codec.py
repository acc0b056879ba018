"""Pins the oracle's E4M3FN and bf16 codecs (oracle/heph_oracle.c).

Checks: the OCP closed form of special codes; the 256-code table against
torch's independent float8_e4m3fn; encoding against brute-force
nearest-even over that table (ties to even, the tie at 464 going to 448,
overflow to NaN); a strided sweep of the f32 bit space against torch.
"""
import json
import os

import numpy as np
import pytest
import torch


def test_special_codes_closed_form(oracle):
    t = oracle.e4m3_decode_table()
    assert t[0x00] == 0.0 and np.signbit(t[0x80])
    assert t[0x01] == 2.0 ** -9            # smallest subnormal
    assert t[0x07] == 7 * 2.0 ** -9        # largest subnormal
    assert t[0x08] == 2.0 ** -6            # smallest normal
    assert t[0x38] == 1.0                  # bias 7
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    finite = t[~np.isnan(t)]
    assert finite.size == 254
    assert len(set(np.abs(finite).tolist())) == 127  # +-0 share a magnitude


def test_decode_table_matches_golden(oracle, golden_dir):
    ref = json.load(open(os.path.join(golden_dir, "e4m3_table.json")))["values"]
    t = oracle.e4m3_decode_table()
    for c in range(256):
        if ref[c] is None:
            assert np.isnan(t[c]), c
        else:
            assert t[c] == ref[c], (c, t[c], ref[c])


def _nearest_even(x: np.ndarray, table: np.ndarray) -> np.ndarray:
    """Brute force: nearest finite code by value, ties to the even code,
    results beyond 448 (|x| > 464 or the tie above) become NaN."""
    codes = np.arange(256)
    fin = ~np.isnan(table)
    vals = table[fin].astype(np.float64)
    cs = codes[fin]
    out = np.empty(x.shape, np.uint8)
    for i, v in enumerate(x.astype(np.float64)):
        if np.isnan(v) or np.isinf(v) or abs(v) > 464.0:
            out[i] = 0x7F | (0x80 if np.signbit(v) else 0)
            continue
        d = np.abs(vals - v)
        best = np.flatnonzero(d == d.min())
        # same sign as x (keeps -0 for negative values that round to zero)
        best = [b for b in best if np.signbit(vals[b]) == np.signbit(v)] or list(best)
        if len(best) > 1:
            best = [b for b in best if cs[b] % 2 == 0]
        out[i] = cs[best[0]]
    return out


def test_encode_brute_force_ties_and_boundaries(oracle):
    table = oracle.e4m3_decode_table()
    pos = np.sort(table[(~np.isnan(table)) & (table >= 0)])
    pos = np.unique(pos)
    mids = (pos[:-1].astype(np.float64) + pos[1:]) / 2
    mids = mids.astype(np.float32)          # midpoints are exact in f32
    up = np.nextafter(mids, np.float32(np.inf))
    dn = np.nextafter(mids, np.float32(-np.inf))
    extra = np.array([448.0, 449.0, 463.99997, 464.0, 464.00003, 480.0, 1e30,
                      2.0 ** -10, 2.0 ** -10 * 3, 2.0 ** -11, 0.0], np.float32)
    x = np.concatenate([mids, up, dn, pos, extra])
    x = np.concatenate([x, -x]).astype(np.float32)
    got = oracle.e4m3_encode(x)
    want = _nearest_even(x, table)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(x[i], got[i], want[i]) for i in bad[:10]]
    # The 464 tie goes to the even code 448 (mantissa 110), not to NaN.
    assert oracle.e4m3_encode(np.float32([464.0]))[0] == 0x7E
    assert oracle.e4m3_encode(np.float32([464.00003]))[0] == 0x7F


def test_encode_all_bf16_values(oracle):
    b = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = oracle.bf16_to_f32(b)
    got = oracle.e4m3_encode(x)
    ref = torch.from_numpy(x.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, ref)


def test_encode_strided_f32_sweep_matches_torch(oracle):
    u = np.arange(0, 2 ** 32, 97, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    got = oracle.e4m3_encode(x)
    ref = torch.from_numpy(x.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, ref)


def test_bf16_rne_matches_torch(oracle):
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.standard_normal(1 << 16).astype(np.float32) * 100,
                        rng.integers(0, 2 ** 32, 1 << 16, dtype=np.uint64)
                        .astype(np.uint32).view(np.float32)])
    x = x[np.isfinite(x)]
    got = oracle.f32_to_bf16(x)
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    assert np.array_equal(oracle.bf16_to_f32(got), torch.from_numpy(x.copy()).to(torch.bfloat16).float().numpy())


@pytest.mark.parametrize("code", [0x38, 0x7E, 0x01, 0xB8])
def test_decode_encode_roundtrip(oracle, code):
    v = oracle.e4m3_decode_table()[code]
    assert oracle.e4m3_encode(np.float32([v]))[0] == code
