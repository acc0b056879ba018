"""Writes the committed golden fixtures under tests/golden/.

The fixtures come from implementations independent of oracle/heph_oracle.c:
  e4m3_table.json   value of each of the 256 E4M3FN codes, decoded by
                    torch.float8_e4m3fn (NaN written as null);
  quant_cases.npz   bf16 activation rows and their expected codes and
                    scales under the reference quantizer formula
                    (src/hephaestus/kernels.mojo:151-186, per 1x128 group and
                    per token), evaluated with numpy float32 arithmetic and
                    torch's float8_e4m3fn cast;
  digests.json      FNV-1a digests of the synthetic benchmark inputs, so a
                    GPU box that regenerates them can prove identical bytes.

The reference itself is Mojo and needs a gfx1201 GPU, so no vector here was
produced by running it; it holds no FP8 golden vectors of its own.

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))


def e4m3_torch(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    return t.to(torch.float8_e4m3fn).view(torch.uint8).numpy().copy()


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16).copy()


def quant_reference(xb: np.ndarray, group: int):
    """kernels.mojo:151-186 per group, in numpy f32 + torch's E4M3 cast."""
    M, K = xb.shape
    x = bf16_bits_to_f32(xb).reshape(M, K // group, group)
    with np.errstate(invalid="ignore"):
        amax = np.nanmax(np.abs(x), axis=2).astype(np.float32)
    amax = np.where(np.isnan(amax), np.float32(0), amax).astype(np.float32)
    scale = (amax / np.float32(448.0)).astype(np.float32)
    scale = np.where(scale < np.float32(1e-12), np.float32(1.0), scale).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    prod = (x * inv[:, :, None]).astype(np.float32)
    q = e4m3_torch(prod.reshape(M, K))
    return q, scale.reshape(M, K // group)


def make_quant_cases():
    rng = np.random.default_rng(20261201)
    cases = {}
    # 1. N(0,1) rows, 0.1% outliers x50 (config 3 style), K = 2560.
    x = rng.standard_normal((8, 2560)).astype(np.float32)
    x[rng.random(x.shape) < 1e-3] *= 50.0
    cases["normal"] = f32_to_bf16_bits(x)
    # 2. Every finite bf16 bit pattern with |v| <= 448, grouped 127 per group
    #    with a 448 anchor so the scale is exactly 1 and the codes are the
    #    plain RNE conversion of the values.
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    v = bf16_bits_to_f32(allb)
    keep = np.isfinite(v) & (np.abs(v) <= 448.0)
    vals = allb[keep]
    n_groups = -(-vals.size // 127)
    pad = n_groups * 127 - vals.size
    vals = np.concatenate([vals, np.zeros(pad, np.uint16)]).reshape(n_groups, 127)
    anchor = f32_to_bf16_bits(np.full((n_groups, 1), 448.0, np.float32))
    grid = np.concatenate([anchor, vals], axis=1).reshape(-1)
    rows = -(-grid.size // 2560)
    grid = np.concatenate([grid, np.zeros(rows * 2560 - grid.size, np.uint16)])
    cases["all_bf16"] = grid.reshape(rows, 2560)
    # 3. Edge groups: zeros, tiny (scale floor), a single spike, negative
    #    amax, a constant group, huge values near bf16 max.
    e = np.zeros((4, 1024), np.float32)
    e[0, 128:256] = 1e-14 * rng.standard_normal(128)       # floor: scale = 1
    e[0, 256 + 5] = -3.0                                     # single spike
    e[0, 384:512] = -rng.random(128) * 7.0                   # all negative
    e[1, :128] = 0.7                                         # constant group
    e[1, 128:256] = 3e38 * rng.random(128)                   # near f32/bf16 max
    e[2] = rng.standard_normal(1024) * 1e-3
    e[3] = rng.standard_normal(1024) * 1e3
    cases["edges"] = f32_to_bf16_bits(e)
    # 4. Wide rows at the configs' K values.
    for K in (4096, 9728):
        cases[f"k{K}"] = f32_to_bf16_bits(rng.standard_normal((3, K)).astype(np.float32))

    out = {}
    for name, xb in cases.items():
        out[f"{name}__x"] = xb
        for group, tag in ((128, "g128"), (xb.shape[1], "token")):
            q, s = quant_reference(xb, group)
            out[f"{name}__{tag}__q"] = q
            out[f"{name}__{tag}__s"] = s
    return out


def make_digests():
    sys.path.insert(0, ROOT)
    from oracle import oracle as O
    d = {}
    for name, (N, K) in {"q_proj": (4096, 2560), "qkv": (6144, 2560),
                         "o_proj": (2560, 4096)}.items():
        qw, sw = O.gen_weight(seed=1000 + N + K, N=N, K=K)
        d[f"{name}_w"] = O.digest(qw)
        d[f"{name}_scale_inv"] = O.digest(sw)
    d["x_config0"] = O.digest(O.gen_act_bf16(0, 1, 2560))
    d["x_config3_m512_k2560"] = O.digest(O.gen_act_bf16(3, 512, 2560, outlier_p=1e-3))
    return d


def main():
    codes = np.arange(256, dtype=np.uint8)
    vals = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    table = [None if np.isnan(v) else float(v) for v in vals]
    with open(os.path.join(HERE, "e4m3_table.json"), "w") as f:
        json.dump({"source": "torch.float8_e4m3fn decode of codes 0..255",
                   "values": table}, f, indent=0)
    np.savez_compressed(os.path.join(HERE, "quant_cases.npz"), **make_quant_cases())
    with open(os.path.join(HERE, "digests.json"), "w") as f:
        json.dump(make_digests(), f, indent=1, sort_keys=True)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
