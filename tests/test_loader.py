"""Checkpoint loader: manifest validation and q|k|v, gate|up fusion (CPU).

Tiny Qwen3-shaped checkpoints are written with the safetensors library in
both scale formats (128x128 `weight_scale_inv` blocks and the reference's
per-channel `weight_scale`), single-file and sharded, and loaded on the CPU.
Error cases follow the reference's own checks (loader.mojo:489-513,
:521-563; stage_weights.py:25-28, :84-93).
"""
import json
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from hephaestus_amd.loader import CheckpointError, Qwen3Config, load_qwen3_fp8

CFG = Qwen3Config(vocab=384, hidden=256, n_layers=2, n_heads=2, n_kv_heads=1, head_dim=128,
                  inter=384)


def _codes(rng, n, k):
    return torch.from_numpy(rng.integers(0, 0x7E, size=(n, k), dtype=np.uint8)).view(
        torch.float8_e4m3fn)


def make_checkpoint(cfg=CFG, block=True, seed=0):
    rng = np.random.default_rng(seed)
    t = {}

    def lin(name, n, k):
        t[name] = _codes(rng, n, k)
        if block:
            t[name + "_scale_inv"] = torch.from_numpy(
                rng.random((-(-n // 128), -(-k // 128)), dtype=np.float32))
        else:
            t[name + "_scale"] = torch.from_numpy(rng.random((n, 1), dtype=np.float32))

    def norm(name, n):
        t[name] = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(torch.bfloat16)

    lin("model.embed_tokens.weight", cfg.vocab, cfg.hidden)
    norm("model.norm.weight", cfg.hidden)
    for i in range(cfg.n_layers):
        p = f"model.layers.{i}."
        norm(p + "input_layernorm.weight", cfg.hidden)
        norm(p + "post_attention_layernorm.weight", cfg.hidden)
        norm(p + "self_attn.q_norm.weight", cfg.head_dim)
        norm(p + "self_attn.k_norm.weight", cfg.head_dim)
        lin(p + "self_attn.q_proj.weight", cfg.q_out, cfg.hidden)
        lin(p + "self_attn.k_proj.weight", cfg.kv_out, cfg.hidden)
        lin(p + "self_attn.v_proj.weight", cfg.kv_out, cfg.hidden)
        lin(p + "self_attn.o_proj.weight", cfg.hidden, cfg.q_out)
        lin(p + "mlp.gate_proj.weight", cfg.inter, cfg.hidden)
        lin(p + "mlp.up_proj.weight", cfg.inter, cfg.hidden)
        lin(p + "mlp.down_proj.weight", cfg.hidden, cfg.inter)
    return t


def save(t, d, shards=1):
    os.makedirs(d, exist_ok=True)
    if shards == 1:
        save_file(t, os.path.join(d, "model.safetensors"), metadata={"format": "pt"})
        return d
    names = sorted(t)
    weight_map = {}
    for s in range(shards):
        part = {n: t[n] for n in names[s::shards]}
        fn = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        save_file(part, os.path.join(d, fn), metadata={"format": "pt"})
        weight_map.update({n: fn for n in part})
    with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": weight_map}, f)
    return d


def u8(x):
    return x.view(torch.uint8) if x.dtype == torch.float8_e4m3fn else x


def check_loaded(m, t, block):
    sfx = "_scale_inv" if block else "_scale"
    assert m.embed.block == block
    assert torch.equal(m.embed.w, u8(t["model.embed_tokens.weight"]))
    assert torch.equal(m.embed.scale, t["model.embed_tokens.weight" + sfx])
    assert torch.equal(m.final_norm, t["model.norm.weight"])
    for i, L in enumerate(m.layers):
        p = f"model.layers.{i}."
        parts = [p + "self_attn.q_proj.weight", p + "self_attn.k_proj.weight",
                 p + "self_attn.v_proj.weight"]
        assert torch.equal(L.qkv.w, torch.cat([u8(t[n]) for n in parts]))
        assert torch.equal(L.qkv.scale, torch.cat([t[n + sfx] for n in parts]))
        assert (L.qkv.N, L.qkv.K) == (CFG.q_out + 2 * CFG.kv_out, CFG.hidden)
        parts = [p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight"]
        assert torch.equal(L.gate_up.w, torch.cat([u8(t[n]) for n in parts]))
        assert torch.equal(L.gate_up.scale, torch.cat([t[n + sfx] for n in parts]))
        assert torch.equal(L.o.w, u8(t[p + "self_attn.o_proj.weight"]))
        assert torch.equal(L.down.scale, t[p + "mlp.down_proj.weight" + sfx])
        assert torch.equal(L.q_norm, t[p + "self_attn.q_norm.weight"])
        assert torch.equal(L.ffn_norm, t[p + "post_attention_layernorm.weight"])
        assert L.down.block == block and L.qkv.block == block


@pytest.mark.parametrize("block", [True, False])
@pytest.mark.parametrize("shards", [1, 3])
def test_load_and_fuse(tmp_path, block, shards):
    t = make_checkpoint(block=block)
    d = save(t, str(tmp_path / "ckpt"), shards)
    m = load_qwen3_fp8(d, CFG, device="cpu")
    check_loaded(m, t, block)


def test_single_file_path(tmp_path):
    t = make_checkpoint()
    d = save(t, str(tmp_path / "ckpt"))
    m = load_qwen3_fp8(os.path.join(d, "model.safetensors"), CFG, device="cpu")
    check_loaded(m, t, True)


def test_tied_lm_head(tmp_path):
    t = make_checkpoint()
    t["lm_head.weight"] = t["model.embed_tokens.weight"].clone()
    load_qwen3_fp8(save(t, str(tmp_path / "a")), CFG, device="cpu")
    t["lm_head.weight"] = _codes(np.random.default_rng(9), CFG.vocab, CFG.hidden)
    with pytest.raises(CheckpointError, match="A2: lm_head.weight present"):
        load_qwen3_fp8(save(t, str(tmp_path / "b")), CFG, device="cpu")


def _expect(tmp_path, t, pattern, cfg=CFG):
    d = save(t, str(tmp_path / "ckpt"))
    with pytest.raises(CheckpointError, match=pattern):
        load_qwen3_fp8(d, cfg, device="cpu")


def test_missing_tensor(tmp_path):
    t = make_checkpoint()
    del t["model.layers.1.mlp.down_proj.weight"]
    _expect(tmp_path, t, "missing tensor: model.layers.1.mlp.down_proj.weight")


def test_dtype_mismatch(tmp_path):
    t = make_checkpoint()
    t["model.layers.0.self_attn.k_norm.weight"] = torch.ones(CFG.head_dim)
    _expect(tmp_path, t, "dtype mismatch model.layers.0.self_attn.k_norm.weight: got F32 want BF16")


def test_shape_mismatch(tmp_path):
    t = make_checkpoint()
    t["model.layers.0.mlp.up_proj.weight"] = _codes(np.random.default_rng(1), CFG.inter, 128)
    _expect(tmp_path, t, r"shape\[1\] mismatch model.layers.0.mlp.up_proj.weight")


def test_missing_or_bad_scale(tmp_path):
    t = make_checkpoint(block=False)
    del t["model.layers.0.self_attn.v_proj.weight_scale"]
    _expect(tmp_path, t, "missing scale for model.layers.0.self_attn.v_proj.weight")
    t = make_checkpoint(block=False)
    t["model.layers.0.self_attn.o_proj.weight_scale"] = torch.ones(CFG.hidden, 2)
    _expect(tmp_path / "x", t, "scale shape bad for model.layers.0.self_attn.o_proj.weight_scale")
    t = make_checkpoint(block=True)
    t["model.layers.0.self_attn.o_proj.weight_scale_inv"] = torch.ones(1, 2)
    _expect(tmp_path / "y", t, r"shape\[0\] mismatch model.layers.0.self_attn.o_proj.weight_scale_inv")


def test_mixed_scale_formats(tmp_path):
    t = make_checkpoint(block=True)
    k = "model.layers.0.self_attn.k_proj.weight"
    del t[k + "_scale_inv"]
    t[k + "_scale"] = torch.ones(CFG.kv_out, 1)
    _expect(tmp_path, t, "mixed scale formats")


def test_block_fusion_needs_128_row_parts(tmp_path):
    cfg = Qwen3Config(vocab=384, hidden=256, n_layers=1, n_heads=2, n_kv_heads=1, head_dim=64,
                      inter=384)
    _expect(tmp_path, make_checkpoint(cfg), "cannot fuse model.layers.0.self_attn.k_proj.weight",
            cfg)


def test_header_format_tag(tmp_path):
    t = make_checkpoint()
    d = str(tmp_path / "ckpt")
    os.makedirs(d)
    save_file(t, os.path.join(d, "model.safetensors"), metadata={"format": "np"})
    with pytest.raises(CheckpointError, match="A12"):
        load_qwen3_fp8(d, CFG, device="cpu")


def test_no_checkpoint(tmp_path):
    with pytest.raises(CheckpointError, match="no safetensors files"):
        load_qwen3_fp8(str(tmp_path), CFG, device="cpu")
