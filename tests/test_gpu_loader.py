"""The HIP path on weights that came through the safetensors loader.

A tiny Qwen3-shaped FP8 checkpoint is written with the safetensors library:
every linear ~N(0, 0.02) quantized by the oracle's weight quantizer, either in
128x128 blocks (`weight_scale_inv`) or per output channel (`weight_scale`
[N, 1]), one file or three shards. load_qwen3_fp8(device="cuda") validates
it and fuses q|k|v and gate|up by copy. Then:

  * every loaded linear (the fused ones included) runs through linear_fp8 at
    M = 1 (decode GEMV), 8 (batched decode) and 64 (GEMM), and
    linear_add_residual_fp8 at M = 1, against the oracle on the checkpoint's
    own parts concatenated on the host (not the loader's tensors), so a
    fusion that misplaces a row or a scale row fails;
  * with 128x128 blocks, a whole decode step on the loaded weights is
    replayed op by op against the oracle.

The reference runs forward_fp8 on the views its loader builds from such a
checkpoint (src/hephaestus/loader.mojo:554-628, forward.mojo:359-615;
scripts/stage_weights.py:20-106 stages the safetensors files).
"""
import numpy as np
import pytest
import torch

from hephaestus_amd import decode as DEC
from hephaestus_amd import kernels as HK
from hephaestus_amd.loader import Qwen3Config, load_qwen3_fp8
from oracle import oracle as O
from tests._gpu import dev, host_bf16, max_abs_rel
from tests.test_gpu_decode import check_ops, replay
from tests.test_loader import save

pytestmark = pytest.mark.gpu

CFG = Qwen3Config(vocab=1024, hidden=512, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=128,
                  inter=768)


def _bf16(x):
    return O.f32_to_bf16(np.ascontiguousarray(x, np.float32))


def _quantized(seed, n, k, block):
    """(codes u8 [n, k], scales f32) of W ~ N(0, 0.02)."""
    w = O.gen_normal(seed, n * k, 0.0, 0.02).reshape(n, k)
    return O.quant_weight(w, 128, 128) if block else O.quant_weight(w, 1, k)


def make_checkpoint(cfg, block, seed=0):
    """(safetensors tensor dict, host parts {name: (codes, scales)} and norms)."""
    t, parts = {}, {}
    s = [seed * 1000]

    def nxt():
        s[0] += 1
        return s[0]

    def lin(name, n, k):
        q, sc = _quantized(nxt(), n, k, block)
        parts[name] = (q, sc)
        t[name] = torch.from_numpy(q.copy()).view(torch.float8_e4m3fn)
        t[name + ("_scale_inv" if block else "_scale")] = torch.from_numpy(sc.copy())

    def norm(name, n):
        b = _bf16(1.0 + 0.1 * O.gen_normal(nxt(), n))
        parts[name] = b
        t[name] = torch.from_numpy(b.view(np.int16).copy()).view(torch.bfloat16)

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
    return t, parts


def host_fused(parts, names):
    """Codes and scale rows of `names` stacked along N on the host."""
    return (np.ascontiguousarray(np.concatenate([parts[n][0] for n in names])),
            np.ascontiguousarray(np.concatenate([parts[n][1] for n in names]), np.float32))


def layer_linears(cfg, i):
    p = f"model.layers.{i}."
    return {"qkv": ([p + "self_attn.q_proj.weight", p + "self_attn.k_proj.weight",
                     p + "self_attn.v_proj.weight"], cfg.hidden),
            "o": ([p + "self_attn.o_proj.weight"], cfg.q_out),
            "gate_up": ([p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight"], cfg.hidden),
            "down": ([p + "mlp.down_proj.weight"], cfg.inter)}


@pytest.mark.parametrize("block", [True, False], ids=["block128", "per_channel"])
@pytest.mark.parametrize("shards", [1, 3])
def test_loaded_linears_vs_oracle(tmp_path, block, shards):
    t, parts = make_checkpoint(CFG, block, seed=3 + shards)
    m = load_qwen3_fp8(save(t, str(tmp_path / "ckpt"), shards), CFG, device="cuda")
    assert m.embed.w.is_cuda and m.layers[0].qkv.w.is_cuda
    # group 128 with block weights; the reference's per-token group with
    # per-channel weights
    checked = 0
    for i, lw in enumerate(m.layers):
        for name, (names, K) in layer_linears(CFG, i).items():
            fw = getattr(lw, name)
            qw, sw = host_fused(parts, names)
            N = qw.shape[0]
            assert (fw.N, fw.K, fw.block) == (N, K, block), name
            gk = 128 if block else K
            bn, bk = (128, 128) if block else (1, K)
            for M in (1, 8, 64):
                x = O.gen_act_bf16(100 * i + M + N, M, K)
                c = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
                q_ws, s_ws = HK.workspace(M, K, group_k=gk, n=N)
                HK.linear_fp8(c, dev(x), fw.w, fw.scale, q_ws, s_ws, M, N, K, group_k=gk)
                torch.cuda.synchronize()
                ref = O.quant_linear(x, qw, sw, group_k=gk, bn=bn, bk=bk)
                got = O.bf16_to_f32(host_bf16(c))
                assert max_abs_rel(got, ref) <= 1e-2, (i, name, M, HK.last_kernel())
                checked += 1
            # the residual form at M = 1 on the same loaded tensors
            x = O.gen_act_bf16(7 + N, 1, K)
            r = _bf16(O.gen_normal(9 + N, N))
            c = dev(r).view(1, N)
            q_ws, s_ws = HK.workspace(1, K, group_k=gk)
            HK.linear_add_residual_fp8(c, dev(x), fw.w, fw.scale, q_ws, s_ws, 1, N, K,
                                       group_k=gk)
            torch.cuda.synchronize()
            ref = O.quant_linear(x, qw, sw, group_k=gk, bn=bn, bk=bk)[0] + O.bf16_to_f32(r)
            assert max_abs_rel(O.bf16_to_f32(host_bf16(c))[0], ref) <= 1e-2, (i, name)
    assert checked == 3 * 4 * CFG.n_layers


def host_model_from_parts(cfg, parts):
    """The oracle's model dict built from the checkpoint parts (q|k|v and
    gate|up stacked here, independently of the loader)."""
    emb, esc = parts["model.embed_tokens.weight"]
    m = {"cfg": {"hidden": cfg.hidden, "n_heads": cfg.n_heads, "n_kv_heads": cfg.n_kv_heads,
                 "inter": cfg.inter, "eps": cfg.eps, "theta": cfg.theta},
         "embed": emb, "embed_scale": esc, "final_norm": parts["model.norm.weight"],
         "layers": []}
    for i in range(cfg.n_layers):
        p = f"model.layers.{i}."
        d = {"attn_norm": parts[p + "input_layernorm.weight"],
             "q_norm": parts[p + "self_attn.q_norm.weight"],
             "k_norm": parts[p + "self_attn.k_norm.weight"],
             "ffn_norm": parts[p + "post_attention_layernorm.weight"]}
        for name, (names, _) in layer_linears(cfg, i).items():
            d[name], d[name + "_scale"] = host_fused(parts, names)
        m["layers"].append(d)
    return m


@pytest.mark.parametrize("shards", [1, 3])
def test_loaded_decode_step_op_by_op(tmp_path, shards):
    # forward_fp8 on loaded, fused weights: every op of the step recomputed by
    # the oracle from the GPU's own inputs (the bars of the random-init
    # decode test), the oracle's weights taken from the checkpoint parts
    t, parts = make_checkpoint(CFG, True, seed=11 + shards)
    w = load_qwen3_fp8(save(t, str(tmp_path / "ckpt"), shards), CFG, device="cuda")
    ctx, token = 200, 777
    kv = DEC.KVCache(CFG, ctx + 1)
    kv.fill_synthetic(ctx, seed=5)
    kvh = DEC.host_kv(kv)
    trace = []
    tok = int(DEC.Qwen3Decoder(w, kv).step(token, ctx, trace=trace).item())
    check_ops(replay(host_model_from_parts(CFG, parts), kvh, token, ctx, trace))
    assert tok == int(trace[-1][2][0])
