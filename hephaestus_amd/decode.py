"""One W8A8 decode step of a Qwen3 model on the FP8 linear path.

The step is the reference's `forward_fp8` (src/hephaestus/forward.mojo:359-615)
with 128x128 block-scaled weights and an E4M3 KV cache holding one scale
per (layer, kv head, K|V):

    x = embed(token)                                     heph_embed_fp8
    per layer:
        qkv = rmsnorm(x, attn_norm) @ Wqkv^T             heph_fp8_linear_rmsnorm
              (norm + quant inside the GEMV; = heph_rmsnorm then heph_fp8_linear)
        q, k, v: per-head q/k norm, RoPE, k/v -> cache   heph_qk_norm_rope_kv
        att = attention(q, K[:pos+1], V[:pos+1])         heph_attention_fp8kv
              (both in the attention's launches:        heph_attention_qkv_fp8kv)
        x  += att @ Wo^T                                 heph_fp8_linear + ADD_RESIDUAL
        gu  = rmsnorm(x, ffn_norm) @ Wgate_up^T          heph_fp8_linear_rmsnorm
        act = silu(gate) * up                            heph_silu_mul
        x  += act @ Wdown^T
    logits = rmsnorm(x, norm) @ E^T   (f32, tied FP8 embedding; fused norm)
    token  = argmax(bf16(logits)), lowest index on ties  heph_argmax_bf16

Every op is a HIP kernel of libhephfp8.so; torch only holds device memory.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib as L
from . import kernels as HK
from .loader import Fp8Weight, Qwen3Config, Qwen3Fp8Weights, Qwen3Layer
from .weights import quantize_weight_fp8


def _ptr(t: torch.Tensor) -> int:
    if not t.is_cuda:
        raise ValueError("decode ops take device memory")
    return t.data_ptr()


def _call(name: str, *args) -> None:
    HK._check(getattr(L.lib(), name)(*args), name)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


# ------------------------------------------------------------- the ops ----

def embed_fp8(x, emb, emb_scale, tokens, block: bool = True) -> None:
    """x[t] = bf16(scale * e4m3(emb[tokens[t]])) (bf16 [n, hidden])."""
    _call("heph_embed_fp8", _ptr(x), _ptr(emb), _ptr(emb_scale), int(block), _ptr(tokens),
          tokens.numel(), emb.shape[0], emb.shape[1], _stream())


def rmsnorm(out, x, gamma, eps: float = 1e-6) -> None:
    rows, cols = (1, x.numel()) if x.dim() == 1 else (x.numel() // x.shape[-1], x.shape[-1])
    _call("heph_rmsnorm", _ptr(out), _ptr(x), _ptr(gamma), rows, cols, eps, _stream())


# The V cache holds 64-key blocks [n_blocks, n_kv, 8, 64, 16] (key j, kv head
# h, dim d at [j // 64, h, d // 16, j % 64, d % 16]); the K cache rows
# [n_keys, n_kv, 128].
V_BLOCK = 64


def v_blocks(rows):
    """[n, n_kv, 128] V codes (numpy or torch) -> the blocked layout
    [ceil(n/64), n_kv, 8, 64, 16], the padding keys zero."""
    n, n_kv = rows.shape[0], rows.shape[1]
    nb = -(-n // V_BLOCK)
    if isinstance(rows, torch.Tensor):
        pad = torch.zeros((nb * V_BLOCK, n_kv, 128), dtype=rows.dtype, device=rows.device)
        pad[:n] = rows
        return pad.view(nb, V_BLOCK, n_kv, 8, 16).permute(0, 2, 3, 1, 4).contiguous()
    pad = np.zeros((nb * V_BLOCK, n_kv, 128), dtype=rows.dtype)
    pad[:n] = rows
    return np.ascontiguousarray(pad.reshape(nb, V_BLOCK, n_kv, 8, 16).transpose(0, 2, 3, 1, 4))


def v_rows(blocks, n: int | None = None):
    """The inverse of v_blocks: [nb, n_kv, 8, 64, 16] -> [n, n_kv, 128]
    (n = nb * 64 by default)."""
    nb, n_kv = blocks.shape[0], blocks.shape[1]
    n = nb * V_BLOCK if n is None else n
    if isinstance(blocks, torch.Tensor):
        return blocks.permute(0, 3, 1, 2, 4).reshape(nb * V_BLOCK, n_kv, 128)[:n]
    return blocks.transpose(0, 3, 1, 2, 4).reshape(nb * V_BLOCK, n_kv, 128)[:n]


def qk_norm_rope_kv(qkv, q_gamma, k_gamma, k_cache, v_cache, kv_inv, n_heads: int, n_kv: int,
                    pos: int, theta: float = 1e6, eps: float = 1e-6) -> None:
    """q/k norm + RoPE at pos (q in place), k and v codes into key pos of
    k_cache (rows) and v_cache (64-key blocks, v_blocks' layout)."""
    _call("heph_qk_norm_rope_kv", _ptr(qkv), _ptr(q_gamma), _ptr(k_gamma), _ptr(k_cache),
          _ptr(v_cache), _ptr(kv_inv), n_heads, n_kv, 128, pos, theta, eps, _stream())


def attention_ws(n_heads: int, n_keys: int, device="cuda") -> torch.Tensor:
    """Scratch for attention_fp8kv with up to n_keys keys."""
    n = L.lib().heph_attention_ws_bytes(n_heads, n_keys)
    return torch.empty(max(n, 16), dtype=torch.uint8, device=device)


def attention_fp8kv(out, q, k_cache, v_cache, kv_scale, n_heads: int, n_kv: int,
                    n_keys: int, ws: torch.Tensor | None = None) -> None:
    """k_cache: rows [>= n_keys, n_kv, 128]; v_cache: 64-key blocks
    (v_blocks' layout) of at least ceil(n_keys / 64) blocks."""
    # (a key count the library refuses is left to its status code)
    if 0 < n_keys <= L.ATTN_MAX_KEYS and \
            v_cache.numel() < -(-n_keys // V_BLOCK) * V_BLOCK * n_kv * 128:
        raise ValueError(f"v_cache of {v_cache.numel()} bytes holds fewer than "
                         f"ceil({n_keys}/64) blocks")
    if ws is None:
        ws = attention_ws(n_heads, n_keys, device=out.device)
    _call("heph_attention_fp8kv", _ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache),
          _ptr(kv_scale), n_heads, n_kv, 128, n_keys, _ptr(ws), ws.numel(), _stream())


def rope_table(n_pos: int, theta: float = 1e6, device="cuda") -> torch.Tensor:
    """(cos, sin) bf16 of the 64 RoPE pairs of a 128-wide head at positions
    0..n_pos-1, [n_pos, 64, 2]: the values qk_norm_rope_kv computes."""
    t = torch.empty(n_pos, 64, 2, dtype=torch.bfloat16, device=device)
    _call("heph_rope_table_bf16", _ptr(t), n_pos, 128, theta, _stream())
    return t


def attention_qkv_fp8kv(out, qkv, q_gamma, k_gamma, k_cache, v_cache, kv_scale, kv_inv,
                        n_heads: int, n_kv: int, pos: int, theta: float = 1e6,
                        eps: float = 1e-6, ws: torch.Tensor | None = None,
                        rope: torch.Tensor | None = None) -> None:
    """qk_norm_rope_kv into cache key pos, then attention_fp8kv over pos + 1
    keys, in the attention's two launches (the same out and cache bytes;
    q in qkv is not rotated in place). rope: a rope_table of more than pos
    rows for this theta, or None to compute pos's cos/sin in the call."""
    if ws is None:
        ws = attention_ws(n_heads, pos + 1, device=out.device)
    if rope is not None and rope.shape[0] <= pos:
        raise ValueError(f"rope table of {rope.shape[0]} rows has no row {pos}")
    if 0 <= pos < L.ATTN_MAX_KEYS and v_cache.numel() < (pos // V_BLOCK + 1) * V_BLOCK * n_kv * 128:
        raise ValueError(f"v_cache of {v_cache.numel()} bytes has no block for key {pos}")
    _call("heph_attention_qkv_fp8kv", _ptr(out), _ptr(qkv), _ptr(q_gamma), _ptr(k_gamma),
          _ptr(k_cache), _ptr(v_cache), _ptr(kv_scale), _ptr(kv_inv),
          None if rope is None else _ptr(rope), 0 if rope is None else rope.shape[0],
          n_heads, n_kv, 128, pos, theta, eps, _ptr(ws), ws.numel(), _stream())


def silu_mul(out, gate, up, n: int) -> None:
    _call("heph_silu_mul", _ptr(out), _ptr(gate), _ptr(up), n, _stream())


def argmax_ws(n: int, device="cuda") -> torch.Tensor:
    """Scratch for argmax_bf16 over n logits."""
    return torch.empty(max(L.lib().heph_argmax_ws_bytes(n), 16), dtype=torch.uint8, device=device)


def argmax_bf16(out_idx, logits, ws: torch.Tensor | None = None) -> None:
    if ws is None:
        ws = argmax_ws(logits.numel(), device=logits.device)
    _call("heph_argmax_bf16", _ptr(out_idx), _ptr(logits), logits.numel(), _ptr(ws), ws.numel(),
          _stream())


# ---------------------------------------------------------------- weights ----

def _rand_fp8(g: torch.Generator, N: int, K: int, device, std: float = 0.02) -> Fp8Weight:
    w = (torch.randn(N, K, generator=g, device=device) * std).to(torch.bfloat16)
    q, s = quantize_weight_fp8(w)
    return Fp8Weight(q, s, True)


def _rand_gamma(g: torch.Generator, n: int, device, centre: float = 1.0,
                std: float = 0.1) -> torch.Tensor:
    return (centre + std * torch.randn(n, generator=g, device=device)).to(torch.bfloat16)


# Std of the residual-branch output projections (o_proj, down_proj) relative
# to the other linears in conditioned_init: with it the 36 branches make up
# ~1 % of the final residual stream of the configs[4] model.
CONDITIONED_BRANCH_SCALE = 3e-5


def random_init(cfg: Qwen3Config, seed: int = 0, device="cuda",
                branch_scale: float = 1.0, final_gamma_centre: float = 1.0,
                final_gamma_std: float = 0.1) -> Qwen3Fp8Weights:
    """Random-init Qwen3 weights: every linear ~N(0, 0.02) quantized per
    128x128 block on the GPU (tied FP8 embedding), norm gammas 1 + 0.1 N(0,1).
    branch_scale multiplies the std of o_proj and down_proj (the projections
    that write into the residual stream); the final norm's gamma is
    final_gamma_centre + final_gamma_std * N(0,1)."""
    g = torch.Generator(device=device).manual_seed(seed)
    H, I = cfg.hidden, cfg.inter
    bstd = 0.02 * branch_scale
    out = Qwen3Fp8Weights(cfg, _rand_fp8(g, cfg.vocab, H, device),
                          _rand_gamma(g, H, device, final_gamma_centre, final_gamma_std))
    for _ in range(cfg.n_layers):
        out.layers.append(Qwen3Layer(
            attn_norm=_rand_gamma(g, H, device), q_norm=_rand_gamma(g, cfg.head_dim, device),
            k_norm=_rand_gamma(g, cfg.head_dim, device), ffn_norm=_rand_gamma(g, H, device),
            qkv=_rand_fp8(g, cfg.q_out + 2 * cfg.kv_out, H, device),
            o=_rand_fp8(g, H, cfg.q_out, device, bstd),
            gate_up=_rand_fp8(g, 2 * I, H, device),
            down=_rand_fp8(g, H, I, device, bstd)))
    return out


def conditioned_init(cfg: Qwen3Config, seed: int = 0, device="cuda") -> Qwen3Fp8Weights:
    """The random init the end-to-end argmax check runs on.

    With every linear ~N(0, 0.02) the residual stream is made of the layers'
    branch outputs (~1 per element against 0.02 for the embedding), each
    layer re-normalizes it, and a W8A8 step is chaotic: two correct
    implementations whose fp32 sums differ in the last bit flip E4M3 codes
    at rounding boundaries, and after 36 layers their logits differ by a
    third of their spread, far more than the top-2 gap of 151936 random
    logits (~1/5 of it). Here o_proj and down_proj are drawn with
    CONDITIONED_BRANCH_SCALE times that std, so the embedding carries the
    stream and the branches stay a small, bounded share of it; the final
    norm's gamma is N(0, 1) (zero mean), since with gamma near 1 the tied
    lm_head would return the input token itself by a margin of ~50
    standard deviations."""
    return random_init(cfg, seed, device, branch_scale=CONDITIONED_BRANCH_SCALE,
                       final_gamma_centre=0.0, final_gamma_std=1.0)


# --------------------------------------------------------------- KV cache ----

class KVCache:
    """E4M3 codes k [n_layers, max_ctx, n_kv, 128] and v in 64-key blocks
    [n_layers, ceil(max_ctx/64), n_kv, 8, 64, 16] (v_blocks' layout) with f32
    scales [n_layers, 2*n_kv] (K heads then V heads) and their reciprocals."""

    def __init__(self, cfg: Qwen3Config, max_ctx: int, device="cuda"):
        if max_ctx > L.ATTN_MAX_KEYS:
            raise ValueError(f"max_ctx {max_ctx} > {L.ATTN_MAX_KEYS}")
        shape = (cfg.n_layers, max_ctx, cfg.n_kv_heads, cfg.head_dim)
        self.cfg, self.max_ctx = cfg, max_ctx
        self.k = torch.zeros(shape, dtype=torch.uint8, device=device)
        self.v = torch.zeros((cfg.n_layers, -(-max_ctx // V_BLOCK), cfg.n_kv_heads, 8, V_BLOCK,
                              16), dtype=torch.uint8, device=device)
        self.scale = torch.ones(cfg.n_layers, 2 * cfg.n_kv_heads, dtype=torch.float32,
                                device=device)
        self.inv = torch.ones_like(self.scale)

    def fill_synthetic(self, n_pos: int, seed: int = 1) -> None:
        """Rows 0..n_pos-1 from bf16 ~N(0,1) values. Each (layer, head, K|V)
        scale is amax/448 over those rows (1.0 below 1e-12), computed on the
        host in f32 as the quantizer does; codes = e4m3(x * (1/s))."""
        g = torch.Generator(device=self.k.device).manual_seed(seed)
        cfg = self.cfg
        scale = np.ones((cfg.n_layers, 2 * cfg.n_kv_heads), np.float32)
        for li in range(cfg.n_layers):
            for j, dst in enumerate((self.k, self.v)):
                x = torch.randn(n_pos, cfg.n_kv_heads, cfg.head_dim, generator=g,
                                device=self.k.device).to(torch.bfloat16).float()
                amax = x.abs().amax(dim=(0, 2)).cpu().numpy().astype(np.float32)
                s = amax / np.float32(448.0)
                s[s < np.float32(1e-12)] = np.float32(1.0)
                inv = (np.float32(1.0) / s).astype(np.float32)
                scale[li, j * cfg.n_kv_heads:(j + 1) * cfg.n_kv_heads] = s
                inv_t = torch.from_numpy(inv).to(x.device).view(1, -1, 1)
                codes = (x * inv_t).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
                if dst is self.k:
                    dst[li, :n_pos] = codes
                else:
                    dst[li, :-(-n_pos // V_BLOCK)] = v_blocks(codes)
        self.scale.copy_(torch.from_numpy(scale))
        self.inv.copy_(torch.from_numpy((np.float32(1.0) / scale).astype(np.float32)))


# ---------------------------------------------------------------- decoder ----

# Longest row heph_fp8_linear_rmsnorm takes (its row and gamma sit in LDS).
NORM_LINEAR_MAX_K = 8192

class Qwen3Decoder:
    """Holds the activations and workspaces of a single-token decode step."""

    def __init__(self, weights: Qwen3Fp8Weights, kv: KVCache):
        self.w, self.kv, cfg = weights, kv, weights.cfg
        if not weights.embed.block:
            raise ValueError("the decode step takes 128x128 block-scaled weights")
        if cfg.head_dim != 128:
            raise ValueError("head_dim must be 128")
        dev = weights.embed.w.device
        H, I, Q, KV = cfg.hidden, cfg.inter, cfg.q_out, cfg.kv_out
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.x = torch.empty(1, H, **bf)
        self.xn = torch.empty(1, H, **bf)
        self.qkv = torch.empty(1, Q + 2 * KV, **bf)
        self.att = torch.empty(1, Q, **bf)
        self.gu = torch.empty(1, 2 * I, **bf)
        self.act = torch.empty(1, I, **bf)
        self.logits = torch.empty(1, cfg.vocab, dtype=torch.float32, device=dev)
        self.next_token = torch.zeros(1, dtype=torch.int32, device=dev)
        self.token = torch.zeros(1, dtype=torch.int32, device=dev)
        self.q_ws, self.s_ws = HK.workspace(1, max(H, Q, I), device=dev)
        self.attn_ws = attention_ws(cfg.n_heads, kv.max_ctx, device=dev)
        self.rope = rope_table(kv.max_ctx, cfg.theta, device=dev)
        self.arg_ws = argmax_ws(cfg.vocab, device=dev)

    def _linear(self, c, a, fw: Fp8Weight, K: int, residual: bool = False):
        fn = HK.linear_add_residual_fp8 if residual else HK.linear_fp8
        fn(c, a, fw.w, fw.scale, self.q_ws, self.s_ws, 1, fw.N, K)

    def _norm_linear(self, c, gamma, fw: Fp8Weight, K: int, eps: float, rec, li, op):
        """c = rmsnorm(self.x, gamma) @ fw: the norm inside the fused GEMV
        (heph_fp8_linear_rmsnorm: heph_rmsnorm + the linear, bit for bit
        under the norm form's launch shape) for
        rows up to NORM_LINEAR_MAX_K; longer rows take heph_rmsnorm, then
        the linear. A traced step also writes the normalized row to self.xn,
        for the record only."""
        if K > NORM_LINEAR_MAX_K:
            rmsnorm(self.xn, self.x, gamma, eps)
            self._linear(c, self.xn, fw, K)
        else:
            HK.linear_fp8_rmsnorm(c, self.x, gamma, eps, fw.w, fw.scale, self.q_ws, self.s_ws,
                                  fw.N, K)
        if rec.tracing:
            rmsnorm(self.xn, self.x, gamma, eps)
            rec(li, op, self.xn)

    def step(self, token, pos: int, trace: list | None = None) -> torch.Tensor:
        """Decode `token` (int or int32 device tensor [1]) at position pos;
        the KV cache row pos is written. Returns the argmax token (int32
        device tensor [1]); logits stay in self.logits. With `trace`, every
        op's output is appended as (layer, op, host copy) after a device
        synchronization (for op-by-op checks; slow)."""
        cfg, w, kv = self.w.cfg, self.w, self.kv
        if not 0 <= pos < kv.max_ctx:
            raise ValueError(f"pos {pos} outside the cache (max_ctx {kv.max_ctx})")
        if isinstance(token, torch.Tensor):
            self.token.copy_(token.view(1))
        else:
            self.token.fill_(int(token))

        def rec(li, op, t):
            if trace is not None:
                torch.cuda.synchronize()
                t = t.detach()
                a = (t.view(torch.int16).cpu().numpy().view(np.uint16) if t.dtype == torch.bfloat16
                     else t.cpu().numpy())
                trace.append((li, op, a.reshape(-1).copy()))
        rec.tracing = trace is not None

        H, I, Q = cfg.hidden, cfg.inter, cfg.q_out
        NH, NKV, eps = cfg.n_heads, cfg.n_kv_heads, cfg.eps
        embed_fp8(self.x, w.embed.w, w.embed.scale, self.token)
        rec(-1, "embed", self.x)
        for li, lw in enumerate(w.layers):
            self._norm_linear(self.qkv, lw.attn_norm, lw.qkv, H, eps, rec, li, "attn_norm")
            rec(li, "qkv", self.qkv)
            if rec.tracing:
                qk_norm_rope_kv(self.qkv, lw.q_norm, lw.k_norm, kv.k[li], kv.v[li],
                                kv.inv[li], NH, NKV, pos, cfg.theta, eps)
                rec(li, "q_rope", self.qkv[:, :Q])
                rec(li, "k_codes", kv.k[li, pos])
                rec(li, "v_codes", kv.v[li, pos // V_BLOCK, :, :, pos % V_BLOCK])
                attention_fp8kv(self.att, self.qkv, kv.k[li], kv.v[li], kv.scale[li], NH, NKV,
                                pos + 1, self.attn_ws)
            else:
                # q/k norm, RoPE and the K/V write inside the attention's
                # scores kernel: bit for bit the two ops above
                attention_qkv_fp8kv(self.att, self.qkv, lw.q_norm, lw.k_norm, kv.k[li],
                                    kv.v[li], kv.scale[li], kv.inv[li], NH, NKV, pos, cfg.theta,
                                    eps, self.attn_ws, self.rope)
            rec(li, "attention", self.att)
            self._linear(self.x, self.att, lw.o, Q, residual=True)
            rec(li, "o_residual", self.x)
            if rec.tracing:
                # the ops one by one, so that the trace holds gate_up's output
                self._norm_linear(self.gu, lw.ffn_norm, lw.gate_up, H, eps, rec, li, "ffn_norm")
                rec(li, "gate_up", self.gu)
                silu_mul(self.act, self.gu, self.gu[:, I:], I)
                rec(li, "silu_mul", self.act)
            elif H <= NORM_LINEAR_MAX_K:
                # RMSNorm, gate/up and SwiGLU in one launch, bit for bit the
                # three ops
                HK.linear_fp8_swiglu(self.act, self.x, lw.ffn_norm, eps, lw.gate_up.w,
                                     lw.gate_up.scale, self.q_ws, self.s_ws, lw.gate_up.N, H)
            else:
                rmsnorm(self.xn, self.x, lw.ffn_norm, eps)
                HK.linear_fp8_swiglu(self.act, self.xn, None, eps, lw.gate_up.w,
                                     lw.gate_up.scale, self.q_ws, self.s_ws, lw.gate_up.N, H)
            # down with its quantization fused in the GEMV: for one row ~1.2 us
            # per layer faster on MI355X than the producer-side form
            # (heph_silu_mul_quant_fp8), which pays at prefill sizes
            self._linear(self.x, self.act, lw.down, I, residual=True)
            rec(li, "down_residual", self.x)
        self._norm_linear(self.logits, w.final_norm, w.embed, H, eps, rec, -1, "final_norm")
        rec(-1, "logits", self.logits)
        argmax_bf16(self.next_token, self.logits, self.arg_ws)
        rec(-1, "argmax", self.next_token)
        return self.next_token


def host_model(w: Qwen3Fp8Weights) -> dict:
    """Host copies of the weights in the form oracle.decode_step takes."""
    def u16(t):
        return t.view(torch.int16).cpu().numpy().view(np.uint16)

    cfg = w.cfg
    m = {"cfg": {"hidden": cfg.hidden, "n_heads": cfg.n_heads, "n_kv_heads": cfg.n_kv_heads,
                 "inter": cfg.inter, "eps": cfg.eps, "theta": cfg.theta},
         "embed": w.embed.w.cpu().numpy(), "embed_scale": w.embed.scale.cpu().numpy(),
         "final_norm": u16(w.final_norm), "layers": []}
    for lw in w.layers:
        d = {"attn_norm": u16(lw.attn_norm), "q_norm": u16(lw.q_norm), "k_norm": u16(lw.k_norm),
             "ffn_norm": u16(lw.ffn_norm)}
        for name in ("qkv", "o", "gate_up", "down"):
            fw = getattr(lw, name)
            d[name] = fw.w.cpu().numpy()
            d[name + "_scale"] = fw.scale.cpu().numpy()
        m["layers"].append(d)
    return m


def host_kv(kv: KVCache) -> dict:
    """Host copies in the oracle's form (v as rows [n_layers, max_ctx, n_kv,
    128])."""
    v = np.stack([v_rows(b, kv.max_ctx) for b in kv.v.cpu().numpy()])
    return {"k": kv.k.cpu().numpy(), "v": v,
            "scale": kv.scale.cpu().numpy(), "inv": kv.inv.cpu().numpy()}


def n_params_bytes(cfg: Qwen3Config) -> int:
    """FP8 weight bytes one decode step streams (linears + tied lm_head)."""
    per_layer = (cfg.q_out + 2 * cfg.kv_out) * cfg.hidden + cfg.hidden * cfg.q_out + \
        2 * cfg.inter * cfg.hidden + cfg.hidden * cfg.inter
    return cfg.n_layers * per_layer + cfg.vocab * cfg.hidden
