"""Qwen3 W8A8 FP8 checkpoint loader (safetensors) for the FP8 linear path.

Mirrors the reference's load path -- `scripts/stage_weights.py:20-106`
(safetensors header checks, sharded or single-file checkpoints, the tied
lm_head) and `src/hephaestus/loader.mojo:478-628` (`_require` /
`verify_manifest_fp8`: every tensor present with the expected dtype and
shape, every FP8 weight paired with its F32 scale, no separate lm_head) --
but reads the safetensors files directly instead of a staged blob.

Two scale formats are accepted for every FP8 weight `<name>.weight`:
  * `<name>.weight_scale_inv`  F32 [ceil(N/128), ceil(K/128)]: 128x128 block
    scales (dequant multipliers), the north-star format;
  * `<name>.weight_scale`      F32 [N, 1]: the reference's per-channel
    scale (docs/fp8-checkpoint-format.md:40-57).
The fused projections the linear path runs -- q|k|v as one N = q_out +
2*kv_out weight and gate|up as one N = 2*inter weight -- are built by
copying the parts and their scale rows into new tensors; arena adjacency is
not relied on (the reference rejected it, DECISIONS.md:45). Block-scaled
parts must then start on a 128-row boundary.

Only data is read: the header is JSON and tensor bytes are mapped with
numpy; nothing in a checkpoint is executed.
"""
from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass, field

import numpy as np

DTYPES = {"F8_E4M3": np.uint8, "BF16": np.uint16, "F32": np.float32}
WIDTH = {"F8_E4M3": 1, "BF16": 2, "F32": 4}
BLOCK = 128


class CheckpointError(ValueError):
    """A checkpoint that does not match the expected Qwen3 FP8 manifest."""


@dataclass(frozen=True)
class Qwen3Config:
    """Qwen3-4B architecture (reference src/hephaestus/constants.mojo:8-30;
    the random-init decode uses RoPE theta 1e6)."""
    vocab: int = 151936
    hidden: int = 2560
    n_layers: int = 36
    n_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = 128
    inter: int = 9728
    eps: float = 1e-6
    theta: float = 1e6

    @property
    def q_out(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def kv_out(self) -> int:
        return self.n_kv_heads * self.head_dim


@dataclass
class Fp8Weight:
    """E4M3 codes [N, K] (uint8) and their scales: block [ceil(N/128),
    ceil(K/128)] when `block`, else per-channel [N, 1]."""
    w: object
    scale: object
    block: bool

    @property
    def N(self) -> int:
        return int(self.w.shape[0])

    @property
    def K(self) -> int:
        return int(self.w.shape[1])


@dataclass
class Qwen3Layer:
    attn_norm: object
    q_norm: object
    k_norm: object
    ffn_norm: object
    qkv: Fp8Weight
    o: Fp8Weight
    gate_up: Fp8Weight
    down: Fp8Weight


@dataclass
class Qwen3Fp8Weights:
    cfg: Qwen3Config
    embed: Fp8Weight            # tied: also the lm_head
    final_norm: object
    layers: list = field(default_factory=list)


# ------------------------------------------------------------ safetensors ----

def read_header(path: str) -> tuple[dict, int]:
    """(header dict, byte offset of the data section) of one file."""
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise CheckpointError(f"{path}: truncated safetensors header")
        n = struct.unpack("<Q", raw)[0]
        if n > (100 << 20):
            raise CheckpointError(f"{path}: header length {n} is implausible")
        header = json.loads(f.read(n))
    # A12 (stage_weights.py:25-28): the torch format tag.
    fmt = header.get("__metadata__", {}).get("format")
    if fmt != "pt":
        raise CheckpointError(f"A12: {path} metadata format is {fmt!r}, expected 'pt'")
    return header, 8 + n


class TensorIndex:
    """Name -> (file, dtype, shape, byte range) over one or more shards."""

    def __init__(self, path: str):
        files = self._files(path)
        self.entries: dict[str, tuple] = {}
        for fp in files:
            header, start = read_header(fp)
            size = os.path.getsize(fp)
            for name, meta in header.items():
                if name == "__metadata__":
                    continue
                if name in self.entries:
                    raise CheckpointError(f"duplicate tensor: {name}")
                a, b = meta["data_offsets"]
                if not (0 <= a <= b and start + b <= size):
                    raise CheckpointError(f"data offsets out of range: {name}")
                self.entries[name] = (fp, meta["dtype"], tuple(meta["shape"]), start + a,
                                      start + b)

    @staticmethod
    def _files(path: str) -> list[str]:
        if os.path.isfile(path):
            return [path]
        index = os.path.join(path, "model.safetensors.index.json")
        single = os.path.join(path, "model.safetensors")
        if os.path.exists(index):
            with open(index) as f:
                weight_map = json.load(f)["weight_map"]
            return [os.path.join(path, s) for s in sorted(set(weight_map.values()))]
        if os.path.exists(single):
            return [single]
        raise CheckpointError(f"no safetensors files found in {path}")

    def __contains__(self, name: str) -> bool:
        return name in self.entries

    def require(self, name: str, dtype: str, shape: tuple) -> None:
        """The reference's `_require` (loader.mojo:489-513)."""
        if name not in self.entries:
            raise CheckpointError("missing tensor: " + name)
        _, dt, shp, a, b = self.entries[name]
        if dt != dtype and not (dtype == "F8_E4M3" and dt == "F8E4M3"):
            raise CheckpointError(f"dtype mismatch {name}: got {dt} want {dtype}")
        if len(shp) != len(shape):
            raise CheckpointError("rank mismatch " + name)
        for i, (got, want) in enumerate(zip(shp, shape)):
            if got != want:
                raise CheckpointError(f"shape[{i}] mismatch {name}: got {got} want {want}")
        if b - a != int(np.prod(shape)) * WIDTH[dtype]:
            raise CheckpointError("byte_size mismatch " + name)

    def read(self, name: str) -> np.ndarray:
        fp, dt, shp, a, b = self.entries[name]
        dtype = DTYPES["F8_E4M3" if dt == "F8E4M3" else dt]
        arr = np.memmap(fp, dtype=np.uint8, mode="r", offset=a, shape=(b - a,))
        return np.asarray(arr).view(dtype).reshape(shp)


# ------------------------------------------------------------------ loader ----

def _to_device(a: np.ndarray, device):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a).copy())
    if a.dtype == np.uint16:
        t = t.view(torch.int16).view(torch.bfloat16)
    return t.to(device)


def _fp8(ix: TensorIndex, name: str, N: int, K: int) -> tuple[np.ndarray, np.ndarray, bool]:
    ix.require(name, "F8_E4M3", (N, K))
    block_name, chan_name = name + "_scale_inv", name + "_scale"
    if block_name in ix:
        ix.require(block_name, "F32", (-(-N // BLOCK), -(-K // BLOCK)))
        return ix.read(name), ix.read(block_name), True
    if chan_name in ix:
        _, dt, shp, _, _ = ix.entries[chan_name]
        if dt != "F32":
            raise CheckpointError("scale not F32: " + chan_name)
        if len(shp) != 2 or shp[0] != N or shp[1] != 1:
            raise CheckpointError("scale shape bad for " + chan_name)
        return ix.read(name), ix.read(chan_name), False
    raise CheckpointError("missing scale for " + name)


def _fused(ix: TensorIndex, names: list[str], Ns: list[int], K: int, device) -> Fp8Weight:
    """Concatenate FP8 weights along N (copy) with their scale rows."""
    parts = [_fp8(ix, n, N, K) for n, N in zip(names, Ns)]
    block = parts[0][2]
    if any(p[2] != block for p in parts):
        raise CheckpointError("mixed scale formats in " + ", ".join(names))
    if block:
        for n, N in zip(names[:-1], Ns[:-1]):
            if N % BLOCK:
                raise CheckpointError(f"cannot fuse {n}: N = {N} is not a multiple of "
                                      f"{BLOCK}, so its scale blocks would straddle")
    w = np.concatenate([p[0] for p in parts], axis=0)
    s = np.concatenate([p[1] for p in parts], axis=0)
    return Fp8Weight(_to_device(w, device), _to_device(s.astype(np.float32), device), block)


def load_qwen3_fp8(path: str, cfg: Qwen3Config = Qwen3Config(), device="cuda") -> Qwen3Fp8Weights:
    """Validate and load a Qwen3 FP8 checkpoint (directory with
    model.safetensors or model.safetensors.index.json, or one file)."""
    ix = TensorIndex(path)
    H, Q, KV, I, D = cfg.hidden, cfg.q_out, cfg.kv_out, cfg.inter, cfg.head_dim

    # Tied embeddings (stage_weights.py:84-93): a separate lm_head is only
    # accepted when it is byte-identical to embed_tokens.
    if "lm_head.weight" in ix:
        same = ("model.embed_tokens.weight" in ix and
                ix.entries["lm_head.weight"][1:3] == ix.entries["model.embed_tokens.weight"][1:3]
                and np.array_equal(ix.read("lm_head.weight"),
                                   ix.read("model.embed_tokens.weight")))
        if not same:
            raise CheckpointError("A2: lm_head.weight present; expected tied embeddings")

    ew, es, eb = _fp8(ix, "model.embed_tokens.weight", cfg.vocab, H)
    embed = Fp8Weight(_to_device(ew, device), _to_device(es, device), eb)
    ix.require("model.norm.weight", "BF16", (H,))
    out = Qwen3Fp8Weights(cfg, embed, _to_device(ix.read("model.norm.weight"), device))
    for i in range(cfg.n_layers):
        p = f"model.layers.{i}."
        norms = {}
        for key, n, dim in (("attn_norm", "input_layernorm.weight", H),
                            ("q_norm", "self_attn.q_norm.weight", D),
                            ("k_norm", "self_attn.k_norm.weight", D),
                            ("ffn_norm", "post_attention_layernorm.weight", H)):
            ix.require(p + n, "BF16", (dim,))
            norms[key] = _to_device(ix.read(p + n), device)
        qkv = _fused(ix, [p + "self_attn.q_proj.weight", p + "self_attn.k_proj.weight",
                          p + "self_attn.v_proj.weight"], [Q, KV, KV], H, device)
        o = _fused(ix, [p + "self_attn.o_proj.weight"], [H], Q, device)
        gate_up = _fused(ix, [p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight"], [I, I], H,
                         device)
        down = _fused(ix, [p + "mlp.down_proj.weight"], [H], I, device)
        out.layers.append(Qwen3Layer(qkv=qkv, o=o, gate_up=gate_up, down=down, **norms))
    return out
