"""ctypes + numpy front end of the C oracle (heph_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker or the CPU baseline and
never as the measured product path.

Function-to-reference map (paths relative to the reference tree):
  e4m3_encode / e4m3_decode  OCP E4M3FN, the FP8 type of
                             src/hephaestus/wmma_gfx12.mojo:631-633
  quant_act                  src/hephaestus/kernels.mojo:151-186 per group
  quant_weight               scripts/stage_tiny_fp8_from_bf16.py:59-71 per block
  linear / linear_f64        experiments/exp4b_wmma_gemm/oracle.py:113-126
  bf16_linear                src/hephaestus/kernels.mojo:89-121 (f32 logits)
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libheph_oracle.so")

_lib = None

_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc); returns the .so path."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.heph_oracle_e4m3_decode.restype = ctypes.c_float
        L.heph_oracle_e4m3_decode.argtypes = [ctypes.c_uint8]
        L.heph_oracle_e4m3_encode.restype = ctypes.c_uint8
        L.heph_oracle_e4m3_encode.argtypes = [ctypes.c_float]
        L.heph_oracle_e4m3_encode_array.argtypes = [_f32p, _u8p, ctypes.c_size_t]
        L.heph_oracle_e4m3_decode_array.argtypes = [_u8p, _f32p, ctypes.c_size_t]
        L.heph_oracle_f32_to_bf16_array.argtypes = [_f32p, _u16p, ctypes.c_size_t]
        L.heph_oracle_bf16_to_f32_array.argtypes = [_u16p, _f32p, ctypes.c_size_t]
        L.heph_oracle_quant_act.argtypes = [_u16p, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, _u8p, _f32p]
        L.heph_oracle_quant_weight.argtypes = [_f32p, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_int, ctypes.c_int, _u8p, _f32p]
        lin_args = [_u8p, _f32p, ctypes.c_int, _u8p, _f32p, ctypes.c_int,
                    ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.heph_oracle_linear.argtypes = lin_args + [_f32p, ctypes.c_int]
        L.heph_oracle_linear_f64.argtypes = lin_args + [_f64p, ctypes.c_int]
        L.heph_oracle_quant_linear.argtypes = [
            _u16p, ctypes.c_int, _u8p, _f32p, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, _u8p, _f32p, _f32p,
            ctypes.c_int]
        L.heph_oracle_bf16_linear.argtypes = [_u16p, _u16p, ctypes.c_int,
                                              ctypes.c_int, ctypes.c_int, _f32p,
                                              ctypes.c_int]
        L.heph_oracle_gen_normal.argtypes = [ctypes.c_uint64, ctypes.c_uint64,
                                             ctypes.c_size_t, ctypes.c_float,
                                             ctypes.c_float, _f32p]
        L.heph_oracle_gen_uniform.argtypes = [ctypes.c_uint64, ctypes.c_uint64,
                                              ctypes.c_size_t, _f64p]
        L.heph_oracle_gen_act_bf16.argtypes = [ctypes.c_uint64, ctypes.c_size_t,
                                               ctypes.c_double, ctypes.c_float, _u16p]
        L.heph_oracle_fnv1a64.restype = ctypes.c_uint64
        L.heph_oracle_fnv1a64.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
        L.heph_oracle_num_threads.restype = ctypes.c_int
        _i32p = ctypes.POINTER(ctypes.c_int32)
        L.heph_oracle_embed_fp8.argtypes = [_u16p, _u8p, _f32p, ctypes.c_int, _i32p,
                                            ctypes.c_int, ctypes.c_int]
        L.heph_oracle_rmsnorm.argtypes = [_u16p, _u16p, _u16p, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_float]
        L.heph_oracle_rope_cs.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_double, _f32p, _f32p]
        L.heph_oracle_qk_norm_rope_kv.argtypes = [_u16p, _u16p, _u16p, _u8p, _u8p, _f32p,
                                                  ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                  ctypes.c_double, ctypes.c_float]
        L.heph_oracle_attention_fp8kv.argtypes = [_u16p, _u16p, _u8p, _u8p, _f32p,
                                                  ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.heph_oracle_attention_fp8kv.restype = ctypes.c_int
        L.heph_oracle_silu_mul.argtypes = [_u16p, _u16p, _u16p, ctypes.c_size_t]
        L.heph_oracle_argmax_bf16.argtypes = [_f32p, ctypes.c_size_t]
        L.heph_oracle_argmax_bf16.restype = ctypes.c_int
        for name in ("heph_oracle_quant_act", "heph_oracle_quant_weight",
                     "heph_oracle_linear", "heph_oracle_linear_f64",
                     "heph_oracle_quant_linear", "heph_oracle_bf16_linear"):
            getattr(L, name).restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    assert a.flags["C_CONTIGUOUS"], "oracle needs C-contiguous arrays"
    return a.ctypes.data_as(t)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what} rejected its arguments (rc={rc})")


# ---- codecs ----------------------------------------------------------------

def e4m3_decode_table() -> np.ndarray:
    """f32 value of every E4M3FN code 0..255."""
    return np.array([lib().heph_oracle_e4m3_decode(c) for c in range(256)],
                    dtype=np.float32)


def e4m3_encode(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.shape, dtype=np.uint8)
    lib().heph_oracle_e4m3_encode_array(_p(x, _f32p), _p(q, _u8p), x.size)
    return q


def e4m3_decode(q) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    x = np.empty(q.shape, dtype=np.float32)
    lib().heph_oracle_e4m3_decode_array(_p(q, _u8p), _p(x, _f32p), q.size)
    return x


def f32_to_bf16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = np.empty(x.shape, dtype=np.uint16)
    lib().heph_oracle_f32_to_bf16_array(_p(x, _f32p), _p(b, _u16p), x.size)
    return b


def bf16_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


# ---- quantizers ------------------------------------------------------------

def quant_act(x_bf16: np.ndarray, group_k: int):
    """bf16 bits [M,K] -> (codes u8 [M,K], scales f32 [M, K/group_k])."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    M, K = x.shape
    q = np.empty((M, K), dtype=np.uint8)
    s = np.empty((M, K // group_k), dtype=np.float32)
    _check(lib().heph_oracle_quant_act(_p(x, _u16p), M, K, group_k,
                                       _p(q, _u8p), _p(s, _f32p)), "quant_act")
    return q, s


def quant_weight(w: np.ndarray, bn: int = 128, bk: int = 128):
    """f32 [N,K] -> (codes u8 [N,K], scale_inv f32 [ceil(N/bn), ceil(K/bk)])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    q = np.empty((N, K), dtype=np.uint8)
    s = np.empty(((N + bn - 1) // bn, (K + bk - 1) // bk), dtype=np.float32)
    _check(lib().heph_oracle_quant_weight(_p(w, _f32p), N, K, bn, bk,
                                          _p(q, _u8p), _p(s, _f32p)), "quant_weight")
    return q, s


# ---- matmuls ---------------------------------------------------------------

def linear(qa, sa, qw, sw, *, bn=128, bk=128, nthreads=0) -> np.ndarray:
    """f32-accumulated dequant-matmul; returns f32 [M,N]."""
    qa = np.ascontiguousarray(qa, np.uint8)
    sa = np.ascontiguousarray(sa, np.float32)
    qw = np.ascontiguousarray(qw, np.uint8)
    sw = np.ascontiguousarray(sw, np.float32)
    M, K = qa.shape
    N = qw.shape[0]
    group_k = K // sa.shape[1]
    out = np.empty((M, N), dtype=np.float32)
    _check(lib().heph_oracle_linear(_p(qa, _u8p), _p(sa, _f32p), group_k,
                                    _p(qw, _u8p), _p(sw, _f32p), bn, bk, M, N, K,
                                    _p(out, _f32p), nthreads), "linear")
    return out


def linear_f64(qa, sa, qw, sw, *, bn=128, bk=128, nthreads=0) -> np.ndarray:
    qa = np.ascontiguousarray(qa, np.uint8)
    sa = np.ascontiguousarray(sa, np.float32)
    qw = np.ascontiguousarray(qw, np.uint8)
    sw = np.ascontiguousarray(sw, np.float32)
    M, K = qa.shape
    N = qw.shape[0]
    group_k = K // sa.shape[1]
    out = np.empty((M, N), dtype=np.float64)
    _check(lib().heph_oracle_linear_f64(_p(qa, _u8p), _p(sa, _f32p), group_k,
                                        _p(qw, _u8p), _p(sw, _f32p), bn, bk, M, N, K,
                                        _p(out, _f64p), nthreads), "linear_f64")
    return out


def quant_linear(x_bf16, qw, sw, *, group_k=128, bn=128, bk=128, nthreads=0):
    """The whole CPU path: quantize the activation, then dequant-matmul."""
    x = np.ascontiguousarray(x_bf16, np.uint16)
    qw = np.ascontiguousarray(qw, np.uint8)
    sw = np.ascontiguousarray(sw, np.float32)
    M, K = x.shape
    N = qw.shape[0]
    q = np.empty((M, K), np.uint8)
    s = np.empty((M, K // group_k), np.float32)
    out = np.empty((M, N), np.float32)
    _check(lib().heph_oracle_quant_linear(_p(x, _u16p), group_k, _p(qw, _u8p),
                                          _p(sw, _f32p), bn, bk, M, N, K,
                                          _p(q, _u8p), _p(s, _f32p), _p(out, _f32p),
                                          nthreads), "quant_linear")
    return out


def bf16_linear(x_bf16, w_bf16, *, nthreads=0) -> np.ndarray:
    x = np.ascontiguousarray(x_bf16, np.uint16)
    w = np.ascontiguousarray(w_bf16, np.uint16)
    M, K = x.shape
    N = w.shape[0]
    out = np.empty((M, N), np.float32)
    _check(lib().heph_oracle_bf16_linear(_p(x, _u16p), _p(w, _u16p), M, N, K,
                                         _p(out, _f32p), nthreads), "bf16_linear")
    return out


# ---- synthetic inputs ------------------------------------------------------

def gen_normal(seed: int, n: int, mean=0.0, std=1.0, offset=0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().heph_oracle_gen_normal(seed, offset, n, mean, std, _p(out, _f32p))
    return out


def gen_uniform(seed: int, n: int, offset=0) -> np.ndarray:
    out = np.empty(n, dtype=np.float64)
    lib().heph_oracle_gen_uniform(seed, offset, n, _p(out, _f64p))
    return out


def gen_act_bf16(seed: int, M: int, K: int, outlier_p=0.0, outlier_mul=50.0):
    out = np.empty((M, K), dtype=np.uint16)
    lib().heph_oracle_gen_act_bf16(seed, M * K, outlier_p, outlier_mul, _p(out, _u16p))
    return out


def gen_weight(seed: int, N: int, K: int, std=0.02, bn=128, bk=128):
    """W ~ N(0, std) quantized per bn x bk block -> (codes, scale_inv)."""
    w = gen_normal(seed, N * K, 0.0, std).reshape(N, K)
    return quant_weight(w, bn, bk)


def digest(a: np.ndarray) -> str:
    a = np.ascontiguousarray(a)
    return "%016x" % lib().heph_oracle_fnv1a64(a.ctypes.data, a.nbytes)


def num_threads() -> int:
    return lib().heph_oracle_num_threads()


# ---- one Qwen3 decode step (heph_decode_oracle.c) ---------------------------

_i32p = ctypes.POINTER(ctypes.c_int32)


def embed_fp8(emb: np.ndarray, scale: np.ndarray, block: bool, tokens) -> np.ndarray:
    """bf16 rows bf16(scale * e4m3(emb[token])) (kernels.mojo:530-548)."""
    tokens = np.ascontiguousarray(tokens, np.int32)
    emb = np.ascontiguousarray(emb, np.uint8)
    scale = np.ascontiguousarray(scale, np.float32)
    H = emb.shape[1]
    x = np.empty((tokens.size, H), np.uint16)
    lib().heph_oracle_embed_fp8(_p(x, _u16p), _p(emb, _u8p), _p(scale, _f32p), int(block),
                                _p(tokens, _i32p), tokens.size, H)
    return x


def rmsnorm(x: np.ndarray, gamma: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """bf16(gamma * bf16(x / sqrt(mean(x^2) + eps))) per row (bf16 in/out)."""
    x = np.ascontiguousarray(x, np.uint16)
    g = np.ascontiguousarray(gamma, np.uint16)
    rows, cols = (1, x.size) if x.ndim == 1 else x.shape
    out = np.empty_like(x)
    lib().heph_oracle_rmsnorm(_p(out, _u16p), _p(x, _u16p), _p(g, _u16p), rows, cols, eps)
    return out


def rope_cs(pos: int, p: int, D: int = 128, theta: float = 1e6):
    c, s = ctypes.c_float(), ctypes.c_float()
    lib().heph_oracle_rope_cs(pos, p, D, theta, ctypes.byref(c), ctypes.byref(s))
    return c.value, s.value


def qk_norm_rope_kv(qkv: np.ndarray, q_gamma, k_gamma, kv_inv, n_heads: int, n_kv: int,
                    pos: int, theta: float = 1e6, eps: float = 1e-6):
    """(q bf16 [n_heads*128] normalized and rotated, k codes, v codes)."""
    qkv = np.array(qkv, dtype=np.uint16, copy=True).reshape(-1)
    qg = np.ascontiguousarray(q_gamma, np.uint16)
    kg = np.ascontiguousarray(k_gamma, np.uint16)
    inv = np.ascontiguousarray(kv_inv, np.float32)
    k = np.empty(n_kv * 128, np.uint8)
    v = np.empty(n_kv * 128, np.uint8)
    lib().heph_oracle_qk_norm_rope_kv(_p(qkv, _u16p), _p(qg, _u16p), _p(kg, _u16p),
                                      _p(k, _u8p), _p(v, _u8p), _p(inv, _f32p), n_heads, n_kv,
                                      pos, theta, eps)
    return qkv[:n_heads * 128].copy(), k, v


def attention_fp8kv(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, kv_scale, n_heads: int,
                    n_kv: int, n_keys: int) -> np.ndarray:
    """bf16 [n_heads*128]; kc / vc: E4M3 codes [>= n_keys, n_kv, 128]."""
    q = np.ascontiguousarray(q, np.uint16)
    kc = np.ascontiguousarray(kc, np.uint8)
    vc = np.ascontiguousarray(vc, np.uint8)
    sc = np.ascontiguousarray(kv_scale, np.float32)
    out = np.empty(n_heads * 128, np.uint16)
    _check(lib().heph_oracle_attention_fp8kv(_p(out, _u16p), _p(q, _u16p), _p(kc, _u8p),
                                             _p(vc, _u8p), _p(sc, _f32p), n_heads, n_kv,
                                             n_keys), "attention_fp8kv")
    return out


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(gate, np.uint16)
    u = np.ascontiguousarray(up, np.uint16)
    out = np.empty_like(g)
    lib().heph_oracle_silu_mul(_p(out, _u16p), _p(g, _u16p), _p(u, _u16p), g.size)
    return out


def argmax_bf16(logits: np.ndarray) -> int:
    x = np.ascontiguousarray(logits, np.float32)
    return int(lib().heph_oracle_argmax_bf16(_p(x, _f32p), x.size))


def _linear_bf16(x_bf16, qw, sw, residual=None, nthreads=0):
    """bf16 output of the FP8 linear (block 128 scales), optionally + residual
    in f32 before the cast (wmma_gfx12.mojo:712-715)."""
    acc = quant_linear(np.ascontiguousarray(x_bf16, np.uint16).reshape(1, -1), qw, sw,
                       nthreads=nthreads)[0]
    if residual is not None:
        acc = acc + bf16_to_f32(np.ascontiguousarray(residual, np.uint16))
    return f32_to_bf16(acc.astype(np.float32))


def decode_step(model: dict, kv: dict, token: int, pos: int, nthreads: int = 0):
    """One W8A8 decode step of a Qwen3 model on the CPU (forward.mojo:359-615
    with 128x128 block scales and an E4M3 KV cache). model: host arrays
    (see hephaestus_amd.decode.Qwen3Decoder.host_model); kv: {"k", "v": codes
    [L, ctx, n_kv, 128], "scale": f32 [L, 2*n_kv], "inv": f32 [L, 2*n_kv]},
    updated in place at row `pos`. Returns (f32 logits, argmax)."""
    cfg = model["cfg"]
    H, NH, NKV, D = cfg["hidden"], cfg["n_heads"], cfg["n_kv_heads"], 128
    Q, KV, I = NH * D, NKV * D, cfg["inter"]
    eps, theta = cfg["eps"], cfg["theta"]
    x = embed_fp8(model["embed"], model["embed_scale"], True, [token])[0]
    for li, L in enumerate(model["layers"]):
        xn = rmsnorm(x, L["attn_norm"], eps)
        qkv = _linear_bf16(xn, L["qkv"], L["qkv_scale"], nthreads=nthreads)
        q, k, v = qk_norm_rope_kv(qkv, L["q_norm"], L["k_norm"], kv["inv"][li], NH, NKV, pos,
                                  theta, eps)
        kv["k"][li, pos] = k.reshape(NKV, D)
        kv["v"][li, pos] = v.reshape(NKV, D)
        att = attention_fp8kv(q, kv["k"][li], kv["v"][li], kv["scale"][li], NH, NKV, pos + 1)
        x = _linear_bf16(att, L["o"], L["o_scale"], residual=x, nthreads=nthreads)
        xn = rmsnorm(x, L["ffn_norm"], eps)
        gu = _linear_bf16(xn, L["gate_up"], L["gate_up_scale"], nthreads=nthreads)
        act = silu_mul(gu[:I], gu[I:])
        x = _linear_bf16(act, L["down"], L["down_scale"], residual=x, nthreads=nthreads)
    xn = rmsnorm(x, model["final_norm"], eps)
    logits = quant_linear(xn.reshape(1, -1), model["embed"], model["embed_scale"],
                          nthreads=nthreads)[0]
    return logits, argmax_bf16(logits)
