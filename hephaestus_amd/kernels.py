"""Host-side mirror of the reference's FP8 linear-layer operator API.

The names, argument order and meaning follow the Mojo functions of the
reference engine (src/hephaestus/kernels.mojo), with torch tensors standing
for its TileTensor / DeviceBuffer device memory and an optional torch stream
for its DeviceContext:

  quantize_act_rows_fp8(a_fp8, act_scale, x, m, k, ctx)        kernels.mojo:270-287
  quantize_act_fp8_pad(a_fp8, act_scale, x, k, ctx)            kernels.mojo:196-211
  gemv_fp8(c, a, w, scale, a_fp8_ws, act_scale_ws, n, k, ctx,
           add_residual=False, do_quantize=True)               kernels.mojo:372-407
  linear_fp8(c, a, w, scale, a_fp8_ws, act_scale_ws, m, n, k, ctx,
             do_quantize=True)                                 kernels.mojo:410-470
  linear_add_residual_fp8(residual, a, w, scale, a_fp8_ws,
             act_scale_ws, m, n, k, ctx, do_quantize=True)     kernels.mojo:473-527
  linear(c, a, b, m, n, k, ctx)      bf16 lm_head, f32 logits  kernels.mojo:89-121

Errors raise HephError (the reference's functions `raise`). Every call goes
through the HIP library; there is no CPU or torch fallback.

Scale granularity follows the `scale` tensor's shape:
  [ceil(n/128), ceil(k/128)]  128x128 weight blocks (weight_scale_inv),
                              activations quantized per 1x128 group;
  [n, 1] or [n]               the reference's per-output-channel scale,
                              activations quantized per token (group = k).
`group_k=` overrides the activation group (128 or k).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib as L


class HephError(RuntimeError):
    def __init__(self, status: int, where: str):
        self.status = status
        super().__init__(f"{where}: {L.strerror(status)} (status {status})")


def _check(status: int, where: str) -> None:
    if status != L.HEPH_OK:
        raise HephError(status, where)


def _stream(ctx) -> int:
    if ctx is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(ctx, torch.cuda.Stream):
        return ctx.cuda_stream
    return int(ctx)


def _dev(t: torch.Tensor, name: str, dtypes) -> int:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be in device memory (got {t.device})")
    if t.dtype not in dtypes:
        raise TypeError(f"{name} has dtype {t.dtype}, expected one of {dtypes}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t.data_ptr()


_FP8 = (torch.uint8, torch.float8_e4m3fn)
_OUT = {torch.bfloat16: L.HEPH_DTYPE_BF16, torch.float32: L.HEPH_DTYPE_F32}


def _weight_block(scale: torch.Tensor, n: int, k: int) -> tuple[int, int]:
    """(w_block_n, w_block_k) implied by the scale tensor's shape."""
    if scale.numel() == n and (scale.dim() == 1 or (scale.dim() == 2 and scale.shape[1] == 1)):
        return 1, k
    nb, kb = -(-n // 128), -(-k // 128)
    if scale.dim() == 2 and tuple(scale.shape) == (nb, kb):
        return 128, 128
    raise ValueError(f"scale shape {tuple(scale.shape)} is neither [{n},1] nor [{nb},{kb}]")


def quantize_act_rows_fp8(a_fp8, act_scale, x, m, k, ctx=None, *, group_k=128):
    """x bf16 [m,k] -> a_fp8 codes [m,k] + act_scale [m, k/group_k]."""
    if x.numel() < m * k:
        raise HephError(L.HEPH_ERR_SHAPE, "quantize_act_rows_fp8")
    if a_fp8.numel() < m * k or act_scale.numel() < m * (k // max(group_k, 1)):
        raise HephError(L.HEPH_ERR_WORKSPACE, "quantize_act_rows_fp8")
    s = L.lib().heph_fp8_quant_act(
        _dev(x, "x", (torch.bfloat16,)), _dev(a_fp8, "a_fp8", _FP8),
        _dev(act_scale, "act_scale", (torch.float32,)), m, k, group_k, _stream(ctx))
    _check(s, "quantize_act_rows_fp8")


def quantize_act_fp8_pad(a_fp8, act_scale, x, k, ctx=None, *, group_k=128):
    """The reference's M=1 quantizer. The MFMA kernels mask rows >= M, so
    no zero pad rows are written (the reference writes 15*k of them)."""
    quantize_act_rows_fp8(a_fp8, act_scale, x, 1, k, ctx, group_k=group_k)


def rmsnorm_quant_fp8(a_fp8, act_scale, x, gamma, m, k, eps=1e-6, ctx=None, *, group_k=128):
    """Producer-side quantization for a linear fed by an RMSNorm: codes and
    scales of bf16(gamma * bf16(x * r)) per row of x [m, k] (bit for bit
    rmsnorm then quantize_act_rows_fp8); the linear then runs with
    do_quantize=False on these workspaces."""
    if x.numel() < m * k or gamma.numel() < k:
        raise HephError(L.HEPH_ERR_SHAPE, "rmsnorm_quant_fp8")
    if a_fp8.numel() < m * k or act_scale.numel() < m * (k // max(group_k, 1)):
        raise HephError(L.HEPH_ERR_WORKSPACE, "rmsnorm_quant_fp8")
    s = L.lib().heph_rmsnorm_quant_fp8(
        _dev(a_fp8, "a_fp8", _FP8), _dev(act_scale, "act_scale", (torch.float32,)),
        _dev(x, "x", (torch.bfloat16,)), _dev(gamma, "gamma", (torch.bfloat16,)), m, k,
        float(eps), group_k, _stream(ctx))
    _check(s, "rmsnorm_quant_fp8")


def silu_mul_quant_fp8(a_fp8, act_scale, gate, up, m, n, ld=None, ctx=None, *, group_k=128):
    """Producer-side quantization for a linear fed by SwiGLU: codes and
    scales of bf16(bf16(silu(gate)) * up) per row (row r at gate + r*ld,
    up + r*ld; ld defaults to n), bit for bit silu_mul then
    quantize_act_rows_fp8."""
    ld = n if ld is None else ld
    if a_fp8.numel() < m * n or act_scale.numel() < m * (n // max(group_k, 1)):
        raise HephError(L.HEPH_ERR_WORKSPACE, "silu_mul_quant_fp8")
    s = L.lib().heph_silu_mul_quant_fp8(
        _dev(a_fp8, "a_fp8", _FP8), _dev(act_scale, "act_scale", (torch.float32,)),
        gate.data_ptr(), up.data_ptr(), m, n, ld, group_k, _stream(ctx))
    _check(s, "silu_mul_quant_fp8")


def _overrides(tune):
    """A heph_launch_overrides for the dict `tune` (keys: its field names)."""
    bad = set(tune) - {f for f, _ in L.LaunchOverrides._fields_}
    if bad:
        raise ValueError(f"unknown launch override(s): {sorted(bad)}")
    return L.LaunchOverrides(**{k: int(v) for k, v in tune.items()})


def _linear_fp8(c, a, w, scale, a_fp8_ws, act_scale_ws, m, n, k, ctx, *,
                do_quantize, add_residual, group_k, flags, where, tune=None):
    bn, bk = _weight_block(scale, n, k)
    if group_k is None:
        group_k = 128 if bn == 128 else k
    if c.dtype not in _OUT:
        raise TypeError(f"{where}: output dtype {c.dtype} not supported")
    if c.numel() < m * n or w.numel() < n * k:
        raise HephError(L.HEPH_ERR_SHAPE, where)
    if do_quantize and a.numel() < m * k:
        raise HephError(L.HEPH_ERR_SHAPE, where)
    f = flags
    if add_residual:
        f |= L.FLAG_ADD_RESIDUAL
    if not do_quantize:
        f |= L.FLAG_SKIP_QUANT
    x_ptr = _dev(a, "a", (torch.bfloat16,)) if do_quantize else (a.data_ptr() if a is not None else None)
    args = (_dev(c, "c", tuple(_OUT)), _OUT[c.dtype], x_ptr,
            _dev(w, "w", _FP8), _dev(scale, "scale", (torch.float32,)), bn, bk,
            _dev(a_fp8_ws, "a_fp8_ws", _FP8), a_fp8_ws.numel(),
            _dev(act_scale_ws, "act_scale_ws", (torch.float32,)), act_scale_ws.numel(),
            m, n, k, group_k, f, _stream(ctx))
    if tune:
        s = L.lib().heph_fp8_linear_with(*args, ctypes.byref(_overrides(tune)))
    else:
        s = L.lib().heph_fp8_linear(*args)
    _check(s, where)


def linear_fp8_rmsnorm(c, x, gamma, eps, w, scale, a_fp8_ws, act_scale_ws, n, k, ctx=None, *,
                       add_residual=False):
    """c = rmsnorm(x, gamma, eps) @ dequant(w)^T for one row (M = 1), the
    norm computed inside the fused GEMV (bit for bit rmsnorm then linear_fp8
    with the norm form's launch shape, norm_shape_tune); the workspaces
    receive the normalized row's codes and scales."""
    bn, bk = _weight_block(scale, n, k)
    if c.dtype not in _OUT:
        raise TypeError(f"linear_fp8_rmsnorm: output dtype {c.dtype} not supported")
    if c.numel() < n or w.numel() < n * k or x.numel() < k or gamma.numel() < k:
        raise HephError(L.HEPH_ERR_SHAPE, "linear_fp8_rmsnorm")
    s = L.lib().heph_fp8_linear_rmsnorm(
        _dev(c, "c", tuple(_OUT)), _OUT[c.dtype], _dev(x, "x", (torch.bfloat16,)),
        _dev(gamma, "gamma", (torch.bfloat16,)), float(eps),
        _dev(w, "w", _FP8), _dev(scale, "scale", (torch.float32,)), bn, bk,
        _dev(a_fp8_ws, "a_fp8_ws", _FP8), a_fp8_ws.numel(),
        _dev(act_scale_ws, "act_scale_ws", (torch.float32,)), act_scale_ws.numel(),
        n, k, L.FLAG_ADD_RESIDUAL if add_residual else 0, _stream(ctx))
    _check(s, "linear_fp8_rmsnorm")


def norm_shape_tune(n: int, k: int) -> dict:
    """Launch-shape overrides under which linear_fp8 at M = 1 sums in the
    order of the RMSNorm-fused forms (linear_fp8_rmsnorm, linear_fp8_swiglu
    with gamma), as include/hephfp8.h states their shape: the fewest K-chunk
    slots (<= 8) giving >= 256 workgroups of 16 / slots columns, 4 waves up
    to 3 chunk steps, else 8, two-step batches when each wave has two."""
    tiles, kc = n // 16, k // 128
    ks = 1
    while ks < 8 and tiles * ks < 256:
        ks *= 2
    steps = -(-kc // ks)
    waves = 4 if steps <= 3 else 8
    return {"gemv_ks": ks, "gemv_waves": waves, "gemv_u": 2 if -(-steps // waves) == 2 else 1}


def linear_fp8_swiglu(act, x, gamma, eps, w, scale, a_fp8_ws, act_scale_ws, n, k, ctx=None):
    """act = silu(g) * u for one row (M = 1), with g and u the gate and up
    halves of x @ dequant(w)^T (w: gate rows, then up rows; n = 2 *
    intermediate) and x first RMS-normalized with gamma unless gamma is
    None; bit for bit the gate/up linear (linear_fp8_rmsnorm with gamma,
    linear_fp8 without) then silu_mul (bf16 act, n / 2)."""
    bn, bk = _weight_block(scale, n, k)
    if act.dtype != torch.bfloat16:
        raise TypeError(f"linear_fp8_swiglu: output dtype {act.dtype} not supported")
    if act.numel() < n // 2 or w.numel() < n * k or x.numel() < k or \
            (gamma is not None and gamma.numel() < k):
        raise HephError(L.HEPH_ERR_SHAPE, "linear_fp8_swiglu")
    g = _dev(gamma, "gamma", (torch.bfloat16,)) if gamma is not None else None
    s = L.lib().heph_fp8_linear_swiglu(
        _dev(act, "act", (torch.bfloat16,)), _dev(x, "x", (torch.bfloat16,)), g, float(eps),
        _dev(w, "w", _FP8), _dev(scale, "scale", (torch.float32,)), bn, bk,
        _dev(a_fp8_ws, "a_fp8_ws", _FP8), a_fp8_ws.numel(),
        _dev(act_scale_ws, "act_scale_ws", (torch.float32,)), act_scale_ws.numel(),
        n, k, _stream(ctx))
    _check(s, "linear_fp8_swiglu")


def linear_fp8(c, a, w, scale, a_fp8_ws, act_scale_ws, m, n, k, ctx=None, *,
               do_quantize=True, group_k=None, flags=0, tune=None):
    """C = A @ W^T through the W8A8 FP8 path (quantize A, FP8 contraction,
    scale epilogue). M <= 32 runs the weight-streaming kernels, larger M the
    MFMA GEMM. `tune` (measurement and tests): launch-shape overrides of this
    call, a dict over the fields of heph_launch_overrides."""
    _linear_fp8(c, a, w, scale, a_fp8_ws, act_scale_ws, m, n, k, ctx,
                do_quantize=do_quantize, add_residual=False, group_k=group_k,
                flags=flags, where="linear_fp8", tune=tune)


def linear_add_residual_fp8(residual, a, w, scale, a_fp8_ws, act_scale_ws, m, n, k,
                            ctx=None, *, do_quantize=True, group_k=None, flags=0, tune=None):
    """residual += A @ W^T (f32 add of the bf16 residual, then the cast)."""
    _linear_fp8(residual, a, w, scale, a_fp8_ws, act_scale_ws, m, n, k, ctx,
                do_quantize=do_quantize, add_residual=True, group_k=group_k,
                flags=flags, where="linear_add_residual_fp8", tune=tune)


def gemv_fp8(c, a, w, scale, a_fp8_ws, act_scale_ws, n, k, ctx=None, *,
             add_residual=False, do_quantize=True, group_k=None):
    """The M = 1 decode form of linear_fp8."""
    _linear_fp8(c, a, w, scale, a_fp8_ws, act_scale_ws, 1, n, k, ctx,
                do_quantize=do_quantize, add_residual=add_residual, group_k=group_k,
                flags=0, where="gemv_fp8")


def linear(c, a, b, m, n, k, ctx=None, *, add_residual=False):
    """bf16 C = A @ B^T with f32 accumulation (the lm_head); c is f32
    (logits, as the reference keeps them) or bf16. M <= 32 streams the
    weights; larger M runs the MFMA GEMM."""
    if c.dtype not in _OUT:
        raise TypeError(f"linear: output dtype {c.dtype} not supported")
    if c.numel() < m * n or a.numel() < m * k or b.numel() < n * k:
        raise HephError(L.HEPH_ERR_SHAPE, "linear")
    s = L.lib().heph_bf16_linear(
        _dev(c, "c", tuple(_OUT)), _OUT[c.dtype], _dev(a, "a", (torch.bfloat16,)),
        _dev(b, "b", (torch.bfloat16,)), m, n, k,
        L.FLAG_ADD_RESIDUAL if add_residual else 0, _stream(ctx))
    _check(s, "linear")


def workspace(m: int, k: int, device="cuda", group_k: int = 128, n: int | None = None):
    """Allocate (a_fp8_ws, act_scale_ws) for up to m rows of width k. With
    n, a_fp8_ws also holds the scratch the large-M GEMM splits K into for
    an m x n output (heph_fp8_linear_ws_bytes)."""
    qb = (L.lib().heph_fp8_linear_ws_bytes(m, n, k) if n is not None
          else L.lib().heph_fp8_q_ws_bytes(m, k))
    q = torch.empty(qb, dtype=torch.uint8, device=device)
    s = torch.empty(L.lib().heph_fp8_s_ws_floats(m, k, group_k), dtype=torch.float32,
                    device=device)
    return q, s


def last_kernel() -> str:
    """Name of the main kernel the last call on this thread launched."""
    return L.lib().heph_last_kernel().decode()
