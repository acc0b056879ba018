"""Helpers shared by the GPU parity tests (not collected by pytest)."""
from __future__ import annotations

import numpy as np
import torch

from hephaestus_amd import kernels as HK
from oracle import oracle as O


def dev(a: np.ndarray) -> torch.Tensor:
    """numpy -> CUDA tensor; uint16 arrays become bfloat16 (bit patterns)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
    return torch.from_numpy(a).cuda()


def host_bf16(t: torch.Tensor) -> np.ndarray:
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def smoke_codes(n: int, seed: int) -> np.ndarray:
    """((i*17 + seed*31) % 17 - 8) * 0.25, exact in E4M3
    (reference src/qwen_small_m_gemm_smoke.mojo:26-31)."""
    i = np.arange(n, dtype=np.int64)
    return O.e4m3_encode((((i * 17 + seed * 31) % 17) - 8).astype(np.float32) * 0.25)


def smoke_ints(n: int, seed: int) -> np.ndarray:
    i = np.arange(n, dtype=np.int64)
    return ((i * 17 + seed * 31) % 17) - 8


# Launch-shape overrides that run_linear passes to every call it makes
# (heph_launch_overrides fields; the library itself keeps no such state).
TUNE: dict = {}


def split_ws(codes: torch.Tensor, M: int, N: int, K: int, splits: int) -> torch.Tensor:
    """A q_ws holding `codes` (M*K bytes) and room for `splits` fp32 K-split
    partials of an M x N output past the next 256-byte boundary."""
    q = torch.zeros(((M * K + 255) // 256) * 256 + splits * M * N * 4, dtype=torch.uint8,
                    device="cuda")
    q[: M * K] = codes.reshape(-1)[: M * K]
    return q


def run_linear(qw, sw, x=None, *, M, N, K, group_k=128, out=torch.bfloat16, flags=0,
               q_ws=None, s_ws=None, residual=None, skip_quant=False, tune=None):
    """Call linear_fp8 (or the residual form) on device copies; returns
    (output tensor, q_ws, s_ws). tune (or TUNE): launch-shape overrides."""
    tune = {**TUNE, **(tune or {})} or None
    w_t = dev(qw)
    sw_t = dev(np.ascontiguousarray(sw, np.float32))
    if q_ws is None:
        q_ws = torch.zeros(M * K, dtype=torch.uint8, device="cuda")
        s_ws = torch.zeros(M * (K // group_k), dtype=torch.float32, device="cuda")
    x_t = dev(x) if x is not None else None
    if residual is not None:
        c = residual.clone()
        HK.linear_add_residual_fp8(c, x_t, w_t, sw_t, q_ws, s_ws, M, N, K,
                                   do_quantize=not skip_quant, group_k=group_k, flags=flags,
                                   tune=tune)
    else:
        c = torch.zeros(M, N, dtype=out, device="cuda")
        HK.linear_fp8(c, x_t, w_t, sw_t, q_ws, s_ws, M, N, K,
                      do_quantize=not skip_quant, group_k=group_k, flags=flags, tune=tune)
    torch.cuda.synchronize()
    return c, q_ws, s_ws


def max_abs_rel(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / max |ref| (the north star's max-abs-rel)."""
    return float(np.abs(got.astype(np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def bf16_of(x: np.ndarray) -> np.ndarray:
    return O.f32_to_bf16(np.ascontiguousarray(x, np.float32))


def f32_of_bf16(b: np.ndarray) -> np.ndarray:
    return O.bf16_to_f32(b)
