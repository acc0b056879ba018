"""hephaestus_amd - MI355X (gfx950) W8A8 FP8 linear-layer path.

A C-ABI HIP library (libhephfp8.so, include/hephfp8.h) and a Python mirror
of the reference engine's FP8 linear operator API (hephaestus_amd.kernels).
"""
from .kernels import (  # noqa: F401
    HephError,
    gemv_fp8,
    last_kernel,
    linear,
    linear_add_residual_fp8,
    linear_fp8,
    quantize_act_fp8_pad,
    quantize_act_rows_fp8,
    workspace,
)

__all__ = [
    "HephError", "gemv_fp8", "last_kernel", "linear", "linear_add_residual_fp8",
    "linear_fp8", "quantize_act_fp8_pad", "quantize_act_rows_fp8", "workspace",
]
