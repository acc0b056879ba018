"""Weight-format helpers: the weight / weight_scale_inv layout on the GPU.

quantize_weight_fp8 turns a bf16 [N, K] weight into E4M3 codes [N, K] and
f32 scale_inv [ceil(N/128), K/128] with the HIP block quantizer
(heph_fp8_quant_weight). The arithmetic follows the reference's offline
quantizer (scripts/stage_tiny_fp8_from_bf16.py:59-71) per 128x128 block.
"""
from __future__ import annotations

import torch

from . import _lib as L
from .kernels import HephError, _dev, _stream


def quantize_weight_fp8(w: torch.Tensor, ctx=None):
    """bf16 [N, K] device tensor -> (codes uint8 [N, K], scale_inv f32)."""
    if w.dim() != 2:
        raise ValueError("weight must be 2-D [N, K]")
    N, K = w.shape
    q = torch.empty((N, K), dtype=torch.uint8, device=w.device)
    s = torch.empty((-(-N // 128), -(-K // 128)), dtype=torch.float32, device=w.device)
    st = L.lib().heph_fp8_quant_weight(_dev(w, "w", (torch.bfloat16,)), q.data_ptr(),
                                       s.data_ptr(), N, K, _stream(ctx))
    if st != L.HEPH_OK:
        raise HephError(st, "quantize_weight_fp8")
    return q, s
