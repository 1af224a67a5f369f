"""Per-channel symmetric W8A16 quantizer and dequantizer (torch).

Same contract as the reference's converter helpers
(python/rpu_backend/quant/_common.py:10-41): int8 storage plus one fp16 scale
per output channel, computed as

    w16   = fp16(w)                                  # cast before amax (:28)
    amax  = max_k |f32(w16)|                         # (:29)
    scale = max(fp16(amax / qmax), fp16 tiny 2**-14) # (:30)
    q     = clamp(round_half_even(f32(w16) / f32(scale)), qmin, qmax)   # (:31-35)

These run on whatever device the tensor lives on (division and rounding are
IEEE-exact, so CPU and GPU results are bit-identical).
"""
from __future__ import annotations

import torch

_FP16_TINY = torch.finfo(torch.float16).tiny


def quantize_linear_per_channel(weight: torch.Tensor, *, bits: int = 8
                                ) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize a Linear weight [N, K] to int8 storage plus a per-row fp16 scale.

    ``bits=4`` stores signed 4-bit values in int8 containers (the reference's
    fake-W4 probe format); nibbles are not packed.
    """
    if weight.dim() != 2:
        raise ValueError(f"expected 2-D Linear weight, got {tuple(weight.shape)}")
    if bits not in (4, 8):
        raise ValueError(f"expected bits to be 4 or 8, got {bits}")
    qmax = (1 << (bits - 1)) - 1
    qmin = -(1 << (bits - 1))
    w32 = weight.detach().to(torch.float16).to(torch.float32)
    amax = w32.abs().amax(dim=1)
    scale = (amax / float(qmax)).to(torch.float16).clamp_min(_FP16_TINY)
    q = torch.round(w32 / scale.to(torch.float32).unsqueeze(1)).clamp_(qmin, qmax).to(torch.int8)
    return q, scale


def dequantize_linear_per_channel(w_int8: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """fp16(scale)[:, None] * fp16(q), i.e. RN_fp16(s*q) elementwise."""
    return scale.to(torch.float16).unsqueeze(1) * w_int8.to(torch.float16)
