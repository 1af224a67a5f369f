"""Symmetric per-output-channel quantizer for W8A16 checkpoints (torch).

Byte-identical to what the reference's converters write
(python/rpu_backend/quant/_common.py:10-41), so a checkpoint converted here
loads there and vice versa.  For a weight row ``w`` and ``L = 2**(bits-1)``:

    w16   = fp16(w)                              the row is cast first
    amax  = max |f32(w16)|
    scale = max(fp16(amax / (L - 1)), 2**-14)    fp16, never below fp16 tiny
    q     = clamp(rint(f32(w16) / f32(scale)), -L, L - 1)     ties to even

Division and rounding are correctly rounded IEEE operations, so the CPU and a
HIP device produce the same bytes.  The int4 quantizers in ``int4`` reuse the
scale and rounding steps below.
"""
from __future__ import annotations

import torch

_FP16_TINY = torch.finfo(torch.float16).tiny   # 2**-14, the smallest normal fp16


def signed_levels(bits: int) -> tuple[int, int]:
    """(lowest, highest) integer a ``bits``-wide two's-complement value takes;
    4- and 8-bit values are supported, both kept in int8 containers."""
    if bits not in (4, 8):
        raise ValueError(f"bits={bits}: values are 4 or 8 bits wide (stored in int8)")
    half = 1 << (bits - 1)
    return -half, half - 1


def scale_from_amax(amax: torch.Tensor, top: int) -> torch.Tensor:
    """fp16 step that maps ``amax`` (fp32) onto level ``top``, floored at fp16 tiny."""
    return (amax / float(top)).to(torch.float16).clamp_min(_FP16_TINY)


def round_to_levels(w32: torch.Tensor, step16: torch.Tensor, lo: int, hi: int) -> torch.Tensor:
    """int8 ``clamp(rint(w32 / f32(step16)), lo, hi)``; ``step16`` broadcasts against ``w32``."""
    return torch.round(w32 / step16.to(torch.float32)).clamp_(lo, hi).to(torch.int8)


def _as_matrix(weight: torch.Tensor) -> torch.Tensor:
    if weight.dim() != 2:
        raise ValueError(f"a linear weight is a 2-D [out_features, in_features] matrix; "
                         f"this one has shape {tuple(weight.shape)}")
    return weight.detach()


def quantize_linear_per_channel(weight: torch.Tensor, *, bits: int = 8
                                ) -> tuple[torch.Tensor, torch.Tensor]:
    """[N, K] floating weight -> (int8 [N, K] values, fp16 [N] step per row).

    With ``bits=4`` the values lie in [-8, 7] but are still one per int8 (the
    reference's fake-W4 checkpoint form); nothing is packed into nibbles.
    """
    lo, hi = signed_levels(bits)
    w32 = _as_matrix(weight).to(torch.float16).to(torch.float32)
    step = scale_from_amax(w32.abs().amax(dim=1), hi)
    return round_to_levels(w32, step.unsqueeze(1), lo, hi), step


def dequantize_linear_per_channel(w_int8: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """fp16 [N, K] weight ``RN_fp16(scale[n] * q[n, k])`` (one fp16 multiply)."""
    return scale.to(torch.float16).unsqueeze(1) * w_int8.to(torch.float16)
