"""rhinoforge_amd -- RhinoForge's W8A16 quantized linear, MI355X-native.

``y = x . (s (.) q)^T (+ b)`` with int8 per-output-channel weights ``q``,
an fp16 scale ``s`` per channel and fp16 activations, on hand-written gfx950
HIP kernels behind a C ABI (``include/w8a16.h``) and a thin torch-library op
(``torch.ops.w8a16.*``).

Importing the package loads ``lib/librf_w8a16_torch.so`` (which links
``lib/librf_w8a16.so``).  If the libraries are missing the import fails
loudly: there is no CPU or pure-PyTorch fallback for the compute path.
Build them with ``python rhinoforge_amd/_build.py``.
"""
from __future__ import annotations

from pathlib import Path

import torch

_LIBDIR = Path(__file__).resolve().parent / "lib"
TORCH_OP_LIBRARY = _LIBDIR / "librf_w8a16_torch.so"
CAPI_LIBRARY = _LIBDIR / "librf_w8a16.so"

if not TORCH_OP_LIBRARY.is_file() or not CAPI_LIBRARY.is_file():
    raise ImportError(
        f"rhinoforge_amd native libraries not built ({TORCH_OP_LIBRARY.name}, "
        f"{CAPI_LIBRARY.name} missing under {_LIBDIR}); run "
        "`python rhinoforge_amd/_build.py` (or __graft_entry__.build())"
    )
torch.ops.load_library(str(TORCH_OP_LIBRARY))

from .ops import (  # noqa: E402
    LAYOUT_ROWMAJOR,
    LAYOUT_TILE16X64,
    KERNEL_AUTO,
    KERNEL_GEMM,
    KERNEL_GEMV,
    LAYOUT_TILE16X128_I4,
    linear,
    linear_argmax,
    linear_into,
    linear_multi,
    linear_multi_w4a16,
    linear_w4a16,
    pack_weight,
    pack_weight_int4,
    packed_shape,
    packed_shape_int4,
    select_kernel,
    unpack_weight,
    unpack_weight_int4,
)
from .quant import (dequantize_int4_group_wise, dequantize_linear_per_channel,  # noqa: E402
                    quantize_int4_group_wise, quantize_int4_per_channel,
                    quantize_linear_per_channel)
from .nn import W4A16Linear, W8A16Embedding, W8A16Linear  # noqa: E402

__all__ = [
    "LAYOUT_ROWMAJOR",
    "LAYOUT_TILE16X64",
    "KERNEL_AUTO",
    "KERNEL_GEMM",
    "KERNEL_GEMV",
    "LAYOUT_TILE16X128_I4",
    "W4A16Linear",
    "W8A16Embedding",
    "W8A16Linear",
    "dequantize_int4_group_wise",
    "dequantize_linear_per_channel",
    "linear",
    "linear_argmax",
    "linear_into",
    "linear_multi",
    "linear_multi_w4a16",
    "linear_w4a16",
    "pack_weight",
    "pack_weight_int4",
    "packed_shape",
    "packed_shape_int4",
    "quantize_int4_group_wise",
    "quantize_int4_per_channel",
    "quantize_linear_per_channel",
    "select_kernel",
    "unpack_weight",
    "unpack_weight_int4",
]
