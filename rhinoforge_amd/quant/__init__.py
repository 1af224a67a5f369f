"""Quantization helpers: the int8 quantizer (``_common``), the int4 quantizers
(``int4``), the checkpoint converter (``convert``) and the loader / swap-in
(``load``, imports transformers)."""
from ._common import dequantize_linear_per_channel, quantize_linear_per_channel
from .int4 import (dequantize_int4_group_wise, quantize_int4_group_wise,
                   quantize_int4_per_channel)

__all__ = ["dequantize_int4_group_wise", "dequantize_linear_per_channel",
           "quantize_int4_group_wise", "quantize_int4_per_channel",
           "quantize_linear_per_channel"]
