"""W8A16 quantization helpers: the quantizer (``_common``), the checkpoint
converter (``convert``) and the loader / swap-in (``load``, imports transformers)."""
from ._common import dequantize_linear_per_channel, quantize_linear_per_channel

__all__ = ["dequantize_linear_per_channel", "quantize_linear_per_channel"]
