"""W8A16 quantization helpers (offline converter side of the path)."""
from ._common import dequantize_linear_per_channel, quantize_linear_per_channel

__all__ = ["dequantize_linear_per_channel", "quantize_linear_per_channel"]
