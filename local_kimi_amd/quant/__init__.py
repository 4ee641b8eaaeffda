"""Packed INT4 + bf16-scale codec (the engine/quant layout contract)."""

from .w4a16 import GROUP_SIZE, QMAX, QMIN, SCALE_DTYPE, W4A16Tensor, dequantise, quantise

__all__ = ["GROUP_SIZE", "QMAX", "QMIN", "SCALE_DTYPE", "W4A16Tensor", "dequantise", "quantise"]
