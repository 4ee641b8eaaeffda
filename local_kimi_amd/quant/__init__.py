"""Weight codecs: packed INT4 + bf16 scales (the engine/quant layout) and OCP MXFP4."""

from .mxfp4 import MXFP4_GROUP_SIZE, dequantize_mxfp4, quantize_mxfp4
from .w4a16 import GROUP_SIZE, QMAX, QMIN, SCALE_DTYPE, W4A16Tensor, dequantise, quantise

__all__ = ["GROUP_SIZE", "QMAX", "QMIN", "SCALE_DTYPE", "W4A16Tensor", "dequantise", "quantise",
           "MXFP4_GROUP_SIZE", "dequantize_mxfp4", "quantize_mxfp4"]
