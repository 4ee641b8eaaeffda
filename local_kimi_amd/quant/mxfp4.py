"""OCP MXFP4 codec on HIP (engine/k3ref/dequant.py:18-73 for the decode).

``dequantize_mxfp4`` keeps the reference signature and errors; the HIP kernel
computes the exact fp32 value ``e2m1 * 2**(e8m0 - 127)`` and the result is
cast once to ``dtype`` (bf16 directly by the kernel). ``quantize_mxfp4`` is
this project's encoder (the reference ships none): shared exponent
``floor(log2(amax)) - 2`` biased by 127 and clamped to [0, 254] (127 for an
all-zero block), E2M1 rounding to nearest with ties to the even code and
saturation at +-6.
"""

from __future__ import annotations

import torch

from .. import _lib

MXFP4_GROUP_SIZE = 32
MXFP4_EXPONENT_BIAS = 127


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dequantize_mxfp4(packed: torch.Tensor, scale: torch.Tensor, *,
                     dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Decode E2M1 nibbles with one E8M0 exponent per group of 32 values."""
    if packed.dtype != torch.uint8 or scale.dtype != torch.uint8:
        raise TypeError("packed and scale tensors must both use torch.uint8")
    if packed.ndim != 2 or scale.ndim != 2:
        raise ValueError("packed and scale tensors must both be matrices")
    if packed.device != scale.device:
        raise ValueError("packed and scale tensors must be on the same device")
    if not torch.empty((), dtype=dtype).is_floating_point():
        raise TypeError("MXFP4 output dtype must be floating point")
    rows, packed_columns = packed.shape
    value_columns = packed_columns * 2
    if scale.shape[0] != rows or value_columns != scale.shape[1] * MXFP4_GROUP_SIZE:
        raise ValueError("MXFP4 scale shape must provide one exponent for every 32 decoded values")
    if packed.device.type != "cuda":
        raise ValueError("the HIP MXFP4 codec requires CUDA tensors")
    direct = dtype in (torch.float32, torch.bfloat16)
    out = torch.empty((rows, value_columns), dtype=dtype if direct else torch.float32,
                      device=packed.device)
    if rows == 0 or value_columns == 0:
        return out.to(dtype)
    p, s = packed.contiguous(), scale.contiguous()
    with torch.cuda.device(packed.device):
        _lib.call("lk_mxfp4_dequantise", p.data_ptr(), s.data_ptr(), out.data_ptr(), rows,
                  value_columns, int(out.dtype == torch.float32), _stream(packed.device))
    return out if direct else out.to(dtype)


def quantize_mxfp4(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 ``[N, K]`` -> ``(packed uint8 [N, K/2], scale uint8 [N, K/32])``."""
    if weight.ndim != 2 or weight.dtype != torch.bfloat16:
        raise TypeError("MXFP4 quantisation takes a BF16 [output, reduction] matrix")
    if weight.device.type != "cuda":
        raise ValueError("the HIP MXFP4 codec requires CUDA tensors")
    n, k = weight.shape
    if n == 0 or k == 0 or k % MXFP4_GROUP_SIZE:
        raise ValueError("MXFP4 reduction dimension must be a nonzero multiple of 32")
    w = weight.contiguous()
    packed = torch.empty((n, k // 2), dtype=torch.uint8, device=w.device)
    scale = torch.empty((n, k // MXFP4_GROUP_SIZE), dtype=torch.uint8, device=w.device)
    with torch.cuda.device(w.device):
        _lib.call("lk_mxfp4_quantise", w.data_ptr(), packed.data_ptr(), scale.data_ptr(), n, k,
                  _stream(w.device))
    return packed, scale
