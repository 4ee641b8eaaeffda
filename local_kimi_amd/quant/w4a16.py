"""Symmetric group-wise INT4 weights with bf16 scales, encoded and decoded on HIP.

Same layout and encoder as engine/quant/w4a16.py:1-129: ``packed [N, K/2]``
uint8 with the even reduction index in the low nibble, codes in [-7, 7],
``scales [N, K/G]`` bf16 equal to ``bf16(absmax / 7)`` (1.0 for an all-zero
group, clamped to the smallest normal bf16). The reference accepts only G=32;
here any power-of-two multiple of 32 that divides K is accepted.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import _lib

GROUP_SIZE = 32
QMIN = -7
QMAX = 7
SCALE_DTYPE = torch.bfloat16


def _check_group(in_features: int, group_size: int) -> None:
    if group_size <= 0 or group_size % 32 or group_size & (group_size - 1):
        raise ValueError(f"group size must be a power-of-two multiple of 32, got {group_size}")
    if in_features % group_size:
        raise ValueError(f"the reduction axis must be divisible by group size {group_size}")


@dataclass(frozen=True)
class W4A16Tensor:
    """Packed INT4 weights and one bf16 scale per reduction-axis group
    (engine/quant/w4a16.py:20-65, with the group size a field that is checked
    against the shapes instead of fixed at 32)."""

    packed: torch.Tensor
    scales: torch.Tensor
    original_shape: tuple[int, int]
    original_dtype: torch.dtype = torch.bfloat16
    group_size: int = GROUP_SIZE

    def __post_init__(self) -> None:
        if len(self.original_shape) != 2:
            raise ValueError("W4A16 weights must have shape [out_features, in_features]")
        out_features, in_features = self.original_shape
        if out_features <= 0 or in_features <= 0:
            raise ValueError("W4A16 dimensions must be positive")
        _check_group(in_features, self.group_size)
        if self.packed.dtype != torch.uint8:
            raise TypeError("packed weights must use torch.uint8 storage")
        if self.scales.dtype != SCALE_DTYPE:
            raise TypeError("W4A16 scales must use torch.bfloat16 storage")
        if self.original_dtype != torch.bfloat16:
            raise TypeError("W4A16 currently accepts and restores BF16 weights only")
        expected_packed = (out_features, in_features // 2)
        expected_scales = (out_features, in_features // self.group_size)
        if tuple(self.packed.shape) != expected_packed:
            raise ValueError(f"packed shape must be {expected_packed}, got {tuple(self.packed.shape)}")
        if tuple(self.scales.shape) != expected_scales:
            raise ValueError(f"scale shape must be {expected_scales}, got {tuple(self.scales.shape)}")
        if self.packed.device != self.scales.device:
            raise ValueError("packed weights and scales must be on the same device")

    @property
    def storage_bytes(self) -> int:
        return (self.packed.numel() * self.packed.element_size()
                + self.scales.numel() * self.scales.element_size())


def quantise(weight: torch.Tensor, *, group_size: int = GROUP_SIZE) -> W4A16Tensor:
    """Quantise a bf16 ``[out, in]`` matrix on the GPU (bit-exact with the reference)."""
    if weight.ndim != 2:
        raise ValueError("weight must have shape [out_features, in_features]")
    if weight.dtype != torch.bfloat16:
        raise TypeError("weight must have dtype torch.bfloat16")
    _check_group(weight.shape[1], group_size)
    if weight.device.type != "cuda":
        raise ValueError("the HIP W4A16 quantiser requires a CUDA (HIP) tensor")
    if not bool(torch.isfinite(weight).all()):
        raise ValueError("weight must contain only finite values")
    n, k = weight.shape
    w = weight.detach().contiguous()
    packed = torch.empty((n, k // 2), dtype=torch.uint8, device=weight.device)
    scales = torch.empty((n, k // group_size), dtype=SCALE_DTYPE, device=weight.device)
    with torch.cuda.device(weight.device):
        _lib.call("lk_w4a16_quantise", w.data_ptr(), packed.data_ptr(), scales.data_ptr(), n, k,
                  group_size, torch.cuda.current_stream(weight.device).cuda_stream)
    return W4A16Tensor(packed=packed, scales=scales, original_shape=(n, k), group_size=group_size)


def dequantise(quantized: W4A16Tensor, *, dtype: torch.dtype | None = None) -> torch.Tensor:
    """Restore ``bf16(q * s)`` (default) or the exact float32 ``q * s``."""
    output_dtype = quantized.original_dtype if dtype is None else dtype
    if output_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("dequantise output dtype must be torch.bfloat16 or torch.float32")
    if quantized.packed.device.type != "cuda":
        raise ValueError("the HIP W4A16 decoder requires CUDA (HIP) tensors")
    n, k = quantized.original_shape
    out = torch.empty((n, k), dtype=output_dtype, device=quantized.packed.device)
    p = quantized.packed.contiguous()
    s = quantized.scales.contiguous()
    with torch.cuda.device(p.device):
        _lib.call("lk_w4a16_dequantise", p.data_ptr(), s.data_ptr(), out.data_ptr(), n, k,
                  quantized.group_size, int(output_dtype == torch.float32),
                  torch.cuda.current_stream(p.device).cuda_stream)
    return out
