"""bfloat16 helpers for the numpy oracle (bf16 carried as uint16 bits).

torch rounds float32 -> bfloat16 with round-to-nearest-even (c10::BFloat16);
these helpers restate that rule so every rounding point in the oracle is
explicit.
"""

from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(values) -> np.ndarray:
    """Round float32 values to bf16 (nearest, ties to even); return uint16 bits."""
    a = np.array(values, dtype=np.float32, copy=True, ndmin=0)
    shape = a.shape
    a = a.reshape(-1)
    bits = a.view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
    out = rounded.astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        out = np.where(nan, np.uint16(0x7FC0), out)
    return out.reshape(shape)


def bf16_bits_to_f32(bits) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32).reshape(b.shape)


def round_bf16(values) -> np.ndarray:
    """float32 -> bf16 -> float32 (the value torch holds after ``.to(bf16)``)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(values))


def bf16_tiny() -> float:
    """Smallest positive normal bf16 (torch.finfo(torch.bfloat16).tiny)."""
    return float(bf16_bits_to_f32(np.array([0x0080], dtype=np.uint16))[0])
