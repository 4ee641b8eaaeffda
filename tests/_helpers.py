"""Shared helpers for the test suite (bf16 bit views, tolerances, seeded inputs)."""

from __future__ import annotations

import numpy as np
import torch

# Tolerance of the quantized-matmul path: bf16 outputs within 1e-2 relative /
# 2e-2 absolute of the oracle (fp32-class accumulation on both sides).
RTOL = 1e-2
ATOL = 2e-2


def to_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def from_bits(bits: np.ndarray, device="cpu") -> torch.Tensor:
    arr = np.ascontiguousarray(bits, dtype=np.uint16)
    return torch.from_numpy(arr.view(np.int16).copy()).view(torch.bfloat16).to(device)


def bf16_values(bits: np.ndarray) -> np.ndarray:
    from oracle.bf16 import bf16_bits_to_f32

    return bf16_bits_to_f32(bits)


def assert_close_bf16(actual_bits: np.ndarray, expected_bits: np.ndarray, *, rtol=RTOL, atol=ATOL,
                      what: str = "") -> float:
    """Assert |a - e| <= atol + rtol*|e| elementwise; return the worst budget fraction."""
    a = bf16_values(actual_bits).astype(np.float64)
    e = bf16_values(expected_bits).astype(np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    assert np.isfinite(a).all(), f"{what}: non-finite output"
    err = np.abs(a - e)
    budget = atol + rtol * np.abs(e)
    worst = float((err / budget).max()) if err.size else 0.0
    if worst > 1.0:
        i = np.unravel_index(np.argmax(err / budget), err.shape)
        raise AssertionError(f"{what}: max error {err[i]:.4g} at {i} (expected {e[i]:.6g}, got "
                             f"{a[i]:.6g}); worst budget fraction {worst:.3f}")
    return worst


def random_bf16_bits(rng: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    from oracle.bf16 import f32_to_bf16_bits

    return f32_to_bf16_bits(rng.normal(0, std, shape).astype(np.float32))
