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


def designed_counts(tokens: int, experts: int, top_k: int) -> np.ndarray:
    """Per-expert route counts for a prefill-sized batch whose expert tiles take
    every shape: unused, a handful of rows (the 16-row path), exactly one 64-row
    tile, a full tile plus a tail of 1..16 rows (which rides with the tile
    before it, an 80-row pass) or 17..63 rows (a partial 64-row tile), and
    several hundred rows with assorted tails."""
    head = [1, 16, 17, 0, 64, 65, 80, 81, 127, 128]
    assert experts > len(head)
    rest = experts - len(head)
    counts = np.array(head + [550 + 13 * j for j in range(rest)], dtype=np.int64)
    counts[-1] += tokens * top_k - int(counts.sum())
    assert counts.min() >= 0 and counts.max() <= tokens and counts.sum() == tokens * top_k
    return counts


def designed_router_logits(rng: np.random.Generator, counts: np.ndarray, tokens: int,
                           top_k: int) -> np.ndarray:
    """fp32 logits [tokens, experts] whose sigmoid top-k selection gives exactly
    ``counts[e]`` routes to expert e: each token takes the top_k experts with the
    most routes left (a feasible assignment when sum(counts) = tokens * top_k
    and no count exceeds tokens); chosen experts get logits in [2, 4], the
    others in [-4, -2]."""
    experts = counts.size
    left = counts.astype(np.int64).copy()
    logits = rng.uniform(-4.0, -2.0, (tokens, experts)).astype(np.float32)
    ids = np.arange(experts)
    for t in range(tokens):
        order = np.lexsort((ids, -left))[:top_k]
        assert (left[order] > 0).all()
        left[order] -= 1
        logits[t, order] = rng.uniform(2.0, 4.0, top_k).astype(np.float32)
    assert not left.any()
    return logits


def bf16_ulp_distance(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """Distance in bf16 units in the last place: bit patterns mapped to a
    monotonic integer order (+0 and -0 coincide)."""
    def order(bits):
        b = np.asarray(bits, dtype=np.uint16).astype(np.int32)
        mag = b & 0x7FFF
        return np.where(b & 0x8000, -mag, mag)
    return np.abs(order(a_bits) - order(b_bits))


def paths_agreement(a_bits: np.ndarray, b_bits: np.ndarray) -> tuple[float, float, float]:
    """(fraction bit-identical, fraction within one bf16 ulp, largest distance
    in ulps) of two bf16 outputs. A distance is counted in ulps of the larger
    magnitude of the pair, floored at 1/16 of the outputs' rms, so values
    near zero that cancel are compared at the scale of the outputs."""
    a = bf16_values(a_bits).astype(np.float64)
    b = bf16_values(b_bits).astype(np.float64)
    scale = float(np.sqrt((b * b).mean())) if b.size else 1.0
    mag = np.maximum(np.maximum(np.abs(a), np.abs(b)), scale / 16.0)
    d = np.abs(a - b) / 2.0 ** (np.floor(np.log2(mag)) - 7)
    return float((d == 0).mean()), float((d <= 1).mean()), float(d.max(initial=0.0))


def assert_paths_agree(actual_bits: np.ndarray, expected_bits: np.ndarray, *, exact: float,
                       within_one: float, max_ulps: float, what: str = "") -> None:
    """Two HIP paths that differ only in fp32 accumulation order: at least
    ``exact`` of the outputs bit-identical, ``within_one`` within one ulp, and
    none beyond ``max_ulps`` (paths_agreement's measure)."""
    same, one, worst = paths_agreement(actual_bits, expected_bits)
    assert same >= exact and one >= within_one and worst <= max_ulps, (
        f"{what}: {same:.4%} identical (bound {exact:.2%}), {one:.4%} within one ulp "
        f"(bound {within_one:.2%}), max {worst:.1f} ulps (bound {max_ulps})")
