"""Shared pytest configuration: markers, import path and seeded helpers."""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture
def rng():
    return np.random.default_rng(20260729)


def bf16_bits(array) -> np.ndarray:
    """float values -> bf16 bit patterns (round to nearest even)."""
    from oracle.bf16 import f32_to_bf16_bits

    return f32_to_bf16_bits(np.asarray(array, dtype=np.float32))
