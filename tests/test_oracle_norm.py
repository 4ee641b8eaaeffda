"""Pins for oracle/norm.py: hand-computed cases, invariants, torch's CPU
evaluation of the reference expressions (engine/klinear/norm.py:9-52, the
third-party arithmetic the reference calls), and planted mistakes that those
pins catch. The reference has no test of these norms of its own."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import norm as N
from oracle.kda import round_to

_TORCH = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}


# ---------------------------------------------------------------------------
# hand-computed cases

def test_three_four_row():
    """x = [3, 4]: mean square 12.5, so x / sqrt(12.5) = [0.848528..., 1.131370...]."""
    got = N.rms_norm([[3.0, 4.0]], [1.0, 1.0], 0.0, "float32", "float32")
    np.testing.assert_allclose(got, [[3 / math.sqrt(12.5), 4 / math.sqrt(12.5)]], rtol=2e-7)
    assert abs(got[0, 0] - 0.8485281) < 1e-6 and abs(got[0, 1] - 1.1313708) < 1e-6


@pytest.mark.parametrize("width,value", [(4, 2.0), (16, 4.0), (64, 8.0)])
def test_one_hot_row_normalises_to_sqrt_width(width, value):
    """c e_i has mean square c^2 / width: it normalises to sqrt(width) e_i for any c > 0."""
    x = np.zeros((3, width))
    x[0, 1], x[1, 0], x[2, width - 1] = 0.75, 3.0, 1024.0
    got = N.rms_norm(x, np.ones(width), 0.0, "bfloat16", "bfloat16")
    want = np.zeros_like(x)
    want[x != 0] = value
    assert np.array_equal(got, want)


def test_rounding_order_case():
    """width 2, x = [1, 0], weight 1.046875 (bf16): n = bf16(sqrt 2) = 1.4140625
    (181/128), w * n = 1.48034668 rounds to 1.4765625 (189/128). Rounding the
    product w * sqrt(2) = 1.48050... once instead gives 1.484375 (190/128)."""
    got = N.rms_norm([[1.0, 0.0]], [1.046875, 1.0], 0.0, "bfloat16", "bfloat16")
    assert got[0, 0] == 1.4765625 and got[0, 1] == 0.0


def test_weight_in_another_dtype_keeps_the_rounded_normalised_value():
    """fp32 weight, bf16 x: the product is fp32 of the bf16-rounded value (torch promotion)."""
    got = N.rms_norm([[1.0, 0.0]], [1.046875, 1.0], 0.0, "bfloat16", "float32")
    assert got[0, 0] == np.float32(1.046875 * 1.4140625)


def test_zero_row_with_eps_gives_zeros():
    got = N.rms_norm(np.zeros((2, 8)), np.ones(8), 1e-6, "bfloat16", "bfloat16")
    assert np.array_equal(got, np.zeros((2, 8)))


def test_eps_enters_under_the_root():
    """x = [1, 1], eps = 3: mean square 1, 1 / sqrt(1 + 3) = 0.5."""
    got = N.rms_norm([[1.0, 1.0]], [1.0, 1.0], 3.0, "float32", "float32")
    assert np.array_equal(got, [[0.5, 0.5]])


def test_add_then_norm():
    """residual [1, 0] + delta [2, 0] = [3, 0]: one-hot, normalises to sqrt(2)
    (within one fp32 ulp: 3 * fp32(1 / fp32(sqrt 4.5)))."""
    s, y = N.add_rms_norm([[1.0, 0.0]], [[2.0, 0.0]], [1.0, 1.0], 0.0, "float32", "float32")
    assert np.array_equal(s, [[3.0, 0.0]])
    assert abs(y[0, 0] - math.sqrt(2.0)) <= 2.0 ** -23 and y[0, 1] == 0.0


def test_add_rounds_the_sum_to_storage():
    """bf16 1 + 2^-9 is 1 + 2^-9 in fp32 but 1.0 in bf16 (ties to even)."""
    s, _ = N.add_rms_norm([[1.0, 1.0]], [[2.0 ** -9, 0.0]], [1.0, 1.0], 0.0, "bfloat16", "bfloat16")
    assert np.array_equal(s, [[1.0, 1.0]])


def test_gated_norm_halves_at_zero_gate_and_passes_at_large_gate():
    """One-hot width 4 normalises to 2; sigmoid(0) = 1/2 gives 1, sigmoid(40) = 1 in fp32 gives 2."""
    x = np.array([[0.0, 5.0, 0.0, 0.0]] * 2)
    gate = np.array([[0.0] * 4, [40.0] * 4])
    got = N.rms_gated_norm(x, gate, np.ones(4), 0.0, "bfloat16")
    assert np.array_equal(got, [[0, 1.0, 0, 0], [0, 2.0, 0, 0]])


def test_gated_norm_rounds_fp32_values_to_the_input_dtype_first():
    """fp32 values [1 + 2^-12, 1] become bf16 [1, 1]: normalised to exactly
    [1, 1] (unrounded they would give 1 + 2^-13 and 1 - 2^-13, which a
    float32 result keeps)."""
    got = N.rms_gated_norm([[1.0 + 2.0 ** -12, 1.0]], [[40.0, 40.0]], [1.0, 1.0], 0.0, "float32")
    assert got[0, 0] != got[0, 1]
    got = N.rms_gated_norm([[1.0 + 2.0 ** -12, 1.0]], [[40.0, 40.0]], [1.0, 1.0], 0.0, "bfloat16")
    assert np.array_equal(got, [[1.0, 1.0]])


def test_scale_invariance():
    rng = np.random.default_rng(3)
    x = round_to(rng.normal(size=(5, 64)), "bfloat16")
    w = round_to(rng.normal(size=64), "bfloat16")
    a = N.rms_norm(x, w, 0.0, "bfloat16", "bfloat16")
    assert np.array_equal(a, N.rms_norm(8.0 * x, w, 0.0, "bfloat16", "bfloat16"))
    assert np.array_equal(a, N.rms_norm(x / 1024.0, w, 0.0, "bfloat16", "bfloat16"))


# ---------------------------------------------------------------------------
# torch's evaluation of the reference expressions (CPU, the library the
# reference calls). torch's fp32 mean and rsqrt may differ from the oracle's
# in the last fp32 place, which can flip the rounding of a normalised value to
# the input dtype: results agree within two ulps of the input dtype
# everywhere (four in fp32, where the rsqrt's own ulp carries through two
# products), and exactly on nearly every element (on most of them in fp32).

def _ulp(values: np.ndarray, dtype: str) -> np.ndarray:
    bits = {"bfloat16": 8, "float16": 11, "float32": 24}[dtype]
    mag = np.maximum(np.abs(values), np.finfo(np.float32).tiny)
    return 2.0 ** (np.floor(np.log2(mag)) - (bits - 1))


def _agree(got, want, dtype):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.abs(got - want) <= (4 if dtype == "float32" else 2) * _ulp(want, dtype))
    assert np.mean(got == want) > (0.5 if dtype == "float32" else 0.99)


@pytest.mark.parametrize("x_dtype,w_dtype", [("bfloat16", "bfloat16"), ("float16", "float16"),
                                             ("float32", "float32"), ("bfloat16", "float32"),
                                             ("float16", "bfloat16")])
def test_rms_norm_matches_torch(x_dtype, w_dtype):
    rng = np.random.default_rng(4)
    x = torch.from_numpy(rng.normal(size=(64, 2304)).astype(np.float32)).to(_TORCH[x_dtype])
    w = torch.from_numpy((1 + 0.1 * rng.normal(size=2304)).astype(np.float32)).to(_TORCH[w_dtype])
    values = x.float()
    ref = w * (values * torch.rsqrt(values.square().mean(dim=-1, keepdim=True) + 1e-6)).to(x.dtype)
    got = N.rms_norm(x.double().numpy(), w.double().numpy(), 1e-6, x_dtype, w_dtype)
    assert N.promoted(x_dtype, w_dtype) == {v: k for k, v in _TORCH.items()}[ref.dtype]
    _agree(got, ref.double().numpy(), x_dtype)


def test_add_rms_norm_matches_torch():
    rng = np.random.default_rng(5)
    r = torch.from_numpy(rng.normal(size=(16, 2304)).astype(np.float32)).bfloat16()
    d = torch.from_numpy(rng.normal(size=(16, 2304)).astype(np.float32) * 3).bfloat16()
    w = torch.from_numpy((1 + 0.1 * rng.normal(size=2304)).astype(np.float32)).bfloat16()
    s = r + d
    values = s.float()
    ref = w * (values * torch.rsqrt(values.square().mean(dim=-1, keepdim=True) + 1e-6)).to(s.dtype)
    got_s, got = N.add_rms_norm(r.double().numpy(), d.double().numpy(), w.double().numpy(), 1e-6,
                                "bfloat16", "bfloat16")
    assert np.array_equal(got_s, s.double().numpy())
    _agree(got, ref.double().numpy(), "bfloat16")


@pytest.mark.parametrize("values_dtype", ["bfloat16", "float32"])
def test_gated_norm_matches_torch(values_dtype):
    rng = np.random.default_rng(6)
    v = torch.from_numpy(rng.normal(size=(32, 4, 128)).astype(np.float32)).to(_TORCH[values_dtype])
    g = torch.from_numpy(rng.normal(size=(32, 4, 128)).astype(np.float32) * 2).bfloat16()
    w = torch.from_numpy((1 + 0.1 * rng.normal(size=128)).astype(np.float32)).bfloat16()
    values = v.to(torch.bfloat16)  # attention.py:324
    vf = values.float()
    normalized = vf * torch.rsqrt(vf.square().mean(dim=-1, keepdim=True) + 1e-5)
    ref = (normalized * w.float() * torch.sigmoid(g.float())).to(values.dtype)
    got = N.rms_gated_norm(v.double().numpy(), g.double().numpy(), w.double().numpy(), 1e-5,
                           "bfloat16")
    _agree(got, ref.double().numpy(), "bfloat16")


# ---------------------------------------------------------------------------
# planted mistakes: each fails one of the hand-computed cases above

def _sum_for_mean(x, weight, eps, x_dtype, weight_dtype):
    v = np.asarray(x, np.float64)
    n = round_to(v / np.sqrt(np.sum(v * v, axis=-1, keepdims=True) + eps), x_dtype)
    return round_to(np.asarray(weight) * n, N.promoted(x_dtype, weight_dtype))


def _eps_outside(x, weight, eps, x_dtype, weight_dtype):
    v = np.asarray(x, np.float64)
    n = round_to(v / (np.sqrt(np.mean(v * v, axis=-1, keepdims=True)) + eps), x_dtype)
    return round_to(np.asarray(weight) * n, N.promoted(x_dtype, weight_dtype))


def _one_rounding(x, weight, eps, x_dtype, weight_dtype):
    v = np.asarray(x, np.float64)
    n = v / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + eps)
    return round_to(np.asarray(weight) * n, N.promoted(x_dtype, weight_dtype))


@pytest.mark.parametrize("broken", [_sum_for_mean, _eps_outside, _one_rounding])
def test_planted_mistakes_fail_a_hand_computed_case(broken):
    cases = [
        (([[3.0, 4.0]], [1.0, 1.0], 0.0, "float32", "float32"),
         [[3 / math.sqrt(12.5), 4 / math.sqrt(12.5)]]),
        (([[1.0, 0.0]], [1.046875, 1.0], 0.0, "bfloat16", "bfloat16"), [[1.4765625, 0.0]]),
        (([[1.0, 1.0]], [1.0, 1.0], 3.0, "float32", "float32"), [[0.5, 0.5]]),
    ]
    for args, want in cases:
        np.testing.assert_allclose(N.rms_norm(*args), want, rtol=2e-7)
    assert any(not np.allclose(broken(*args), want, rtol=1e-6, atol=0) for args, want in cases)


def test_planted_gate_mistake_fails_the_half_gate_case():
    x = np.array([[0.0, 5.0, 0.0, 0.0]])
    ungated = round_to(N.rms_norm(x, np.ones(4), 0.0, "float32", "float32") * np.zeros((1, 4)),
                       "bfloat16")  # gate applied raw (g = 0) instead of sigmoid(g)
    assert not np.array_equal(ungated, N.rms_gated_norm(x, np.zeros((1, 4)), np.ones(4), 0.0,
                                                        "bfloat16"))
