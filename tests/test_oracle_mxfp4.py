"""Pins the oracle's MXFP4 codec: reference decode KATs and the OCP encoder rules."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

from oracle import mxfp4 as X
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


def test_decode_both_nibbles_and_exponents():
    kat = KATS["mxfp4_nibbles_and_exponents"]
    got = X.dequantize(np.asarray(kat["packed"], np.uint8), np.asarray(kat["scale"], np.uint8))
    assert np.array_equal(got, np.asarray(kat["expected"], np.float32))


def test_hand_built_buffer_is_bit_exact_with_negative_zero():
    kat = KATS["mxfp4_hand_built_buffer"]
    got = X.dequantize(np.asarray(kat["packed"], np.uint8), np.asarray(kat["scale"], np.uint8))
    assert np.array_equal(got.view(np.uint32), np.asarray(kat["expected_float32_bits"], np.uint32))
    for pos in kat["negative_zero_positions"]:
        assert np.signbit(got[0, pos]) and got[0, pos] == 0
    assert not np.signbit(got[0, 0])
    # swapped nibble order (the reference's negative control) is rejected
    p = np.asarray(kat["packed"], np.uint8)
    swapped = ((p & 0xF) << 4 | (p >> 4)).astype(np.uint8)
    bad = X.dequantize(swapped, np.asarray(kat["scale"], np.uint8))
    assert not np.array_equal(bad.view(np.uint32), got.view(np.uint32))


def test_two_group_spot_values():
    kat = KATS["mxfp4_two_groups"]
    got = X.dequantize(np.asarray(kat["packed"], np.uint8), np.asarray(kat["scale"], np.uint8))
    for key, value in kat["spot_values"].items():
        r, c = (int(v) for v in key.split(","))
        assert got[r, c] == value


def test_encoder_grid_values_round_trip_exactly(rng):
    # pick codes and exponents; values on the grid must come back bit exact
    codes = rng.integers(0, 16, (8, 64))
    codes[:, ::32] = 7  # every block holds +-6 so the shared exponent is implied
    exps = rng.integers(100, 140, (8, 2))
    w = X.E2M1_CODEBOOK[codes] * np.ldexp(np.float32(1), np.repeat(exps - 127, 32, axis=1)).astype(np.float32)
    packed, scale = X.quantize(w.astype(np.float32))
    assert np.array_equal(scale, exps.astype(np.uint8))
    back = X.dequantize(packed, scale)
    assert np.array_equal(np.abs(back), np.abs(w))


def test_encoder_ties_to_even_and_saturation():
    # block with amax 6 (exponent 0): values at midpoints
    vals = np.array([6.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0] + [0.0] * 24, np.float32)[None]
    packed, scale = X.quantize(vals)
    assert scale[0, 0] == 127
    got = X.dequantize(packed, scale)[0, :8]
    assert got.tolist() == [6.0, 0.0, 1.0, 1.0, 2.0, 2.0, 4.0, 4.0]
    # amax 7 -> exponent floor(log2 7) - 2 = 0, so 7 saturates to 6
    packed, scale = X.quantize(np.array([[7.0] + [0.0] * 31], np.float32))
    assert scale[0, 0] == 127 and X.dequantize(packed, scale)[0, 0] == 6.0


def test_encoder_is_nearest_grid_point_brute_force(rng):
    w = rng.normal(0, 0.02, (16, 128)).astype(np.float32)
    packed, scale = X.quantize(w)
    back = X.dequantize(packed, scale)
    s = np.repeat(np.ldexp(np.float32(1), scale.astype(np.int32) - 127), 32, axis=1)
    grid = X.E2M1_CODEBOOK[None, None, :8] * s[..., None]
    best = np.abs(np.abs(w)[..., None] - grid).min(-1)
    assert np.allclose(np.abs(np.abs(back) - np.abs(w)), best, rtol=0, atol=1e-12)
    assert np.all(np.sign(back) * np.sign(w) >= 0)


def test_zero_block_uses_unit_exponent():
    packed, scale = X.quantize(np.zeros((2, 32), np.float32))
    assert np.all(scale == 127) and np.all(X.dequantize(packed, scale) == 0)


def test_linear_matches_bf16_matmul(rng):
    vec = np.load(os.path.join(HERE, "golden", "oracle_vectors.npz"))
    y = X.linear(vec["mx_x"], vec["mx_packed"], vec["mx_scale"])
    assert np.array_equal(y, vec["mx_y"])
    import torch
    import torch.nn.functional as F
    xt = torch.from_numpy(vec["mx_x"].view(np.int16)).view(torch.bfloat16)
    wt = torch.from_numpy(X.dequantize(vec["mx_packed"], vec["mx_scale"])).to(torch.bfloat16)
    ref = F.linear(xt.double(), wt.double()).float().to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    d = np.abs(y.astype(np.int32) - ref.astype(np.int32))
    assert d.max() <= 1
