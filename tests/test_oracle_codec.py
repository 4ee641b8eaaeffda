"""Pins the oracle's W4A16 codec against the reference's own known answers.

KAT data lives in tests/golden/reference_kats.json (each entry names the
reference test it restates). Beyond the KATs, properties the mathematics fixes
are checked: the brute-force nearest-grid code, the absmax element landing on
+-7, the scale-aware round-trip bound of quant/verify.py:58-95, and three
deliberately broken decoders (quant/verify.py:140-162) that must be rejected.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from oracle import w4a16 as W
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


def _grid_weight(code_pattern, scales):
    scales = np.asarray(scales, dtype=np.float32)
    codes = np.asarray(code_pattern, dtype=np.float32)
    w = codes[None, None, :] * scales[..., None]
    return f32_to_bf16_bits(w.reshape(scales.shape[0], -1))


def test_grid_round_trip_is_exact_and_recovers_scales():
    kat = KATS["codec_grid_round_trip"]
    w = _grid_weight(kat["code_pattern"], kat["scales"])
    packed, scales = W.quantise(w, kat["group_size"])
    assert np.array_equal(bf16_bits_to_f32(scales), np.asarray(kat["scales"], dtype=np.float32))
    assert np.array_equal(W.dequantise(packed, scales, kat["group_size"]), w)


def test_all_zero_tensor_gets_unit_scales():
    kat = KATS["codec_zero_tensor"]
    w = np.zeros(kat["shape"], dtype=np.uint16)
    packed, scales = W.quantise(w, kat["group_size"])
    assert np.all(bf16_bits_to_f32(scales) == kat["expected_scale"])
    assert np.array_equal(W.dequantise(packed, scales, kat["group_size"]), w)


def test_non_finite_weights_are_rejected():
    w = np.zeros((1, 32), dtype=np.uint16)
    w[0, 0] = 0x7F80  # +inf
    with pytest.raises(ValueError, match="finite"):
        W.quantise(w, 32)


@pytest.mark.parametrize("name", ["codec_nibble_sign_group", "codec_dense_two_rows"])
def test_decode_nibble_order_sign_and_group_index(name):
    kat = KATS[name]
    packed = np.asarray(kat["packed"], dtype=np.uint8)
    scales = f32_to_bf16_bits(np.asarray(kat["scales"], dtype=np.float32))
    got = W.dequantise(packed, scales, kat["group_size"], dtype="f32")
    assert np.array_equal(got, np.asarray(kat["expected"], dtype=np.float32))
    for key, value in kat["spot_values"].items():
        pos = tuple(int(v) for v in key.split(","))
        pos = (0,) + pos if len(pos) == 1 else pos
        assert got[pos] == value


def _brute_force_codes(w_f32, scales_f32, group):
    """Nearest of the 15 grid points, ties to the even code (independent search)."""
    n, k = w_f32.shape
    cands = np.arange(-7, 8, dtype=np.float32)
    s = np.repeat(scales_f32, group, axis=1)
    # distance measured in units of the scale, as the reference divides first
    ratio = (w_f32 / s).astype(np.float32)
    dist = np.abs(ratio[..., None] - cands)
    best = dist.min(axis=-1, keepdims=True)
    tied = dist == best
    # among tied candidates choose the even one (round-half-even)
    even = tied & (np.abs(cands.astype(np.int64)) % 2 == 0)
    pick = np.where(even.any(-1, keepdims=True), even, tied)
    return cands[np.argmax(pick, axis=-1)].astype(np.int16)


@pytest.mark.parametrize("group", [32, 64, 128])
def test_codes_are_nearest_grid_points_and_absmax_hits_seven(rng, group):
    w = f32_to_bf16_bits(rng.normal(0, 0.02, (16, 512)).astype(np.float32))
    packed, scales = W.quantise(w, group)
    codes = W.unpack_codes(packed)
    sf = bf16_bits_to_f32(scales)
    wf = bf16_bits_to_f32(w)
    assert np.array_equal(codes, _brute_force_codes(wf, sf, group))
    assert codes.min() >= -7 and codes.max() <= 7
    grouped = np.abs(wf).reshape(16, -1, group)
    arg = grouped.argmax(-1)
    top = np.take_along_axis(codes.reshape(16, -1, group), arg[..., None], -1)[..., 0]
    assert np.all(np.abs(top) == 7)
    # stored scale is absmax / 7 rounded once to bf16
    absmax = grouped.max(-1)
    assert np.array_equal(sf, round_bf16((absmax / np.float32(7)).astype(np.float32)))


@pytest.mark.parametrize("group", [32, 128])
def test_round_trip_within_scale_aware_bound(group):
    # Same seeded tensor as tests/test_quant_w4a16.py:124-132 (torch RNG).
    torch.manual_seed(20260728)
    w = torch.randn((4, 128 if group == 128 else 96), dtype=torch.bfloat16)
    bits = w.view(torch.int16).numpy().view(np.uint16)
    packed, scales = W.quantise(bits, group)
    restored = W.dequantise(packed, scales, group, dtype="f32")
    wf = bf16_bits_to_f32(bits)
    eps = float(torch.finfo(torch.bfloat16).eps)
    absmax = np.abs(wf).reshape(4, -1, group).max(-1)
    allowed = 0.5 * np.abs(bf16_bits_to_f32(scales)) + 2.0 * eps * absmax
    err = np.abs(restored - wf).reshape(4, -1, group)
    assert np.all(err <= allowed[..., None])


def _signed_groups(packed, shape, group, swapped=False):
    p = packed
    low, high = (p >> 4, p & 0xF) if swapped else (p & 0xF, p >> 4)
    nib = np.stack((low, high), -1).reshape(shape).astype(np.int16)
    return np.where(nib >= 8, nib - 16, nib).reshape(shape[0], shape[1] // group, group)


def test_negative_control_decoders_are_rejected():
    kat = KATS["negative_control_probe"]
    g = kat["group_size"]
    w = _grid_weight(kat["code_pattern"], kat["scales"])
    packed, scales = W.quantise(w, g)
    good = W.dequantise(packed, scales, g)
    assert np.array_equal(good, w)
    s = bf16_bits_to_f32(scales)
    shape = w.shape
    broken = {
        # quant/verify.py:140-148: scales associated with the output axis
        "wrong_group_axis": _signed_groups(packed, shape, g) * s.T[..., None],
        # quant/verify.py:151-155: factor-of-two scale
        "wrong_scale": _signed_groups(packed, shape, g) * (2 * s)[..., None],
        # quant/verify.py:158-162: odd positions decoded first
        "swapped_nibbles": _signed_groups(packed, shape, g, swapped=True) * s[..., None],
    }
    assert sorted(broken) == sorted(kat["broken_decoders"])
    for name, values in broken.items():
        decoded = f32_to_bf16_bits(values.reshape(shape).astype(np.float32))
        assert not np.array_equal(decoded, good), name
