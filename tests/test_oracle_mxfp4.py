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


# ---------------------------------------------------------------------------
# SiTU (engine/kernels/moe_grouped.py:163-178) and the MXFP4 expert compositions


def _bits(values):
    return f32_to_bf16_bits(np.asarray(values, dtype=np.float32))


def test_situ_closed_forms():
    # g = 0 -> 0 for any u
    assert np.all(bf16_bits_to_f32(X.situ(_bits([0.0, 0.0]), _bits([3.0, -7.0]))) == 0.0)
    # saturation: tanh and sigmoid round to 1 in fp32 -> beta * linear_beta
    assert bf16_bits_to_f32(X.situ(_bits([88.0]), _bits([1e4]))) == 4.0 * 25.0
    # no linear_beta: the up term passes through -> beta * u
    assert bf16_bits_to_f32(X.situ(_bits([88.0]), _bits([3.0]), linear_beta=None)) == 12.0
    # odd in u, bit for bit
    g = _bits(np.linspace(-6, 6, 25))
    u = _bits(np.linspace(0.1, 40, 25))
    pos, neg = X.situ(g, u), X.situ(g, _bits(-bf16_bits_to_f32(u)))
    assert np.array_equal(pos ^ neg, np.where(pos & 0x7FFF, 0x8000, pos ^ neg).astype(np.uint16))
    # small arguments: beta * tanh(g / beta) * sigmoid(g) -> g / 2, tanh(u / lb) * lb -> u
    small = X.situ(_bits([2.0 ** -10]), _bits([2.0 ** -10]))
    assert bf16_bits_to_f32(small)[0] == pytest.approx(2.0 ** -21, rel=2 ** -7)


def test_situ_catches_swapped_betas():
    rng = np.random.default_rng(5)
    g, u = _bits(rng.normal(0, 3, 200)), _bits(rng.normal(0, 30, 200))
    good = X.situ(g, u, 4.0, 25.0)
    assert not np.array_equal(good, X.situ(g, u, 25.0, 4.0))


def test_grouped_matches_per_route_linear():
    rng = np.random.default_rng(6)
    banks = [X.quantize(rng.normal(0, 0.02, (24, 64)).astype(np.float32)) for _ in range(3)]
    p = np.stack([b[0] for b in banks])
    s = np.stack([b[1] for b in banks])
    x = _bits(rng.normal(0, 1, (4, 64)))
    idx = np.array([[0, 2], [1, 1], [2, 0], [0, 0]])
    out = X.grouped(x, idx, p, s)
    for t in range(4):
        for r in range(2):
            assert np.array_equal(out[t, r], X.linear(x[t:t + 1], p[idx[t, r]], s[idx[t, r]])[0])


def test_moe_block_matches_a_token_loop():
    from oracle import moe as OM
    from oracle.w4a16 import mul_bf16, silu_bf16

    rng = np.random.default_rng(7)
    e_routed, h, inter, k = 5, 64, 32, 2

    def bank(n, kk):
        enc = [X.quantize(rng.normal(0, 0.05, (n, kk)).astype(np.float32)) for _ in range(e_routed + 1)]
        return np.stack([a for a, _ in enc]), np.stack([b for _, b in enc])

    w1, w3, w2 = bank(inter, h), bank(inter, h), bank(h, inter)
    x = _bits(rng.normal(0, 1, (3, h)))
    logits = rng.normal(0, 1, (3, e_routed)).astype(np.float32)
    y, idx, w = X.moe_block(x, logits, None, *w1, *w3, *w2, top_k=k, routed_scaling_factor=2.446)
    for t in range(3):
        eo = []
        for e in list(idx[t]) + [e_routed]:
            act = mul_bf16(silu_bf16(X.linear(x[t:t + 1], w1[0][e], w1[1][e])),
                           X.linear(x[t:t + 1], w3[0][e], w3[1][e]))
            eo.append(X.linear(act, w2[0][e], w2[1][e])[0])
        want = OM.combine(np.stack(eo)[None], np.concatenate((w[t], [1.0]))[None].astype(np.float32))
        assert np.array_equal(y[t], want[0])


def test_expert_mlp_composition_and_f16_linear():
    rng = np.random.default_rng(8)
    w1, w3 = (X.quantize(rng.normal(0, 0.05, (32, 64)).astype(np.float32)) for _ in range(2))
    w2 = X.quantize(rng.normal(0, 0.05, (64, 32)).astype(np.float32))
    x = _bits(rng.normal(0, 1, (2, 64)))
    y = X.expert_mlp(x, *w1, *w3, *w2)
    act = X.situ(X.linear(x, *w1), X.linear(x, *w3))
    assert np.array_equal(y, X.linear(act, *w2))
    # fp16 linear agrees with the bf16 one where both types hold the inputs exactly
    xf = np.asarray(bf16_bits_to_f32(x), np.float16).view(np.uint16)
    a = np.asarray(X.linear_f16(xf, *w1), np.uint16).view(np.float16).astype(np.float64)
    b = bf16_bits_to_f32(X.linear(x, *w1)).astype(np.float64)
    assert np.allclose(a, b, rtol=1e-2, atol=1e-2)


# ---------------------------------------------------------------------------
# fp8 hi/lo activation split (the scaled fp4 MFMA's A operand)

def _e4m3_grid():
    codes = np.arange(256)
    codes = codes[(codes & 0x7F) != 0x7F]  # 0x7F / 0xFF are NaN in OCP E4M3
    return codes, X.e4m3_decode(codes)


def test_e4m3_decode_known_codes():
    kat = {0x38: 1.0, 0xB8: -1.0, 0x7E: 448.0, 0x08: 2.0 ** -6, 0x01: 2.0 ** -9, 0x00: 0.0,
           0x3C: 1.5, 0x40: 2.0, 0x78: 256.0}
    for c, v in kat.items():
        assert X.e4m3_decode(np.array([c]))[0] == v, hex(c)


def test_e4m3_encode_is_nearest_with_ties_to_even(rng):
    codes, vals = _e4m3_grid()
    normal = vals[(np.abs(vals) >= 2.0 ** -6) & (np.abs(vals) <= 256.0)]
    v = np.exp(rng.uniform(np.log(2.0 ** -6), np.log(255.0), 20000)) * rng.choice([-1.0, 1.0], 20000)
    v = v.astype(np.float32)
    got = X.e4m3_decode(X.e4m3_encode(v))
    dist = np.abs(normal[None, :] - v.astype(np.float64)[:, None]).min(1)
    assert np.array_equal(np.abs(got - v), dist)
    # exact midpoints between neighbours go to the even mantissa
    pos = np.sort(normal[normal > 0])
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    enc = X.e4m3_encode(mids)
    assert np.all((enc & 1) == 0)
    assert np.all(np.isin(X.e4m3_decode(enc), pos))


def test_e4m3_encode_flushes_below_smallest_normal():
    v = np.array([2.0 ** -6, 0.99 * 2.0 ** -6, -(2.0 ** -7), 0.0, -0.0], np.float32)
    assert list(X.e4m3_encode(v)) == [0x08, 0x00, 0x80, 0x00, 0x80]


def test_split_reconstructs_bf16_blocks(rng):
    x = f32_to_bf16_bits((rng.normal(0, 1, (32, 2304)) * np.exp(rng.normal(0, 2, (32, 1))))
                         .astype(np.float32))
    hi, lo, sc = X.split_fp8(x)
    xf = bf16_bits_to_f32(x).astype(np.float64)
    d = X.split_decode(hi, lo, sc)
    amax = np.repeat(np.abs(xf).reshape(32, -1, 32).max(-1), 32, axis=-1)
    # hi holds the top 4 significant bits, lo the next 4: error below 2**-9 of the block max
    assert np.all(np.abs(d - xf) <= amax * 2.0 ** -9)
    assert np.linalg.norm(d - xf) / np.linalg.norm(xf) < 1e-6
    # the scaled block max lies in [128, 256): hi never saturates
    assert np.all(np.abs(X.e4m3_decode(hi)) <= 256.0)


def test_split_exact_for_four_bit_values_and_zero_blocks():
    vals = np.array([1.0, -1.5, 0.75, 3.5, 0.0, 448.0 / 64, -0.125, 2.0], np.float32)
    x = f32_to_bf16_bits(np.tile(vals, 8)[None, :].astype(np.float32))
    x = np.concatenate((x, np.zeros((1, 64), np.uint16)), 0)
    hi, lo, sc = X.split_fp8(x)
    assert np.array_equal(X.split_decode(hi, lo, sc), bf16_bits_to_f32(x).astype(np.float64))
    assert np.all(lo[0] & 0x7F == 0)  # no residual
    assert np.all(hi[1] == 0) and np.all(lo[1] == 0) and np.all(sc[1] == 0)  # exponent -127 -> byte 0
    # block exponents: block max 7.0 -> E = 2 -> e = -5 (byte 122)
    assert np.all((sc[0] & 0xFF) == 122)


def test_split_keeps_the_mxfp4_product_within_tolerance(rng):
    """The whole point: x . W with x split is within the bf16 tolerance of x . W."""
    w = rng.normal(0, 0.02, (256, 2304)).astype(np.float32)
    p, s = X.quantize(w)
    wd = X.dequantize(p, s).astype(np.float64)
    x = f32_to_bf16_bits(rng.normal(0, 1, (16, 2304)).astype(np.float32))
    ref = bf16_bits_to_f32(x).astype(np.float64) @ wd.T
    got = X.split_decode(*X.split_fp8(x)) @ wd.T
    assert np.max(np.abs(got - ref) / (2e-2 + 1e-2 * np.abs(ref))) < 0.01
