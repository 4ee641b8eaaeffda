"""Pins the oracle's dense / grouped / SwiGLU projections.

Checks: a brute-force scalar loop on tiny shapes; torch's own ``F.linear`` and
``F.silu`` on bf16 tensors (the library routines the reference calls); the
SwiGLU rounding-contract KAT; planted mistakes in a copy of the oracle (wrong
group axis, swapped nibbles, missing bf16 rounding) that these checks catch;
and the tolerance budget of the unrounded-weight arithmetic the HIP GEMV uses.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import w4a16 as W
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))
RTOL, ATOL = 1e-2, 2e-2  # bf16 output tolerance of the quantized-matmul path


def _t(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _ulp_diff(a_bits, b_bits):
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    # bf16 bit patterns are monotone within a sign; values here share signs or are tiny
    return np.abs(a - b)


def _random_layer(rng, n, k, g, std=0.02):
    w = f32_to_bf16_bits(rng.normal(0, std, (n, k)).astype(np.float32))
    return W.quantise(w, g)


def test_dense_matches_scalar_loop(rng):
    n, k, g = 5, 64, 32
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = f32_to_bf16_bits((rng.random((n, k // g)) * 0.05 + 0.001).astype(np.float32))
    x = f32_to_bf16_bits(rng.normal(0, 1, (2, k)).astype(np.float32))
    got = W.dense(x, packed, scales, g)
    xf = bf16_bits_to_f32(x)
    sf = bf16_bits_to_f32(scales)
    for m in range(2):
        for row in range(n):
            acc = 0.0
            for kk in range(k):
                byte = int(packed[row, kk // 2])
                nib = (byte >> 4) if kk % 2 else (byte & 0xF)
                q = nib - 16 if nib >= 8 else nib
                wv = float(bf16_bits_to_f32(f32_to_bf16_bits(np.float32(q) * sf[row, kk // g]))[()])
                acc += float(xf[m, kk]) * wv
            assert got[m, row] == f32_to_bf16_bits(np.float32(acc))[()]


@pytest.mark.parametrize("g", [32, 128])
def test_dense_matches_torch_linear_on_decoded_weights(rng, g):
    packed, scales = _random_layer(rng, 192, 512, g)
    x = f32_to_bf16_bits(rng.normal(0, 1, (4, 512)).astype(np.float32))
    got = W.dense(x, packed, scales, g)
    wt = _t(W.dequantise(packed, scales, g))
    ref = F.linear(_t(x).double(), wt.double()).float().to(torch.bfloat16)
    d = _ulp_diff(got, _bits(ref))
    assert d.max() <= 1 and (d > 0).mean() < 0.01


def test_grouped_is_one_dense_projection_per_route(rng):
    e, n, k, g = 4, 48, 256, 128
    banks = [_random_layer(rng, n, k, g) for _ in range(e)]
    packed = np.stack([b[0] for b in banks])
    scales = np.stack([b[1] for b in banks])
    x = f32_to_bf16_bits(rng.normal(0, 1, (3, k)).astype(np.float32))
    idx = np.array([[0, 2, 3], [1, 1, 0], [3, 2, 1]])
    got = W.grouped(x, idx, packed, scales, g)
    for t in range(3):
        for r in range(3):
            exp = W.dense(x[t:t + 1], packed[idx[t, r]], scales[idx[t, r]], g)[0]
            assert np.array_equal(got[t, r], exp)


def test_swiglu_rounding_contract_kat():
    kat = KATS["swiglu_rounding_contract"]
    g_acc = np.float32(kat["gate_accumulator"])
    u_acc = np.float32(kat["up_accumulator"])
    bf16_first = W.mul_bf16(W.silu_bf16(f32_to_bf16_bits(g_acc)), f32_to_bf16_bits(u_acc))
    fp32_through = f32_to_bf16_bits((g_acc / (1 + np.exp(-g_acc))) * u_acc)
    assert bf16_first != fp32_through
    # and torch agrees with the bf16-first contract
    t = F.silu(torch.tensor([float(g_acc)]).to(torch.bfloat16)) * torch.tensor([float(u_acc)]).to(torch.bfloat16)
    assert _bits(t)[0] == bf16_first


def test_swiglu_matches_torch_silu_mul_on_bf16(rng):
    e, n, k, g = 3, 64, 256, 128
    w1 = [_random_layer(rng, n, k, g) for _ in range(e)]
    w3 = [_random_layer(rng, n, k, g) for _ in range(e)]
    w1p, w1s = np.stack([b[0] for b in w1]), np.stack([b[1] for b in w1])
    w3p, w3s = np.stack([b[0] for b in w3]), np.stack([b[1] for b in w3])
    x = f32_to_bf16_bits(rng.normal(0, 1, (2, k)).astype(np.float32))
    idx = np.array([[0, 2], [1, 2]])
    got = W.swiglu(x, idx, w1p, w1s, w3p, w3s, g)
    gate = _t(W.grouped(x, idx, w1p, w1s, g))
    up = _t(W.grouped(x, idx, w3p, w3s, g))
    ref = F.silu(gate) * up
    d = _ulp_diff(got, _bits(ref))
    assert d.max() <= 1 and (d > 0).mean() < 0.01


def test_planted_mistakes_are_caught(rng):
    """Mistakes planted in copies of the oracle fail the checks above."""
    n, k, g = 32, 256, 32
    packed, scales = _random_layer(rng, n, k, g)
    x = f32_to_bf16_bits(rng.normal(0, 1, (1, k)).astype(np.float32))
    good = W.dense(x, packed, scales, g)
    ref = _bits(F.linear(_t(x).double(), _t(W.dequantise(packed, scales, g)).double())
                .float().to(torch.bfloat16))
    # swapped nibble order
    swapped = ((packed & 0xF) << 4 | (packed >> 4)).astype(np.uint8)
    bad1 = W.dense(x, swapped, scales, g)
    # scale groups taken along the wrong axis (rolled rows)
    bad2 = W.dense(x, packed, np.roll(scales, 1, axis=0), g)
    for bad in (bad1, bad2):
        assert _ulp_diff(bad, ref).max() > 1
    assert _ulp_diff(good, ref).max() <= 1


def test_unrounded_weight_arithmetic_stays_inside_tolerance(rng):
    """The HIP GEMV computes sum_k x*q*s exactly in fp32 (no bf16(q*s) step).

    At the MoE decode shapes (K=2304 and K=1024, G=128, weights N(0, 0.02),
    x ~ N(0, 1)) that choice moves each output by under half of the
    1e-2 relative / 2e-2 absolute tolerance.
    """
    for n, k in ((512, 2304), (512, 1024)):
        packed, scales = _random_layer(rng, n, k, 128)
        x = f32_to_bf16_bits(rng.normal(0, 1, (1, k)).astype(np.float32))
        ref = bf16_bits_to_f32(W.dense(x, packed, scales, 128))
        exact_w = W.dequantise(packed, scales, 128, dtype="f32")
        alt = bf16_bits_to_f32(f32_to_bf16_bits(
            (bf16_bits_to_f32(x).astype(np.float64) @ exact_w.astype(np.float64).T).astype(np.float32)))
        err = np.abs(alt - ref)
        budget = ATOL + RTOL * np.abs(ref)
        assert np.all(err <= budget)
        assert (err / budget).max() < 0.5
