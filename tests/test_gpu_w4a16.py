"""GPU parity of the HIP W4A16 path against the numpy oracle.

Bit-exact: the codec (quantise / dequantise) and router expert selection.
Tolerance (stated here, from the quantized-matmul contract): bf16 outputs
within 1e-2 relative / 2e-2 absolute of the oracle, fp32-class accumulation.
Every kernel is also rerun to check run-to-run bit equality.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as OM
from oracle import w4a16 as OW
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

from ._helpers import (ATOL, RTOL, assert_close_bf16, bf16_ulp_distance, from_bits,
                       random_bf16_bits, to_bits)

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _require_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from local_kimi_amd import _lib

    _lib.load()


def _layer(rng, n, k, g, std=0.02):
    w = random_bf16_bits(rng, (n, k), std)
    p, s = OW.quantise(w, g)
    return w, p, s


def _dev_u8(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _dev_bf16(bits):
    return from_bits(bits, DEV)


# ---------------------------------------------------------------------------
# codec


@pytest.mark.parametrize("g", [32, 128])
@pytest.mark.parametrize("n,k", [(7, 256), (96, 2304), (33, 1024)])
def test_quantise_is_bit_exact(rng, n, k, g):
    from local_kimi_amd.quant import dequantise, quantise

    w = random_bf16_bits(rng, (n, k), 0.02)
    w[0, :g] = 0  # an all-zero group -> scale 1.0
    w[1, 3] = f32_to_bf16_bits(np.float32(1e-39))  # subnormal input
    p, s = OW.quantise(w, g)
    enc = quantise(_dev_bf16(w), group_size=g)
    assert np.array_equal(enc.packed.cpu().numpy(), p)
    assert np.array_equal(to_bits(enc.scales), s)
    assert np.array_equal(to_bits(dequantise(enc)), OW.dequantise(p, s, g))
    f32 = dequantise(enc, dtype=torch.float32).cpu().numpy()
    assert np.array_equal(f32, OW.dequantise(p, s, g, dtype="f32"))


def test_quantise_grid_kat_round_trip():
    from local_kimi_amd.quant import dequantise, quantise

    codes = np.asarray([i % 15 - 7 for i in range(32)], np.float32)
    scales = np.asarray([[0.25, 2.0], [8.0, 0.5]], np.float32)
    w = f32_to_bf16_bits((codes[None, None, :] * scales[..., None]).reshape(2, 64))
    enc = quantise(_dev_bf16(w), group_size=32)
    assert np.array_equal(bf16_bits_to_f32(to_bits(enc.scales)), scales)
    assert np.array_equal(to_bits(dequantise(enc)), w)


# ---------------------------------------------------------------------------
# dense


@pytest.mark.parametrize("g", [32, 128])
@pytest.mark.parametrize("m,n,k", [(1, 96, 256), (1, 200, 1024), (2, 64, 2304), (3, 40, 512),
                                   (5, 128, 4096), (8, 72, 256), (13, 50, 768), (1, 24, 6144)])
def test_dense_matches_oracle(rng, m, n, k, g):
    from local_kimi_amd.kernels import w4a16_dense, w4a16_dense_reference

    _, p, s = _layer(rng, n, k, g)
    x = random_bf16_bits(rng, (m, k))
    expected = OW.dense(x, p, s, g)
    args = (_dev_bf16(x), _dev_u8(p), _dev_bf16(s))
    y1 = w4a16_dense(*args)
    y2 = w4a16_dense(*args)
    assert torch.equal(y1, y2)
    assert_close_bf16(to_bits(y1), expected, what="hip dense")
    yr = to_bits(w4a16_dense_reference(*args))
    # the reference-rounding kernel differs from the oracle only by fp32 summation order
    assert np.abs(yr.astype(np.int32) - expected.astype(np.int32)).max() <= 1


def test_dense_reference_test_inputs(rng):
    """Inputs shaped like tests/test_w4a16_dense_gemv.py: uniform nibbles, small scales."""
    from local_kimi_amd.kernels import w4a16_dense

    k, n = 256, 256
    p = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    s = f32_to_bf16_bits((rng.random((n, k // 32)) * 0.05 + 0.001).astype(np.float32))
    for m in (1, 4):
        x = random_bf16_bits(rng, (m, k))
        y = w4a16_dense(_dev_bf16(x), _dev_u8(p), _dev_bf16(s))
        assert_close_bf16(to_bits(y), OW.dense(x, p, s, 32), what=f"dense m={m}")


def test_dense_decode_shape_full_size(rng):
    """The dense decode projection at its real size: x [1, 2304], W [9216, 2304], G=128."""
    from local_kimi_amd.kernels import w4a16_dense
    from local_kimi_amd.quant import quantise

    torch.manual_seed(20260729)
    w = (torch.randn(9216, 2304, device=DEV) * 0.02).to(torch.bfloat16)
    enc = quantise(w, group_size=128)
    x = random_bf16_bits(rng, (1, 2304))
    y = w4a16_dense(_dev_bf16(x), enc.packed, enc.scales)
    expected = OW.dense(x, enc.packed.cpu().numpy(), to_bits(enc.scales), 128)
    worst = assert_close_bf16(to_bits(y), expected, what="dense 9216x2304")
    assert worst < 0.75


# decode GEMV at output widths that leave a partial last 16-row block
@pytest.mark.parametrize("n", [5000, 9000, 10000])
def test_dense_decode_partial_row_blocks(rng, n):
    from local_kimi_amd.kernels import w4a16_dense

    _, p, s = _layer(rng, n, 2304, 128)
    x = random_bf16_bits(rng, (1, 2304))
    y = w4a16_dense(_dev_bf16(x), _dev_u8(p), _dev_bf16(s))
    assert_close_bf16(to_bits(y), OW.dense(x, p, s, 128), what=f"dense n={n}")


# ---------------------------------------------------------------------------
# grouped / swiglu


def _bank(rng, e, n, k, g):
    ps, ss = [], []
    for _ in range(e):
        _, p, s = _layer(rng, n, k, g)
        ps.append(p)
        ss.append(s)
    return np.stack(ps), np.stack(ss)


@pytest.mark.parametrize("g", [32, 128])
def test_grouped_matches_oracle(rng, g):
    from local_kimi_amd.kernels import grouped_w4a16_gemv, grouped_w4a16_reference

    e, n, k = 5, 96, 512
    p, s = _bank(rng, e, n, k, g)
    x = random_bf16_bits(rng, (3, k))
    idx = np.array([[0, 2, 4], [1, 1, 3], [4, 0, 2]], np.int64)
    expected = OW.grouped(x, idx, p, s, g)
    args = (_dev_bf16(x), torch.from_numpy(idx).to(DEV), _dev_u8(p), _dev_bf16(s))
    out = grouped_w4a16_gemv(*args)
    assert torch.equal(out, grouped_w4a16_gemv(*args))
    assert_close_bf16(to_bits(out), expected, what="grouped")
    ref = to_bits(grouped_w4a16_reference(*args))
    assert np.abs(ref.astype(np.int32) - expected.astype(np.int32)).max() <= 1


def test_grouped_reference_test_shape(rng):
    """tests/test_w4a16_gemv.py:60-109 shapes: 3 experts, N=96, K=64, routes [[0, 2]]."""
    from local_kimi_amd.kernels import grouped_w4a16_gemv

    p = rng.integers(0, 256, (3, 96, 32), dtype=np.uint8)
    s = f32_to_bf16_bits((rng.random((3, 96, 2)) * 0.05 + 0.001).astype(np.float32))
    x = random_bf16_bits(rng, (1, 64))
    idx = np.array([[0, 2]], np.int64)
    out = grouped_w4a16_gemv(_dev_bf16(x), torch.from_numpy(idx).to(DEV), _dev_u8(p), _dev_bf16(s))
    expected = OW.grouped(x, idx, p, s, 32)
    assert_close_bf16(to_bits(out), expected, what="grouped K=64")
    assert np.array_equal(bf16_bits_to_f32(to_bits(out)).argmax(-1), bf16_bits_to_f32(expected).argmax(-1))


def test_grouped_out_of_range_index_gives_zeros(rng):
    from local_kimi_amd.kernels import grouped_w4a16_gemv, grouped_w4a16_reference

    p, s = _bank(rng, 2, 16, 256, 128)
    x = random_bf16_bits(rng, (1, 256))
    idx = torch.tensor([[1, -1, 7]], device=DEV)
    for fn in (grouped_w4a16_gemv, grouped_w4a16_reference):
        out = fn(_dev_bf16(x), idx, _dev_u8(p), _dev_bf16(s))
        assert torch.all(out[0, 1:] == 0)
        assert_close_bf16(to_bits(out[0, :1]), OW.grouped(x, np.array([[1]]), p, s, 128)[0])


@pytest.mark.parametrize("g", [32, 128])
def test_swiglu_matches_oracle(rng, g):
    from local_kimi_amd.kernels import grouped_w4a16_swiglu_gemv, registry

    e, n, k = 4, 128, 2304
    w1p, w1s = _bank(rng, e, n, k, g)
    w3p, w3s = _bank(rng, e, n, k, g)
    x = random_bf16_bits(rng, (2, k))
    idx = np.array([[0, 3, 1], [2, 2, 3]], np.int64)
    expected = OW.swiglu(x, idx, w1p, w1s, w3p, w3s, g)
    args = (_dev_bf16(x), torch.from_numpy(idx).to(DEV), _dev_u8(w1p), _dev_bf16(w1s),
            _dev_u8(w3p), _dev_bf16(w3s))
    out = grouped_w4a16_swiglu_gemv(*args)
    assert torch.equal(out, grouped_w4a16_swiglu_gemv(*args))
    assert_close_bf16(to_bits(out), expected, what="swiglu")
    with registry.using("w4a16_grouped", "reference"):
        ref = registry.reference_of("w4a16_swiglu").fn(*args)
    assert np.abs(to_bits(ref).astype(np.int32) - expected.astype(np.int32)).max() <= 1


def test_silu_mul_follows_the_rounding_contract_bit_for_bit(rng):
    """``silu_mul`` against torch's own bf16 ``F.silu(gate) * up`` on the GPU
    (the reference's two ops): bit-identical on 1M random pairs plus edge
    values; against the oracle (numpy's fp32 exp, which may differ from the
    device's in the last fp32 bit) within one bf16 ulp, and equal on at least
    99.9 %."""
    import torch.nn.functional as F

    from local_kimi_amd.kernels import silu_mul

    gate = random_bf16_bits(rng, (1 << 20,), 3.0)
    up = random_bf16_bits(rng, (1 << 20,), 1.0)
    edges = np.array([0.0, -0.0, 1e-30, -1e-30, 88.0, -88.0, 100.0, -100.0, 3e38, -3e38],
                     np.float32)
    gate[:edges.size] = f32_to_bf16_bits(edges)
    g, u = _dev_bf16(gate), _dev_bf16(up)
    out = silu_mul(g, u)
    assert torch.equal(out, F.silu(g) * u)
    want = OW.mul_bf16(OW.silu_bf16(gate), up)
    d = bf16_ulp_distance(to_bits(out), want)
    assert d.max() <= 1 and (d == 0).mean() >= 0.999


# ---------------------------------------------------------------------------
# W2 + combine


def test_w2_combine_kat_72():
    from local_kimi_amd.kernels import fused_w2_combine, fused_w2_combine_reference

    act = torch.ones((1, 2, 32), dtype=torch.bfloat16, device=DEV)
    packed = torch.stack([torch.full((1, 16), c | (c << 4), dtype=torch.uint8) for c in (1, 2)]).to(DEV)
    scales = torch.ones((2, 1, 1), dtype=torch.bfloat16, device=DEV)
    idx = torch.tensor([[0, 1]], device=DEV)
    cw = torch.tensor([[0.25, 0.0]], dtype=torch.float32, device=DEV)
    for fn in (fused_w2_combine, fused_w2_combine_reference):
        y = fn(act, idx, cw, packed, scales)
        assert y.float().cpu().tolist() == [[72.0]]


@pytest.mark.parametrize("g", [32, 128])
def test_w2_combine_matches_oracle(rng, g):
    from local_kimi_amd.kernels import fused_w2_combine, fused_w2_combine_reference

    e, h, i, t, r = 6, 200, 1024, 3, 9
    w2p, w2s = _bank(rng, e, h, i, g)
    act = random_bf16_bits(rng, (t, r, i), 0.1)
    idx = rng.integers(0, e, (t, r)).astype(np.int64)
    cw = rng.random((t, r)).astype(np.float32)
    expected = OM.w2_combine(act, idx, cw, w2p, w2s, g)
    args = (_dev_bf16(act), torch.from_numpy(idx).to(DEV), torch.from_numpy(cw).to(DEV),
            _dev_u8(w2p), _dev_bf16(w2s))
    y = fused_w2_combine(*args)
    assert torch.equal(y, fused_w2_combine(*args))
    assert_close_bf16(to_bits(y), expected, what="w2 combine")
    yr = fused_w2_combine_reference(*args)
    assert_close_bf16(to_bits(yr), expected, what="w2 combine reference")


# H / CUs rounded up gives the rows per block of the one-wave-per-route W2 form
# (reduction width 1024): 2, 3, 9 (last block partial) and 16 rows on 256 CUs
@pytest.mark.parametrize("h,r,g", [(300, 9, 128), (700, 5, 64), (2300, 9, 128), (2300, 9, 256),
                                   (4096, 16, 128)])
def test_w2_combine_route_form_row_splits(rng, h, r, g):
    from local_kimi_amd.kernels import fused_w2_combine

    e, i, t = 3, 1024, 2
    w2p, w2s = _bank(rng, e, h, i, g)
    act = random_bf16_bits(rng, (t, r, i), 0.1)
    idx = rng.integers(0, e, (t, r)).astype(np.int64)
    cw = rng.random((t, r)).astype(np.float32)
    expected = OM.w2_combine(act, idx, cw, w2p, w2s, g)
    args = (_dev_bf16(act), torch.from_numpy(idx).to(DEV), torch.from_numpy(cw).to(DEV),
            _dev_u8(w2p), _dev_bf16(w2s))
    y = fused_w2_combine(*args)
    assert torch.equal(y, fused_w2_combine(*args))
    assert_close_bf16(to_bits(y), expected, what=f"w2 combine h={h} routes={r}")


def test_w2_combine_out_of_range_index_counts_zero(rng):
    """Routes whose expert id lies outside the bank contribute nothing."""
    from local_kimi_amd.kernels import fused_w2_combine

    e, h, i, t, r, g = 3, 512, 1024, 2, 9, 128
    w2p, w2s = _bank(rng, e, h, i, g)
    act = random_bf16_bits(rng, (t, r, i), 0.1)
    idx = rng.integers(0, e, (t, r)).astype(np.int64)
    idx[0, 2], idx[1, 5], idx[1, 0] = -1, e, 1000
    cw = rng.random((t, r)).astype(np.float32)
    bad = (idx < 0) | (idx >= e)
    expected = OM.w2_combine(act, np.where(bad, 0, idx), np.where(bad, 0.0, cw).astype(np.float32),
                             w2p, w2s, g)
    y = fused_w2_combine(_dev_bf16(act), torch.from_numpy(idx).to(DEV), torch.from_numpy(cw).to(DEV),
                         _dev_u8(w2p), _dev_bf16(w2s))
    assert_close_bf16(to_bits(y), expected, what="w2 combine, routes outside the bank")


# ---------------------------------------------------------------------------
# router


@pytest.mark.parametrize("e,k", [(256, 8), (64, 6), (4, 2), (384, 8)])
def test_router_selection_is_bit_exact(rng, e, k):
    from local_kimi_amd.kernels import moe_router

    logits = rng.normal(0, 1, (37, e)).astype(np.float32)
    bias = rng.normal(0, 0.05, e).astype(np.float32)
    for b in (None, bias):
        idx, w = moe_router(torch.from_numpy(logits).to(DEV),
                            None if b is None else torch.from_numpy(b).to(DEV), k,
                            routed_scaling_factor=2.446)
        eidx, ew = OM.route(logits, b, k, routed_scaling_factor=2.446)
        assert np.array_equal(idx.cpu().numpy(), eidx)
        np.testing.assert_allclose(w.cpu().numpy(), ew, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("experts,top_k", [(256, 8), (256, 1), (200, 6), (64, 8), (9, 8),
                                           (8, 8), (256, 3)])
def test_router_many_tokens_bit_exact(rng, experts, top_k):
    """Up to 256 experts and top_k <= 8 select by merging sorted lists across
    the wave; a token whose boundary is closer than the merge keys resolve
    takes the exact rounds. 4096 tokens, with and without a bias, against the
    oracle: selections bit-exact, weights within 2e-6."""
    from local_kimi_amd.kernels import moe_router

    logits = rng.normal(0, 1, (4096, experts)).astype(np.float32)
    bias = rng.normal(0, 0.05, experts).astype(np.float32)
    for b in (None, bias):
        idx, w = moe_router(torch.from_numpy(logits).to(DEV),
                            None if b is None else torch.from_numpy(b).to(DEV), top_k,
                            routed_scaling_factor=2.446)
        eidx, ew = OM.route(logits, b, top_k, routed_scaling_factor=2.446)
        assert np.array_equal(idx.cpu().numpy(), eidx)
        np.testing.assert_allclose(w.cpu().numpy(), ew, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("step_ulps", [1, 3, 256, 512])
def test_router_boundary_near_ties(rng, step_ulps):
    """Candidates with logit 0 (sigmoid exactly 0.5 on every side) whose bias
    puts their choice scores a multiple of `step_ulps` ulps apart, others far
    below: at 1 and 3 ulps the candidates agree in the merge keys' high 24 bits
    and the exact rounds decide (including exact ties, to the lower id); at 256
    and 512 ulps the merge selection is exact by itself."""
    from local_kimi_amd.kernels import moe_router

    tokens, experts = 96, 256
    ulp = np.float32(2.0 ** -24)  # spacing of floats in [0.5, 1)
    bias = ((np.arange(experts) % 12) * step_ulps * ulp).astype(np.float32)
    tied = np.arange(0, experts - 1, 5)
    bias[tied] = bias[tied + 1]  # exact ties too
    logits = np.full((tokens, experts), -6.0, dtype=np.float32)
    for t in range(tokens):
        logits[t, rng.choice(experts, size=12, replace=False)] = 0.0
    idx, w = moe_router(torch.from_numpy(logits).to(DEV), torch.from_numpy(bias).to(DEV), 8,
                        routed_scaling_factor=2.446)
    eidx, ew = OM.route(logits, bias, 8, routed_scaling_factor=2.446)
    assert np.array_equal(idx.cpu().numpy(), eidx)
    np.testing.assert_allclose(w.cpu().numpy(), ew, rtol=2e-6, atol=1e-7)


def test_router_saturated_scores_tie_to_the_lower_id(rng):
    """Logits >= 40: every sigmoid is exactly 1.0, so the top 8 are the lowest
    ids among them."""
    from local_kimi_amd.kernels import moe_router

    logits = rng.normal(0, 1, (32, 256)).astype(np.float32)
    for t in range(32):
        logits[t, rng.choice(256, size=11, replace=False)] = 40.0 + t
    idx, _ = moe_router(torch.from_numpy(logits).to(DEV), None, 8)
    eidx, _ = OM.route(logits, None, 8)
    assert np.array_equal(idx.cpu().numpy(), eidx)


def test_router_kat_and_ties():
    from local_kimi_amd.kernels import moe_router

    idx, w = moe_router(torch.tensor([[3.0, 2.0, 1.0, 0.0]], device=DEV), None, 2,
                        routed_scaling_factor=2.446)
    assert idx.cpu().tolist() == [[0, 1]]
    assert abs(float(w.sum()) - 2.446) < 1e-6
    logits = torch.zeros((1, 16), device=DEV)
    logits[0, [3, 9, 12]] = 1.0
    idx, _ = moe_router(logits, None, 4)
    assert idx.cpu().tolist() == [[3, 9, 12, 0]]


# ---------------------------------------------------------------------------
# whole MoE block


def _moe_case(rng, e_routed, h, i, g, tokens):
    w1p, w1s = _bank(rng, e_routed + 1, i, h, g)
    w3p, w3s = _bank(rng, e_routed + 1, i, h, g)
    w2p, w2s = _bank(rng, e_routed + 1, h, i, g)
    x = random_bf16_bits(rng, (tokens, h))
    logits = rng.normal(0, 1, (tokens, e_routed)).astype(np.float32)
    return x, logits, (w1p, w1s, w3p, w3s, w2p, w2s)


@pytest.mark.parametrize("tokens", [1, 3, 5])  # token-major below 4 tokens, expert-major from 4
def test_moe_block_matches_oracle_small_bank(rng, tokens):
    from local_kimi_amd.kernels import w4a16_moe_block, w4a16_moe_block_reference

    x, logits, banks = _moe_case(rng, 16, 512, 256, 128, tokens)
    ey, eidx, ew = OM.moe_block(x, logits, None, *banks, top_k=4, routed_scaling_factor=2.446,
                                group_size=128)
    dev_banks = [_dev_u8(b) if b.dtype == np.uint8 else _dev_bf16(b) for b in banks]
    args = (_dev_bf16(x), torch.from_numpy(logits).to(DEV), None, *dev_banks, 4, 2.446)
    y, idx, w = w4a16_moe_block(*args)
    assert np.array_equal(idx.cpu().numpy(), eidx)
    np.testing.assert_allclose(w.cpu().numpy(), ew, rtol=2e-6)
    assert_close_bf16(to_bits(y), ey, what="moe block")
    y2, _, _ = w4a16_moe_block(*args)
    assert torch.equal(y, y2)
    yr, idxr, _ = w4a16_moe_block_reference(*args)
    assert torch.equal(idxr, idx)
    assert_close_bf16(to_bits(yr), ey, what="moe block reference")


@pytest.mark.parametrize("with_bias", [False, True])
def test_moe_block_decode_full_size(rng, with_bias):
    """Batch-1 decode at the Kimi-Linear MoE shape: hidden 2304, 256 routed +
    1 shared expert, intermediate 1024, top-8, G=128, weights N(0, 0.02);
    with a router bias, and logits with exact ties near the top-8 boundary."""
    from local_kimi_amd.kernels import w4a16_moe_block
    from local_kimi_amd.quant import quantise

    e_total, h, i, g = 257, 2304, 1024, 128
    gen = torch.Generator(device=DEV).manual_seed(20260729)

    def bank(n, k):
        packed = torch.empty((e_total, n, k // 2), dtype=torch.uint8, device=DEV)
        scales = torch.empty((e_total, n, k // g), dtype=torch.bfloat16, device=DEV)
        for e in range(e_total):
            w = (torch.randn(n, k, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
            enc = quantise(w, group_size=g)
            packed[e].copy_(enc.packed)
            scales[e].copy_(enc.scales)
        return packed, scales

    w1p, w1s = bank(i, h)
    w3p, w3s = bank(i, h)
    w2p, w2s = bank(h, i)
    x = random_bf16_bits(rng, (1, h))
    logits = rng.normal(0, 1, (1, e_total - 1)).astype(np.float32)
    bias = rng.normal(0, 0.05, e_total - 1).astype(np.float32) if with_bias else None
    if not with_bias:  # ties: copies of the 6th..9th largest logits at other ids
        order = np.argsort(-logits[0], kind="stable")
        logits[0, order[100:104]] = logits[0, order[5:9]]
    y, idx, w = w4a16_moe_block(_dev_bf16(x), torch.from_numpy(logits).to(DEV),
                                None if bias is None else torch.from_numpy(bias).to(DEV),
                                w1p, w1s, w3p, w3s, w2p, w2s, 8, 2.446)
    eidx, ew = OM.route(logits, bias, 8, routed_scaling_factor=2.446)
    assert np.array_equal(idx.cpu().numpy(), eidx)
    np.testing.assert_allclose(w.cpu().numpy(), ew, rtol=2e-6, atol=1e-7)
    # the oracle needs only the 9 experts this token uses
    used = list(eidx[0]) + [e_total - 1]
    sub = [t[used].cpu().numpy() if t.dtype == torch.uint8 else to_bits(t[used])
           for t in (w1p, w1s, w3p, w3s, w2p, w2s)]
    stable = np.arange(9)[None, :]
    act = OW.swiglu(x, stable, sub[0], sub[1], sub[2], sub[3], g)
    cw = np.concatenate((ew, np.ones((1, 1), np.float32)), 1)
    ey = OM.w2_combine(act, stable, cw, sub[4], sub[5], g)
    worst = assert_close_bf16(to_bits(y), ey, what="moe decode full size")
    assert worst < 0.75


def test_moe_block_under_graph_replay(rng):
    """Captured once, replayed several times with eager work in between."""
    from local_kimi_amd.kernels import w4a16_moe_block

    x, logits, banks = _moe_case(rng, 8, 256, 128, 128, 1)
    dev_banks = [_dev_u8(b) if b.dtype == np.uint8 else _dev_bf16(b) for b in banks]
    xd, ld = _dev_bf16(x), torch.from_numpy(logits).to(DEV)
    eager, eidx, _ = w4a16_moe_block(xd, ld, None, *dev_banks, 2, 2.446)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        w4a16_moe_block(xd, ld, None, *dev_banks, 2, 2.446)  # warm-up on the side stream
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gy, gidx, _ = w4a16_moe_block(xd, ld, None, *dev_banks, 2, 2.446)
    for _ in range(4):
        gy.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gy, eager) and torch.equal(gidx, eidx)
        _ = (xd.float() * 2).sum().item()  # unrelated eager work between replays


# ---------------------------------------------------------------------------
# registry equivalence harness on the GPU


@pytest.mark.parametrize("op", ["w4a16_dense", "w4a16_grouped", "w4a16_swiglu", "w4a16_w2_combine",
                                "w4a16_fused_qkv"])
def test_every_variant_matches_the_reference_variant(op):
    from local_kimi_amd.kernels import equivalence

    def make(device):
        g = torch.Generator().manual_seed(20260730)
        k, n, e = 512, 64, 4

        def packed(*shape):
            return torch.randint(0, 256, shape, generator=g, dtype=torch.uint8)

        def scales(*shape):
            return (torch.rand(shape, generator=g) * 0.05 + 0.001).to(torch.bfloat16)

        x = torch.randn((2, k), generator=g).to(torch.bfloat16)
        idx = torch.tensor([[0, 3], [2, 2]])
        if op == "w4a16_dense":
            return x, packed(n, k // 2), scales(n, k // 128)
        if op == "w4a16_grouped":
            return x, idx, packed(e, n, k // 2), scales(e, n, k // 128)
        if op == "w4a16_swiglu":
            return x, idx, packed(e, n, k // 2), scales(e, n, k // 128), packed(e, n, k // 2), scales(e, n, k // 128)
        if op == "w4a16_w2_combine":
            act = (torch.randn((2, 2, k), generator=g) * 0.1).to(torch.bfloat16)
            return act, idx, torch.rand((2, 2), generator=g), packed(e, n, k // 2), scales(e, n, k // 128)
        return (x, packed(n, k // 2), scales(n, k // 128), packed(n, k // 2), scales(n, k // 128),
                packed(n, k // 2), scales(n, k // 128))

    # uniform random nibbles with scales up to 0.051 give large outputs; this is
    # the reference's own GPU tolerance for such inputs (tests/test_w4a16_gemv.py:102)
    reports = equivalence.assert_equivalent(op, make, rtol=0.05, atol=0.125, device=DEV)
    assert reports and all(r.passed for r in reports)
