"""Pins the oracle's router, route bookkeeping, combine and MoE block."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

from oracle import moe as M
from oracle import w4a16 as W
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


def test_router_kat_renormalises_and_scales():
    kat = KATS["router_renorm_scale"]
    hidden = f32_to_bf16_bits(np.asarray(kat["hidden"], dtype=np.float32))
    logits = M.router_logits(hidden, np.asarray(kat["router_weight"], dtype=np.float32))
    idx, w = M.route(logits, None, kat["top_k"], routed_scaling_factor=kat["routed_scaling_factor"])
    assert set(idx[0].tolist()) == set(kat["expected_index_set"])
    by_id = dict(zip(idx[0].tolist(), w[0].tolist()))
    np.testing.assert_allclose([by_id[0], by_id[1]], kat["expected_weights_for_indices_0_1"], rtol=1e-6)
    np.testing.assert_allclose(w.sum(-1), [kat["expected_weight_sum"]], rtol=1e-6)


def test_router_matches_brute_force_full_sort(rng):
    logits = rng.normal(0, 1, (16, 256)).astype(np.float32)
    bias = rng.normal(0, 0.1, 256).astype(np.float32)
    idx, w = M.route(logits, bias, 8, routed_scaling_factor=2.446)
    for t in range(16):
        s = 1.0 / (1.0 + np.exp(-logits[t].astype(np.float64)))
        order = sorted(range(256), key=lambda e: (-(s[e] + bias[e]), e))[:8]
        assert idx[t].tolist() == order
        g = s[order]
        np.testing.assert_allclose(w[t], g / g.sum() * 2.446, rtol=2e-6)


def test_sigmoid_matches_torch_sigmoid():
    """The oracle's fp32 sigmoid (1 / (1 + exp(-x)) in fp32, the HIP router's
    formula) against torch.sigmoid (the reference's call, klinear/router.py:52)
    and against the correctly rounded value, over a dense sweep: within 2 ulp
    of torch for x >= 0 (where top-k selections are made), 4 ulp in the
    negative tail, and the selection made from either is the same."""
    import torch

    def ulps(a, b):
        return np.abs(a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64))

    x = np.linspace(-30, 30, 2_000_001, dtype=np.float32)
    ours = M.sigmoid_f32(x)
    theirs = torch.sigmoid(torch.from_numpy(x)).numpy()
    exact = (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)
    assert ulps(ours, theirs).max() <= 4
    assert ulps(ours, theirs)[x >= 0].max() <= 2
    assert ulps(ours, exact).max() <= 4
    assert ulps(ours, exact)[x >= 0].max() <= 1
    assert (ulps(ours, theirs)[x >= 0] == 0).mean() > 0.95
    rng = np.random.default_rng(7)
    logits = rng.normal(0, 1, (256, 256)).astype(np.float32)
    idx, _ = M.route(logits, None, 8)
    choice = torch.sigmoid(torch.from_numpy(logits))
    want = torch.topk(choice, 8, dim=1).indices.numpy()
    assert np.array_equal(np.sort(idx, axis=1), np.sort(want, axis=1))


def test_router_ties_break_to_lower_expert_id():
    logits = np.zeros((1, 16), dtype=np.float32)
    logits[0, [3, 9, 12]] = 1.0
    idx, _ = M.route(logits, None, 4)
    assert idx[0].tolist() == [3, 9, 12, 0]


def test_router_grouped_topk_masks_unselected_groups(rng):
    logits = rng.normal(0, 1, (4, 32)).astype(np.float32)
    idx, _ = M.route(logits, None, 4, num_expert_group=4, topk_group=2)
    s = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    for t in range(4):
        grp = s[t].reshape(4, 8)
        gscore = np.sort(grp, -1)[:, ::-1][:, :2].sum(-1)
        keep = sorted(range(4), key=lambda g: (-gscore[g], g))[:2]
        allowed = {g * 8 + j for g in keep for j in range(8)}
        assert set(idx[t].tolist()) <= allowed


def test_router_grouped_kat_changes_the_selection():
    # 4 groups of 2 experts, logits 0 (score 0.5), the bias sets each choice:
    # choices 0.9 0.5 | 0.8 0.8 | 0.95 0.0 | 0.7 0.75 -> group scores 1.4, 1.6,
    # 0.95, 1.45: groups 1 and 3 kept; top-2 of (0.8, 0.8, 0.7, 0.75) is
    # experts 2 and 3 (tie to the lower id), where ungrouped routing takes 4, 0
    logits = np.zeros((1, 8), dtype=np.float32)
    bias = np.array([0.4, 0.0, 0.3, 0.3, 0.45, -0.5, 0.2, 0.25], dtype=np.float32)
    idx, w = M.route(logits, bias, 2, num_expert_group=4, topk_group=2)
    assert idx[0].tolist() == [2, 3]
    assert w[0].tolist() == [0.5, 0.5]
    assert M.route(logits, bias, 2)[0][0].tolist() == [4, 0]


def test_router_grouped_masks_to_zero_not_minus_infinity():
    # the kept group's choices are negative (-0.1, -0.2); the masked group's
    # experts get choice 0.0 and therefore win (router.py:78, masked_fill 0.0)
    logits = np.zeros((1, 4), dtype=np.float32)
    bias = np.array([-0.6, -0.7, -0.8, -0.9], dtype=np.float32)
    idx, _ = M.route(logits, bias, 2, num_expert_group=2, topk_group=1)
    assert idx[0].tolist() == [2, 3]


@pytest.mark.parametrize("groups", [1, 4, 8])
def test_router_grouped_with_every_group_kept_is_ungrouped(rng, groups):
    logits = rng.normal(0, 1, (16, 64)).astype(np.float32)
    bias = rng.normal(0, 0.1, 64).astype(np.float32)
    a = M.route(logits, bias, 6, num_expert_group=groups, topk_group=groups)
    b = M.route(logits, bias, 6)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_shape_stable_indices_kat():
    kat = KATS["shape_stable_indices"]
    got = M.shape_stable_expert_indices(np.asarray(kat["expert_indices"]), kat["shared_expert_id"])
    assert got.tolist() == kat["expected"]


def _const_packed(code, n, k):
    nib = code & 0xF
    return np.full((n, k // 2), nib | (nib << 4), dtype=np.uint8)


def test_combine_kat_shared_expert_weight_is_one():
    kat = KATS["combine_shared_weight_one"]
    k = kat["reduction"]
    act = f32_to_bf16_bits(np.full((1, 2, k), kat["activated_value"], dtype=np.float32))
    w2p = np.stack([_const_packed(c, 1, k) for c in kat["constant_codes"]])
    w2s = f32_to_bf16_bits(np.full((2, 1, k // kat["group_size"]), kat["scales"], dtype=np.float32))
    y = M.w2_combine(act, np.asarray(kat["expert_indices"]), np.asarray(kat["combine_weights"], dtype=np.float32),
                     w2p, w2s, kat["group_size"])
    assert bf16_bits_to_f32(y).tolist() == kat["expected"]


def test_combine_matches_explicit_route_loop(rng):
    """Mirrors tests/test_moe_combine.py:93-132 with an explicit scalar-ish loop."""
    t_count, r_count, e, n, k, g = 2, 3, 4, 5, 64, 32
    act = f32_to_bf16_bits(rng.normal(0, 1, (t_count, r_count, k)).astype(np.float32))
    idx = np.array([[0, 1, 3], [2, 0, 3]])
    cw = np.array([[0.25, 0.75, 0.125], [0.6, 0.4, 7.0]], dtype=np.float32)
    w2p = rng.integers(0, 256, (e, n, k // 2), dtype=np.uint8)
    w2s = f32_to_bf16_bits((rng.random((e, n, k // g)) * 0.05 + 0.001).astype(np.float32))
    got = M.w2_combine(act, idx, cw, w2p, w2s, g)
    af = bf16_bits_to_f32(act)
    for t in range(t_count):
        eo = []
        for r in range(r_count):
            dec = bf16_bits_to_f32(W.dequantise(w2p[idx[t, r]], w2s[idx[t, r]], g))
            eo.append(bf16_bits_to_f32(f32_to_bf16_bits(
                np.float32(0) + (af[t, r][None, :].astype(np.float64) * dec).sum(-1).astype(np.float32))))
        routed = sum(eo[r].astype(np.float64) * cw[t, r] for r in range(r_count - 1))
        expect = bf16_bits_to_f32(f32_to_bf16_bits(
            bf16_bits_to_f32(f32_to_bf16_bits(routed.astype(np.float32))) + eo[-1]))
        assert np.array_equal(bf16_bits_to_f32(got[t]), expect)


@pytest.mark.parametrize("name", ["schedule_union_counts"])
def test_schedule_union_and_counts_kat(name):
    kat = KATS[name]
    sched = M.build_expert_schedule(np.asarray(kat["expert_indices"]))
    assert len(sched) == kat["expected_union_size"]
    assert [[e, len(t)] for e, t, _ in sched] == kat["expected_counts"]


def test_schedule_zero_and_duplicate_routes_kat():
    kat = KATS["schedule_zero_and_duplicate_routes"]
    hidden = np.asarray(kat["hidden"], dtype=np.float32)
    idx = np.asarray(kat["expert_indices"])
    calls = []

    def fn(e, tokens):
        calls.append((e, tokens.shape[0]))
        return tokens + float(e)

    values, union, counts = M.expert_major_moe(hidden, idx, np.asarray(kat["routing_weights"]), fn)
    assert union == kat["expected_union_size"]
    assert [list(c) for c in counts] == kat["expected_counts"]
    assert calls == [(3, 2)]
    np.testing.assert_allclose(values, kat["expected_values"], rtol=1e-6)


def test_expert_major_matches_token_major(rng):
    hidden = rng.normal(0, 1, (9, 6)).astype(np.float32)
    idx = rng.integers(0, 7, (9, 4))
    idx[0, 3] = -1
    idx[5, 1:] = -1
    w = rng.random((9, 4)).astype(np.float32)
    mats = rng.normal(0, 1, (7, 6, 6)).astype(np.float32)

    def fn(e, tokens):
        return (tokens.astype(np.float64) @ mats[e].T.astype(np.float64)).astype(np.float32)

    values, union, _ = M.expert_major_moe(hidden, idx, w, fn)
    naive = M.naive_token_major_moe(hidden, idx, w, fn)
    np.testing.assert_allclose(values, naive, rtol=1e-6, atol=1e-6)
    assert union == len(np.unique(idx[idx >= 0]))


def test_schedule_tables_match_schedule(rng):
    idx = rng.integers(-1, 12, (7, 5))
    counts, offsets, perm = M.schedule_tables(idx, 12)
    sched = M.build_expert_schedule(idx)
    flat_sched = np.concatenate([tok * 5 + slot for _, tok, slot in sched])
    assert np.array_equal(perm, flat_sched)
    for e, tok, _ in sched:
        assert counts[e] == len(tok)
        assert offsets[e + 1] - offsets[e] == len(tok)


def test_moe_block_is_router_then_swiglu_then_w2_combine(rng):
    vec = np.load(os.path.join(HERE, "golden", "oracle_vectors.npz"))
    y, idx, w = M.moe_block(vec["moe_x"], vec["moe_logits"], None, vec["moe_w1p"], vec["moe_w1s"],
                            vec["moe_w3p"], vec["moe_w3s"], vec["moe_w2p"], vec["moe_w2s"], top_k=2,
                            routed_scaling_factor=2.446, group_size=128)
    assert np.array_equal(y, vec["moe_y"]) and np.array_equal(idx, vec["moe_idx"])
    # the same composition spelled out
    stable = M.shape_stable_expert_indices(idx, vec["moe_w1p"].shape[0] - 1)
    act = W.swiglu(vec["moe_x"], stable, vec["moe_w1p"], vec["moe_w1s"], vec["moe_w3p"], vec["moe_w3s"], 128)
    cw = np.concatenate((w, np.ones((w.shape[0], 1), np.float32)), 1)
    y2 = M.w2_combine(act, stable, cw, vec["moe_w2p"], vec["moe_w2s"], 128)
    assert np.array_equal(y, y2)
    # and the moe block equals expert-major evaluation of the same experts
    e_count = vec["moe_w1p"].shape[0]

    def expert(e, tokens_bits):
        sub = np.full((tokens_bits.shape[0], 1), e)
        a = W.swiglu(tokens_bits, sub, vec["moe_w1p"], vec["moe_w1s"], vec["moe_w3p"], vec["moe_w3s"], 128)
        o = W.grouped(a[:, 0], np.zeros((a.shape[0], 1), np.int64), vec["moe_w2p"][e:e + 1],
                      vec["moe_w2s"][e:e + 1], 128)
        return o[:, 0]

    outs = np.zeros((idx.shape[0], 3, y.shape[1]), np.uint16)
    for e, tok, slot in M.build_expert_schedule(stable):
        outs[tok, slot] = expert(e, vec["moe_x"][tok])
    assert np.array_equal(M.combine(outs, cw), y)
    assert e_count == 7


def test_oracle_vectors_regression():
    vec = np.load(os.path.join(HERE, "golden", "oracle_vectors.npz"))
    for g in (32, 128):
        p, s = W.quantise(vec[f"dense_g{g}_w"], g)
        assert np.array_equal(p, vec[f"dense_g{g}_packed"]) and np.array_equal(s, vec[f"dense_g{g}_scales"])
        assert np.array_equal(W.dense(vec[f"dense_g{g}_x"], p, s, g), vec[f"dense_g{g}_y"])
