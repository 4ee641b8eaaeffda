"""GPU parity of grouped top-k routing (engine/klinear/router.py:62-80).

Expert selection bit-exact with oracle.moe.route (which the CPU suite pins by
hand-computed cases: a grouping that changes the selection, the masked fill
with 0.0 rather than -inf, and every group kept = ungrouped); weights within
2e-6 relative (fp32, the renormalising sum in selection order on the GPU).
The block on grouped routes: bf16 outputs within 1e-2 relative / 2e-2
absolute of the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as OM
from oracle import w4a16 as OW

from ._helpers import assert_close_bf16, from_bits, random_bf16_bits, to_bits

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _require_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from local_kimi_amd import _lib

    _lib.load()


def _dev(a):
    if a.dtype == np.uint16:
        return from_bits(a, DEV)
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.mark.parametrize("experts,groups,topk_group,top_k", [
    (256, 8, 4, 8), (256, 16, 3, 8), (64, 4, 2, 6), (8, 4, 2, 2), (128, 64, 8, 8),
    (1024, 32, 4, 8), (96, 3, 1, 5), (256, 8, 8, 8)])
def test_grouped_selection_is_bit_exact(rng, experts, groups, topk_group, top_k):
    from local_kimi_amd.kernels import moe_router

    logits = rng.normal(0, 1, (37, experts)).astype(np.float32)
    bias = rng.normal(0, 0.05, experts).astype(np.float32)
    for b in (None, bias):
        idx, w = moe_router(_dev(logits), None if b is None else _dev(b), top_k,
                            routed_scaling_factor=2.446, num_expert_group=groups,
                            topk_group=topk_group)
        eidx, ew = OM.route(logits, b, top_k, routed_scaling_factor=2.446,
                            num_expert_group=groups, topk_group=topk_group)
        assert np.array_equal(idx.cpu().numpy(), eidx)
        np.testing.assert_allclose(w.cpu().numpy(), ew, rtol=2e-6, atol=1e-7)


def test_grouped_kats_on_the_gpu():
    from local_kimi_amd.kernels import moe_router

    logits = torch.zeros((1, 8), dtype=torch.float32, device=DEV)
    bias = torch.tensor([0.4, 0.0, 0.3, 0.3, 0.45, -0.5, 0.2, 0.25], device=DEV)
    idx, w = moe_router(logits, bias, 2, num_expert_group=4, topk_group=2)
    assert idx.cpu().tolist() == [[2, 3]] and w.cpu().tolist() == [[0.5, 0.5]]
    logits = torch.zeros((1, 4), dtype=torch.float32, device=DEV)
    bias = torch.tensor([-0.6, -0.7, -0.8, -0.9], device=DEV)
    idx, _ = moe_router(logits, bias, 2, num_expert_group=2, topk_group=1)
    assert idx.cpu().tolist() == [[2, 3]]  # the masked group's 0.0 beats negative choices


def test_grouped_kernel_with_one_group_matches_the_router(rng):
    from local_kimi_amd import _lib
    from local_kimi_amd.kernels import moe_router

    logits = _dev(rng.normal(0, 1, (64, 256)).astype(np.float32))
    bias = _dev(rng.normal(0, 0.05, 256).astype(np.float32))
    idx = torch.empty((64, 8), dtype=torch.long, device=DEV)
    w = torch.empty((64, 8), dtype=torch.float32, device=DEV)
    _lib.call("lk_moe_router_grouped", logits.data_ptr(), bias.data_ptr(), idx.data_ptr(),
              w.data_ptr(), 64, 256, 8, 1, 1, 2.446, 1,
              torch.cuda.current_stream().cuda_stream)
    ridx, rw = moe_router(logits, bias, 8, routed_scaling_factor=2.446)
    assert torch.equal(idx, ridx)
    assert torch.equal(w, rw)


def test_grouped_near_ties_at_group_and_expert_level(rng):
    from local_kimi_amd.kernels import moe_router

    # quantised logits: many exact ties between group scores and between experts
    logits = (np.round(rng.normal(0, 1, (64, 64)) * 4) / 4).astype(np.float32)
    idx, w = moe_router(_dev(logits), None, 8, num_expert_group=8, topk_group=3)
    eidx, ew = OM.route(logits, None, 8, num_expert_group=8, topk_group=3)
    assert np.array_equal(idx.cpu().numpy(), eidx)
    np.testing.assert_allclose(w.cpu().numpy(), ew, rtol=2e-6, atol=1e-7)


def _bank(rng, e, n, k, g):
    ps, ss = zip(*(OW.quantise(random_bf16_bits(rng, (n, k), 0.02), g) for _ in range(e)))
    return np.stack(ps), np.stack(ss)


@pytest.mark.parametrize("tokens", [1, 3, 37])
def test_block_on_grouped_routes_matches_the_oracle(rng, tokens):
    from local_kimi_amd.kernels import w4a16_moe_block

    e, h, i, g = 32, 512, 256, 128
    banks = (*_bank(rng, e + 1, i, h, g), *_bank(rng, e + 1, i, h, g), *_bank(rng, e + 1, h, i, g))
    x = random_bf16_bits(rng, (tokens, h))
    logits = rng.normal(0, 1, (tokens, e)).astype(np.float32)
    bias = rng.normal(0, 0.05, e).astype(np.float32)
    ey, eidx, ew = OM.moe_block(x, logits, bias, *banks, top_k=4, routed_scaling_factor=2.446,
                                group_size=g, num_expert_group=4, topk_group=2)
    y, idx, w = w4a16_moe_block(_dev(x), _dev(logits), _dev(bias), *(_dev(b) for b in banks), 4,
                                2.446, num_expert_group=4, topk_group=2)
    assert np.array_equal(idx.cpu().numpy(), eidx)
    np.testing.assert_allclose(w.cpu().numpy(), ew, rtol=2e-6, atol=1e-7)
    assert_close_bf16(to_bits(y), ey, what=f"grouped-route block T={tokens}")
    # the grouping changed some selections, so the grouped path is what ran
    uidx, _ = OM.route(logits, bias, 4, routed_scaling_factor=2.446)
    assert not np.array_equal(uidx, eidx) or tokens < 3


def test_klinear_moe_with_grouped_routing(rng):
    from local_kimi_amd.checkpoint import MoeBanks
    from local_kimi_amd.klinear import KLinearMoE

    e, h, i, g, tokens = 16, 256, 128, 128, 5
    w1, w3, w2 = _bank(rng, e + 1, i, h, g), _bank(rng, e + 1, i, h, g), _bank(rng, e + 1, h, i, g)
    gate = random_bf16_bits(rng, (e, h), 0.05)
    bias = rng.normal(0, 0.05, e).astype(np.float32)
    banks = MoeBanks(*(_dev(a) for a in (*w1, *w3, *w2)))
    moe = KLinearMoE(_dev(gate), _dev(bias), banks, top_k=3, routed_scaling_factor=2.446,
                     num_expert_group=4, topk_group=2)
    x = random_bf16_bits(rng, (tokens, h))
    y = moe(_dev(x))
    logits = moe.router_logits(_dev(x)).cpu().numpy()
    ey, _, _ = OM.moe_block(x, logits, bias, *w1, *w3, *w2, top_k=3, routed_scaling_factor=2.446,
                            group_size=g, num_expert_group=4, topk_group=2)
    assert_close_bf16(to_bits(y), ey, what="KLinearMoE grouped routing")
