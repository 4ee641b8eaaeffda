"""GPU parity of the model-slice callers (engine/klinear/quantized.py:160-180,
engine/klinear/moe.py:278-334, engine/generate.py:226-306).

``W4A16Linear`` and ``KLinearMoE`` are loaded from a W4A16 checkpoint written
in the reference's layout (G = 128, bf16 router weight), run through the
registry's default (HIP) ops, and are checked against the oracle within the
quantized-matmul tolerance (1e-2 relative / 2e-2 absolute in bf16). The
router logits (router.py:50-51) are fp32 sums of exact bf16 products in this
build's fixed order, the same for every batch size, not the oracle's or
torch's: they are checked against a float64 sum within 2e-6 relative and
against torch's F.linear, whose selections they reproduce (near-ties within
the two summation orders' rounding counted); the oracle block is fed the
logits the GPU computed (the selection from given logits is what the kernels
own, and is compared bit-exactly elsewhere).
``MoEDecodeGraph`` replays are compared with eager forwards bit for bit,
with eager work between replays.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as OM
from oracle import w4a16 as OW

from ._helpers import assert_close_bf16, bf16_values, from_bits, random_bf16_bits, to_bits

pytestmark = pytest.mark.gpu

DEV = "cuda"
LAYER, EXPERTS, HIDDEN, INTER, G, TOP_K = 2, 16, 256, 128, 128, 4


@pytest.fixture(scope="module", autouse=True)
def _require_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from local_kimi_amd import _lib

    _lib.load()


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    """A small W4A16 checkpoint: one linear, one MoE layer, and the oracle's copies."""
    from local_kimi_amd.checkpoint import expert_name, save_w4a16_checkpoint, shared_expert_name
    from local_kimi_amd.quant.w4a16 import W4A16Tensor

    rng = np.random.default_rng(20260801)
    path = tmp_path_factory.mktemp("ckpt")

    def enc(n, k):
        p, s = OW.quantise(random_bf16_bits(rng, (n, k), 0.02), G)
        return W4A16Tensor(packed=torch.from_numpy(p), scales=from_bits(s), original_shape=(n, k),
                           group_size=G), (p, s)

    tensors, banks = {}, {"w1": [], "w3": [], "w2": []}
    shared = {"w1": "gate_proj", "w3": "up_proj", "w2": "down_proj"}
    for e in range(EXPERTS + 1):
        for bank, (n, k) in (("w1", (INTER, HIDDEN)), ("w3", (INTER, HIDDEN)), ("w2", (HIDDEN, INTER))):
            t, ps = enc(n, k)
            name = expert_name(LAYER, e, bank) if e < EXPERTS else shared_expert_name(LAYER, shared[bank])
            tensors[name] = t
            banks[bank].append(ps)
    lin, lin_ps = enc(384, HIDDEN)
    tensors["model.layers.0.mlp.up_proj.weight"] = lin
    prefix = f"model.layers.{LAYER}.block_sparse_moe.gate."
    tensors[prefix + "weight"] = torch.from_numpy(
        rng.normal(0, 0.05, (EXPERTS, HIDDEN)).astype(np.float32)).to(torch.bfloat16)
    tensors[prefix + "e_score_correction_bias"] = torch.from_numpy(
        rng.normal(0, 0.02, EXPERTS).astype(np.float32))
    save_w4a16_checkpoint(path, tensors)
    stacked = [np.stack([ps[j] for ps in banks[b]]) for b in ("w1", "w3", "w2") for j in (0, 1)]
    bias = tensors[prefix + "e_score_correction_bias"].numpy()
    return path, lin_ps, stacked, bias


@pytest.mark.parametrize("tokens,experts,h", [(1, 256, 2304), (5, 16, 256), (64, 40, 4096), (3, 7, 8)])
def test_router_logits(rng, tokens, experts, h):
    from local_kimi_amd.kernels import router_logits

    x = random_bf16_bits(rng, (tokens, h))
    w = random_bf16_bits(rng, (experts, h), 0.05)
    got = router_logits(from_bits(x, DEV), from_bits(w, DEV))
    assert got.dtype == torch.float32 and got.shape == (tokens, experts)
    want = bf16_values(x).astype(np.float64) @ bf16_values(w).astype(np.float64).T
    np.testing.assert_allclose(got.cpu().numpy(), want, rtol=2e-6, atol=2e-6 * np.abs(want).max())
    assert torch.equal(got, router_logits(from_bits(x, DEV), from_bits(w, DEV)))


@pytest.mark.parametrize("wdtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("tokens,experts,h", [(1, 256, 2304), (37, 24, 512), (3, 7, 8)])
def test_router_logits_with_a_float_router_weight(rng, tokens, experts, h, wdtype):
    """fp32 and fp16 router weights go through the same HIP launch (fp16
    widened exactly); the fp32 products are rounded, so the bound is a few
    fp32 ulps of the row's magnitude against a float64 sum."""
    from local_kimi_amd.kernels import router_logits

    x = random_bf16_bits(rng, (tokens, h))
    w = torch.from_numpy(rng.normal(0, 0.05, (experts, h)).astype(np.float32)).to(wdtype)
    got = router_logits(from_bits(x, DEV), w.to(DEV))
    want = bf16_values(x).astype(np.float64) @ w.double().numpy().T
    scale = np.abs(bf16_values(x)).astype(np.float64) @ np.abs(w.double().numpy()).T
    assert np.all(np.abs(got.cpu().numpy() - want) <= 4e-6 * scale + 1e-30)
    assert torch.equal(got, router_logits(from_bits(x, DEV), w.to(DEV)))


def test_router_logits_do_not_depend_on_the_batch(rng):
    """Every token's logits are summed in the same order whatever the batch size
    (decode T=1, a 64-token tile boundary, a 300-token prefill)."""
    from local_kimi_amd.kernels import router_logits

    x = from_bits(random_bf16_bits(rng, (300, 2304)), DEV)
    w = from_bits(random_bf16_bits(rng, (256, 2304), 2304 ** -0.5), DEV)
    full = router_logits(x, w)
    for lo, hi in ((0, 1), (5, 6), (0, 16), (3, 67), (64, 65), (100, 300)):
        assert torch.equal(router_logits(x[lo:hi].contiguous(), w), full[lo:hi]), (lo, hi)
    with pytest.raises(ValueError, match="router logits need"):
        router_logits(x, w[:, :128])
    with pytest.raises(TypeError, match="BF16"):
        router_logits(x.float(), w)


@pytest.mark.parametrize("tokens", [1, 64, 2048])
def test_selection_from_hip_logits_matches_torch_linear_logits(rng, tokens):
    """The reference computes logits with F.linear(x.float(), W.float())
    (klinear/router.py:50-51). The HIP logits differ from torch's only in the
    fp32 summation order; the selections made from the two must be identical
    except at a near-tie within that rounding, which the check counts."""
    from local_kimi_amd.kernels import moe_router, router_logits

    x = from_bits(random_bf16_bits(rng, (tokens, 2304)), DEV)
    w = from_bits(random_bf16_bits(rng, (256, 2304), 2304 ** -0.5), DEV)
    bias = torch.from_numpy(rng.normal(0, 0.01, 256).astype(np.float32)).to(DEV)
    ours = router_logits(x, w)
    theirs = torch.nn.functional.linear(x.float(), w.float())
    # both are fp32 sums of 2304 exact products (error ~ sqrt(K) * eps * |terms|)
    mag = theirs.abs().amax(dim=1, keepdim=True)
    assert ((ours - theirs).abs() <= 1e-5 * mag).all()
    idx_a, w_a = moe_router(ours, bias, 8, routed_scaling_factor=2.446)
    idx_b, w_b = moe_router(theirs, bias, 8, routed_scaling_factor=2.446)
    # near-ties: 8th and 9th choice scores closer than the logits' disagreement
    # can take (sigmoid' <= 1/4, so 1e-5 * |logits| <= 1e-5 in score)
    choice = torch.sigmoid(theirs) + bias
    top9 = choice.topk(9, dim=1).values
    near = (top9[:, 7] - top9[:, 8]) < 2e-5
    same = (idx_a == idx_b).all(dim=1)
    assert bool((same | near).all())
    assert int((~same).sum()) <= max(1, tokens // 1000)
    torch.testing.assert_close(w_a[same], w_b[same], rtol=1e-5, atol=0)
    # the oracle router on torch's logits selects what the GPU router selects
    eidx, ew = OM.route(theirs.cpu().numpy(), bias.cpu().numpy(), 8, routed_scaling_factor=2.446)
    assert np.array_equal(idx_b.cpu().numpy(), eidx)


def test_router_weights_match_torch_sigmoid(rng):
    """Combine weights: torch.sigmoid gathered, renormalised by sum + 1e-20 and
    scaled (klinear/router.py:52-85), computed by torch on the same device."""
    from local_kimi_amd.kernels import moe_router

    logits = torch.from_numpy(rng.normal(0, 1.5, (512, 256)).astype(np.float32)).to(DEV)
    idx, got = moe_router(logits, None, 8, routed_scaling_factor=2.446)
    s = torch.sigmoid(logits)
    want_idx = s.topk(8, dim=1).indices
    assert torch.equal(idx.sort(dim=1).values, want_idx.sort(dim=1).values)
    picked = s.gather(1, idx)
    want = picked / (picked.sum(dim=1, keepdim=True) + 1e-20) * 2.446
    torch.testing.assert_close(got, want, rtol=4e-7 * 8, atol=0)


def test_w4a16_linear_matches_oracle(ckpt, rng):
    from local_kimi_amd.checkpoint import W4A16Index
    from local_kimi_amd.kernels import w4a16_dense
    from local_kimi_amd.klinear import W4A16Linear

    path, (p, s), _, _ = ckpt
    enc = W4A16Index(path).load_w4a16("model.layers.0.mlp.up_proj.weight", (384, HIDDEN), device=DEV)
    lin = W4A16Linear.from_encoded(enc)
    x = random_bf16_bits(rng, (2, 3, HIDDEN))
    y = lin(from_bits(x, DEV))
    assert y.shape == (2, 3, 384) and y.dtype == torch.bfloat16
    want = OW.dense(x.reshape(6, HIDDEN), p, s, G)
    assert_close_bf16(to_bits(y).reshape(6, 384), want, what="W4A16Linear")
    direct = w4a16_dense(from_bits(x, DEV).reshape(6, HIDDEN), enc.packed, enc.scales)
    assert torch.equal(y.reshape(6, 384), direct)
    with pytest.raises(ValueError, match="does not match"):
        lin(torch.zeros(2, HIDDEN + 1, dtype=torch.bfloat16, device=DEV))


@pytest.mark.parametrize("tokens", [1, 3, 8, 40])  # token-major below 4 tokens, expert-major from 4
def test_klinear_moe_from_checkpoint_matches_oracle(ckpt, rng, tokens):
    from local_kimi_amd.checkpoint import W4A16Index
    from local_kimi_amd.klinear import KLinearMoE

    path, _, banks, bias = ckpt
    moe = KLinearMoE.from_checkpoint(W4A16Index(path), LAYER, device=DEV, num_experts=EXPERTS,
                                     hidden=HIDDEN, intermediate=INTER, top_k=TOP_K,
                                     routed_scaling_factor=2.446)
    x = random_bf16_bits(rng, (tokens, HIDDEN))
    xd = from_bits(x, DEV)
    y = moe(xd.reshape(1, tokens, HIDDEN))
    assert y.shape == (1, tokens, HIDDEN)
    logits = moe.router_logits(xd).cpu().numpy()
    want, _, _ = OM.moe_block(x, logits, bias, *banks, top_k=TOP_K, routed_scaling_factor=2.446,
                              group_size=G)
    assert_close_bf16(to_bits(y.reshape(tokens, HIDDEN)), want, what=f"KLinearMoE T={tokens}")


def test_moe_decode_graph_replays_match_eager(ckpt, rng):
    from local_kimi_amd.checkpoint import W4A16Index
    from local_kimi_amd.klinear import KLinearMoE, MoEDecodeGraph

    path, _, _, _ = ckpt
    moe = KLinearMoE.from_checkpoint(W4A16Index(path), LAYER, device=DEV, num_experts=EXPERTS,
                                     hidden=HIDDEN, intermediate=INTER, top_k=TOP_K)
    runner = MoEDecodeGraph(moe, tokens=1)
    for _ in range(4):
        x = from_bits(random_bf16_bits(rng, (1, HIDDEN)), DEV)
        eager = moe(x)
        torch.cuda.synchronize()
        got = runner(x)
        torch.cuda.synchronize()
        assert torch.equal(got, eager)
