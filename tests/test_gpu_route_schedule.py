"""GPU parity of the one-block schedule forms of the expert-major block.

With at most 256 routed experts, batches of at most 16 tokens route and
schedule in one launch (schedule_one_kernel with routing), or, on the
persistent 16-row GEMMs (K >= 512), batches of at most 8 tokens route and
schedule inside every block of the gate/up GEMM with no launch before it,
and batches of up to 1024 token-routes are ranked there after the router
launch; otherwise batches of at most 1024 token-routes route on a grid and
schedule in one launch; larger batches, or the path knob
moe_fused_schedule=off for any batch, take the router launch and the chunked
schedule launches. All run the same selection code and the same stable
ranking, so the selections, combine weights and block outputs must be
bit-identical; the results are also checked against the oracle within the
quantized-matmul tolerance (1e-2 relative / 2e-2 absolute in bf16), with the
expert indices bit-exact. Cases: with and without a router bias, tied logits
(equal keys keep the lower expert id first), both sides of the 8-token
routing limit, the largest one-launch schedule (113 tokens x 9 routes = 1017
token-routes) and one token past it, batches on the 64-row tiles (whose
router launch also writes the paired activation rows in W4A16), and both
weight formats.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as OM
from oracle import mxfp4 as X
from oracle import w4a16 as OW
from oracle.bf16 import bf16_bits_to_f32

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


def _w4_bank(rng, e, n, k, g=128):
    ps, ss = [], []
    for _ in range(e):
        p, s = OW.quantise(random_bf16_bits(rng, (n, k), 0.02), g)
        ps.append(p)
        ss.append(s)
    return np.stack(ps), np.stack(ss)


def _mx_bank(rng, e, n, k):
    enc = [X.quantize(bf16_bits_to_f32(random_bf16_bits(rng, (n, k), 0.02))) for _ in range(e)]
    return np.stack([p for p, _ in enc]), np.stack([s for _, s in enc])


def _fused_and_split(monkeypatch, fn, *args):
    """fn(*args) on the one-launch forms, then on the router and chunked schedule."""
    from local_kimi_amd._lib import forced_path

    a = fn(*args)
    torch.cuda.synchronize()
    with forced_path("moe_fused_schedule", "off"):
        b = fn(*args)
        torch.cuda.synchronize()
    return a, b


@pytest.mark.parametrize("weights", ["w4a16", "mxfp4"])
@pytest.mark.parametrize("tokens,top_k,bias,ties", [
    (4, 8, False, False),
    (8, 8, True, True),
    (16, 8, True, True),     # the largest batch routed in the schedule's block
    (17, 8, False, False),   # routed on a grid, scheduled in one launch
    (23, 8, True, False),
    (64, 8, False, True),
    (113, 8, True, False),   # 1017 token-routes: the largest one-launch schedule
    (114, 8, False, False),  # 1026 token-routes: separate launches on both sides
    (200, 4, True, True),    # 1000 token-routes at top-4
    (231, 8, True, False),   # 2079 token-routes: 64-row tiles, the router launch pairs x
    (300, 8, False, True),
])
def test_fused_router_schedule_matches_separate_launches(rng, monkeypatch, weights, tokens, top_k,
                                                         bias, ties):
    from local_kimi_amd.kernels import mxfp4_moe_block, w4a16_moe_forward

    e_routed, h, inter = 256, 256, 128
    bank = _mx_bank if weights == "mxfp4" else _w4_bank
    banks = (*bank(rng, e_routed + 1, inter, h), *bank(rng, e_routed + 1, inter, h),
             *bank(rng, e_routed + 1, h, inter))
    x = random_bf16_bits(rng, (tokens, h))
    logits = rng.normal(0, 1, (tokens, e_routed)).astype(np.float32)
    if ties:  # blocks of equal logits across the selection boundary
        logits[:, 40:72] = logits[:, 40:41]
        logits[::3, 200:230] = 3.0
    b = rng.normal(0, 0.05, e_routed).astype(np.float32) if bias else None
    args = (_dev(x), _dev(logits), None if b is None else _dev(b), *(_dev(v) for v in banks),
            top_k, 2.446)
    block = mxfp4_moe_block if weights == "mxfp4" else w4a16_moe_forward
    (y, idx, w), (y0, idx0, w0) = _fused_and_split(monkeypatch, block, *args)
    assert torch.equal(idx, idx0)
    assert torch.equal(w, w0)
    assert torch.equal(y, y0), "one-launch and chunked router + schedule differ"
    # oracle on a few tokens (the selections of all of them)
    eidx, ew = OM.route(logits, b, top_k, routed_scaling_factor=2.446)
    assert np.array_equal(idx.cpu().numpy(), eidx)
    np.testing.assert_allclose(w.cpu().numpy(), ew, rtol=2e-6)
    sel = np.unique(np.array([0, tokens // 2, tokens - 1]))
    if weights == "mxfp4":
        ey, _, _ = X.moe_block(x[sel], logits[sel], b, *banks, top_k=top_k,
                               routed_scaling_factor=2.446)
    else:
        ey, _, _ = OM.moe_block(x[sel], logits[sel], b, *banks, top_k=top_k,
                                routed_scaling_factor=2.446, group_size=128)
    assert_close_bf16(to_bits(y)[sel], ey, what=f"{weights} block T={tokens} k={top_k}")


@pytest.mark.parametrize("weights", ["w4a16", "mxfp4"])
@pytest.mark.parametrize("tokens,top_k,routed,bias,ties", [
    (1, 8, 256, False, False),
    (2, 8, 256, True, True),
    (3, 8, 256, False, True),
    (4, 8, 256, True, False),
    (4, 2, 64, False, False),
    (4, 6, 32, True, True),     # few experts: routes of one token land on few tiles
    (5, 8, 256, False, False),  # split SwiGLU: the down GEMM reads block 0's tables
    (8, 8, 256, True, True),    # the most tokens routed in the GEMM (one per wave)
    (9, 8, 256, False, True),   # router launch, ranking in the GEMM
    (12, 4, 32, True, False),
    (16, 8, 256, True, True),   # 144 token-routes over three groups' bitmaps
    (16, 16, 64, False, False),  # 272 token-routes, 256 selections
])
def test_gate_up_gemm_that_routes_matches_separate_launches(rng, monkeypatch, weights, tokens,
                                                            top_k, routed, bias, ties):
    """Batches of at most 8 tokens at K >= 512: the persistent gate/up GEMM
    routes and schedules the batch in every block (no router or schedule
    launch); from 9 tokens the router launch selects and every block ranks
    the selections. On the split SwiGLU (5 tokens and more in W4A16, every
    size in MXFP4) block 0 also writes the schedule the down GEMM reads.
    Selections, weights and outputs bit-identical to the router and chunked
    schedule launches (path knob off), and the block against the oracle on
    every token."""
    from local_kimi_amd.kernels import mxfp4_moe_block, w4a16_moe_forward

    h, inter = 512, 256
    bank = _mx_bank if weights == "mxfp4" else _w4_bank
    banks = (*bank(rng, routed + 1, inter, h), *bank(rng, routed + 1, inter, h),
             *bank(rng, routed + 1, h, inter))
    x = random_bf16_bits(rng, (tokens, h))
    logits = rng.normal(0, 1, (tokens, routed)).astype(np.float32)
    if ties:
        logits[:, 4:12] = logits[:, 4:5]
    b = rng.normal(0, 0.05, routed).astype(np.float32) if bias else None
    args = (_dev(x), _dev(logits), None if b is None else _dev(b), *(_dev(v) for v in banks),
            top_k, 2.446)
    block = mxfp4_moe_block if weights == "mxfp4" else w4a16_moe_forward
    (y, idx, w), (y0, idx0, w0) = _fused_and_split(monkeypatch, block, *args)
    assert torch.equal(idx, idx0)
    assert torch.equal(w, w0)
    assert torch.equal(y, y0), "the routing gate/up GEMM and the separate launches differ"
    eidx, ew = OM.route(logits, b, top_k, routed_scaling_factor=2.446)
    assert np.array_equal(idx.cpu().numpy(), eidx)
    np.testing.assert_allclose(w.cpu().numpy(), ew, rtol=2e-6)
    if weights == "mxfp4":
        ey, _, _ = X.moe_block(x, logits, b, *banks, top_k=top_k, routed_scaling_factor=2.446)
    else:
        ey, _, _ = OM.moe_block(x, logits, b, *banks, top_k=top_k, routed_scaling_factor=2.446,
                                group_size=128)
    assert_close_bf16(to_bits(y), ey,
                      what=f"{weights} routing gate/up T={tokens} k={top_k} E={routed}")


@pytest.mark.parametrize("weights", ["w4a16", "mxfp4"])
@pytest.mark.parametrize("tokens,top_k,routed,h,bias", [
    (17, 8, 256, 1024, True),
    (24, 8, 64, 512, False),
    (40, 6, 256, 1024, True),
    (64, 8, 256, 1024, False),  # 576 token-routes: two entries per thread
    (113, 8, 32, 512, True),    # 1017 token-routes, the most that rank in the GEMM
    (100, 1, 256, 1024, False),  # 200 token-routes at top-1
])
def test_gate_up_gemm_that_ranks_the_router_selections(rng, monkeypatch, weights, tokens, top_k,
                                                       routed, h, bias):
    """Batches above 8 tokens on the split SwiGLU with at most 1024
    token-routes: the router launch, then every block of the gate/up GEMM
    ranks its selections and block 0 writes the schedule for the down GEMM
    (no schedule launch). Selections, weights and outputs bit-identical to
    the router and chunked schedule launches (path knob off), and the block
    against the oracle on a third of the tokens."""
    from local_kimi_amd.kernels import mxfp4_moe_block, w4a16_moe_forward

    inter = 256
    bank = _mx_bank if weights == "mxfp4" else _w4_bank
    banks = (*bank(rng, routed + 1, inter, h), *bank(rng, routed + 1, inter, h),
             *bank(rng, routed + 1, h, inter))
    x = random_bf16_bits(rng, (tokens, h))
    logits = rng.normal(0, 1, (tokens, routed)).astype(np.float32)
    logits[::5, 3:9] = logits[::5, 3:4]  # tied choices
    b = rng.normal(0, 0.05, routed).astype(np.float32) if bias else None
    args = (_dev(x), _dev(logits), None if b is None else _dev(b), *(_dev(v) for v in banks),
            top_k, 2.446)
    block = mxfp4_moe_block if weights == "mxfp4" else w4a16_moe_forward
    (y, idx, w), (y0, idx0, w0) = _fused_and_split(monkeypatch, block, *args)
    assert torch.equal(idx, idx0)
    assert torch.equal(w, w0)
    assert torch.equal(y, y0), "the ranking gate/up GEMM and the separate launches differ"
    eidx, ew = OM.route(logits, b, top_k, routed_scaling_factor=2.446)
    assert np.array_equal(idx.cpu().numpy(), eidx)
    sel = np.arange(0, tokens, 3)
    if weights == "mxfp4":
        ey, _, _ = X.moe_block(x[sel], logits[sel], b, *banks, top_k=top_k,
                               routed_scaling_factor=2.446)
    else:
        ey, _, _ = OM.moe_block(x[sel], logits[sel], b, *banks, top_k=top_k,
                                routed_scaling_factor=2.446, group_size=128)
    assert_close_bf16(to_bits(y)[sel], ey,
                      what=f"{weights} ranking gate/up T={tokens} k={top_k} E={routed}")


@pytest.mark.parametrize("tokens", [4, 12])
def test_gate_up_gemm_that_routes_under_graph_replay(rng, tokens):
    """The same launch captured in a HIP graph and replayed with new logits
    copied in between: every replay matches an eager call on those logits
    (4 tokens: the gate/up GEMM routes and the token-major W2 launch follows;
    12: the router launch selects, the gate/up GEMM ranks, and the split
    SwiGLU's down GEMM reads the schedule that the gate/up launch wrote)."""
    from local_kimi_amd.kernels import w4a16_moe_forward

    top_k, routed, h, inter = 8, 256, 512, 256
    banks = [_dev(v) for v in (*_w4_bank(rng, routed + 1, inter, h),
                               *_w4_bank(rng, routed + 1, inter, h),
                               *_w4_bank(rng, routed + 1, h, inter))]
    x = _dev(random_bf16_bits(rng, (tokens, h)))
    logits = _dev(rng.normal(0, 1, (tokens, routed)).astype(np.float32))
    w4a16_moe_forward(x, logits, None, *banks, top_k, 2.446)  # allocations outside the graph
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        out = w4a16_moe_forward(x, logits, None, *banks, top_k, 2.446)
    torch.cuda.synchronize()
    for _ in range(4):
        fresh = _dev(rng.normal(0, 1, (tokens, routed)).astype(np.float32))
        logits.copy_(fresh)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = w4a16_moe_forward(x, fresh, None, *banks, top_k, 2.446)
        torch.cuda.synchronize()
        for a, e in zip(out, want):
            assert torch.equal(a, e)
