"""GPU parity of the persistent 16-row expert GEMM (decode batches).

The persistent kernel and the per-tile streaming kernel (path knob moe_persist=off)
perform the same MFMA chains in the same order, so their outputs must be
bit-identical; the per-tile kernel is itself checked against the oracle
elsewhere, and every case here is also checked against the oracle within the
quantized-matmul tolerance (1e-2 relative / 2e-2 absolute in bf16). Shapes
are chosen to reach every ring depth (6 k-steps for k = 768, 8 for k = 1024,
4 for k = 512), both weight formats, routes outside the bank, and a tile list
longer than the grid, where one block covers more tiles than its two LDS
buffers and stages them in phases.
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


def _both(monkeypatch, fn, *args):
    """fn(*args) with the persistent kernel, then with the per-tile kernel."""
    from local_kimi_amd._lib import forced_path

    with forced_path("moe_gemm", "auto"):
        a = fn(*args)
        torch.cuda.synchronize()
        with forced_path("moe_persist", "off"):
            b = fn(*args)
            torch.cuda.synchronize()
    return a, b


@pytest.mark.parametrize("weights", ["w4a16", "mxfp4"])
@pytest.mark.parametrize("h,inter,tokens", [(768, 512, 40), (512, 768, 13), (1024, 512, 21)])
def test_moe_block_persistent_matches_per_tile_and_oracle(rng, monkeypatch, weights, h, inter,
                                                          tokens):
    from local_kimi_amd.kernels import mxfp4_moe_block, w4a16_moe_forward

    e_routed, k = 24, 4
    bank = _mx_bank if weights == "mxfp4" else _w4_bank
    banks = (*bank(rng, e_routed + 1, inter, h), *bank(rng, e_routed + 1, inter, h),
             *bank(rng, e_routed + 1, h, inter))
    x = random_bf16_bits(rng, (tokens, h))
    logits = rng.normal(0, 1, (tokens, e_routed)).astype(np.float32)
    args = (_dev(x), _dev(logits), None, *(_dev(b) for b in banks), k, 2.446)
    block = mxfp4_moe_block if weights == "mxfp4" else w4a16_moe_forward
    (y, idx, _), (y0, idx0, _) = _both(monkeypatch, block, *args)
    assert torch.equal(idx, idx0)
    assert torch.equal(y, y0), "persistent and per-tile kernels differ"
    if weights == "mxfp4":
        ey, eidx, _ = X.moe_block(x, logits, None, *banks, top_k=k, routed_scaling_factor=2.446)
    else:
        ey, eidx, _ = OM.moe_block(x, logits, None, *banks, top_k=k, routed_scaling_factor=2.446,
                                   group_size=128)
    assert np.array_equal(idx.cpu().numpy(), eidx)
    assert_close_bf16(to_bits(y), ey, what=f"{weights} moe block h={h} i={inter} T={tokens}")


@pytest.mark.parametrize("weights", ["w4a16", "mxfp4"])
def test_grouped_gemms_persistent_with_routes_outside_the_bank(rng, monkeypatch, weights):
    from local_kimi_amd.kernels import (grouped_mxfp4_gemm, grouped_mxfp4_swiglu_gemm,
                                        grouped_w4a16_gemm, grouped_w4a16_swiglu_gemm)

    t, r, e, n, k = 40, 3, 6, 96, 512
    x = random_bf16_bits(rng, (t, k))
    idx = rng.integers(0, e, (t, r)).astype(np.int64)
    idx[3, 1] = -1
    idx[7, 0] = e + 2
    bad = (idx < 0) | (idx >= e)
    safe = np.where(bad, 0, idx)
    if weights == "mxfp4":
        p, s = _mx_bank(rng, e, n, k)
        p3, s3 = _mx_bank(rng, e, n, k)
        gemm, swiglu = grouped_mxfp4_gemm, grouped_mxfp4_swiglu_gemm
        want_g, want_s = X.grouped(x, safe, p, s), X.swiglu(x, safe, p, s, p3, s3)
    else:
        p, s = _w4_bank(rng, e, n, k)
        p3, s3 = _w4_bank(rng, e, n, k)
        gemm, swiglu = grouped_w4a16_gemm, grouped_w4a16_swiglu_gemm
        want_g, want_s = OW.grouped(x, safe, p, s, 128), OW.swiglu(x, safe, p, s, p3, s3, 128)
    want_g[bad] = 0
    want_s[bad] = 0
    dx, didx = _dev(x), _dev(idx)
    out, out0 = _both(monkeypatch, gemm, dx, didx, _dev(p), _dev(s))
    assert torch.equal(out, out0)
    assert_close_bf16(to_bits(out), want_g, what=f"{weights} grouped gemm")
    assert not to_bits(out)[bad].any()
    act, act0 = _both(monkeypatch, swiglu, dx, didx, _dev(p), _dev(s), _dev(p3), _dev(s3))
    assert torch.equal(act, act0)
    assert_close_bf16(to_bits(act), want_s, what=f"{weights} swiglu gemm")


def _gpu_w4_bank(gen, e, n, k, g=128):
    from local_kimi_amd.quant import quantise

    packed = torch.empty((e, n, k // 2), dtype=torch.uint8, device=DEV)
    scales = torch.empty((e, n, k // g), dtype=torch.bfloat16, device=DEV)
    for j in range(e):
        enc = quantise((torch.randn(n, k, device=DEV, generator=gen) * 0.02).to(torch.bfloat16),
                       group_size=g)
        packed[j].copy_(enc.packed)
        scales[j].copy_(enc.scales)
    return packed, scales


def test_moe_block_persistent_in_phases(rng, monkeypatch):
    """255 routed experts, 220 tokens x 9 routes: about 380 16-row tiles for a
    grid of one block per CU, so blocks cover three tiles and stage them in two
    phases."""
    from local_kimi_amd.kernels import w4a16_moe_forward
    from local_kimi_amd.workloads import normal_router_logits

    e_routed, h, inter, tokens, k = 255, 512, 512, 220, 8
    gen = torch.Generator(device=DEV).manual_seed(20260801)
    banks = (*_gpu_w4_bank(gen, e_routed + 1, inter, h), *_gpu_w4_bank(gen, e_routed + 1, inter, h),
             *_gpu_w4_bank(gen, e_routed + 1, h, inter))
    x = random_bf16_bits(rng, (tokens, h))
    logits = normal_router_logits(rng, tokens, e_routed)
    args = (_dev(x), _dev(logits), None, *banks, k, 2.446)
    (y, idx, w), (y0, idx0, _) = _both(monkeypatch, w4a16_moe_forward, *args)
    assert torch.equal(idx, idx0)
    assert torch.equal(y, y0), "persistent and per-tile kernels differ"
    # oracle on a few tokens, with only the experts they route to
    sel = np.array([0, 57, 131, 219])
    eidx, ew = OM.route(logits[sel], None, k, routed_scaling_factor=2.446)
    assert np.array_equal(idx.cpu().numpy()[sel], eidx)
    used = sorted(set(eidx.reshape(-1).tolist()) | {e_routed})
    remap = {e: j for j, e in enumerate(used)}
    sub = [b[used].cpu().numpy() if b.dtype == torch.uint8 else to_bits(b[used]) for b in banks]
    stable = np.array([[remap[e] for e in row] + [remap[e_routed]] for row in eidx.tolist()])
    act = OW.swiglu(x[sel], stable, sub[0], sub[1], sub[2], sub[3], 128)
    cw = np.concatenate((ew, np.ones((len(sel), 1), np.float32)), 1)
    ey = OM.w2_combine(act, stable, cw, sub[4], sub[5], 128)
    assert_close_bf16(to_bits(y)[sel], ey, what="moe block in phases")


def test_persistent_block_under_graph_replay(rng):
    from local_kimi_amd.kernels import w4a16_moe_forward

    e_routed, h, inter, tokens = 8, 768, 512, 24
    banks = (*_w4_bank(rng, e_routed + 1, inter, h), *_w4_bank(rng, e_routed + 1, inter, h),
             *_w4_bank(rng, e_routed + 1, h, inter))
    x = random_bf16_bits(rng, (tokens, h))
    logits = rng.normal(0, 1, (tokens, e_routed)).astype(np.float32)
    dev = [_dev(b) for b in banks]
    xd, ld = _dev(x), _dev(logits)
    eager, eidx, _ = w4a16_moe_forward(xd, ld, None, *dev, 4, 2.446)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        w4a16_moe_forward(xd, ld, None, *dev, 4, 2.446)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gy, gidx, _ = w4a16_moe_forward(xd, ld, None, *dev, 4, 2.446)
    for _ in range(4):
        gy.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gy, eager)
        assert torch.equal(gidx, eidx)


@pytest.mark.parametrize("weights,tokens", [("w4a16", 16), ("w4a16", 64), ("w4a16", 150),
                                            ("mxfp4", 64)])
def test_split_swiglu_matches_the_fused_epilogue(rng, weights, tokens):
    """The Kimi-Linear layer (hidden 2304, intermediate 1024, 256 routed
    experts + shared, top-8): split gate/up units with the SwiGLU in the down
    GEMM's staging against the fused gate/up epilogue (path knob
    moe_split_swiglu=off), bit-identical, and the oracle on three tokens."""
    from local_kimi_amd._lib import forced_path
    from local_kimi_amd.kernels import mxfp4_moe_block, w4a16_moe_forward
    from local_kimi_amd.quant import quantize_mxfp4
    from local_kimi_amd.workloads import zipf_router_logits

    e_routed, h, inter, k = 256, 2304, 1024, 8
    gen = torch.Generator(device=DEV).manual_seed(20260802 + tokens)
    if weights == "w4a16":
        banks = (*_gpu_w4_bank(gen, e_routed + 1, inter, h),
                 *_gpu_w4_bank(gen, e_routed + 1, inter, h),
                 *_gpu_w4_bank(gen, e_routed + 1, h, inter))
        block = w4a16_moe_forward
    else:
        def mx_bank(n, kk):
            enc = [quantize_mxfp4((torch.randn(n, kk, device=DEV, generator=gen) * 0.02)
                                  .to(torch.bfloat16)) for _ in range(e_routed + 1)]
            return torch.stack([p for p, _ in enc]), torch.stack([q for _, q in enc])
        banks = (*mx_bank(inter, h), *mx_bank(inter, h), *mx_bank(h, inter))
        block = mxfp4_moe_block
    x = random_bf16_bits(rng, (tokens, h))
    logits = zipf_router_logits(rng, tokens, e_routed)
    args = (_dev(x), _dev(logits), None, *banks, k, 2.446)
    with forced_path("moe_gemm", "auto"):
        y, idx, w = block(*args)
        torch.cuda.synchronize()
        with forced_path("moe_split_swiglu", "off"):
            y0, idx0, w0 = block(*args)
            torch.cuda.synchronize()
    assert torch.equal(idx, idx0) and torch.equal(w, w0)
    assert torch.equal(y, y0), "split and fused SwiGLU forms differ"
    # oracle on three tokens, with only the experts they route to
    sel = np.array([0, tokens // 2, tokens - 1])
    eidx, ew = OM.route(logits[sel], None, k, routed_scaling_factor=2.446)
    assert np.array_equal(idx.cpu().numpy()[sel], eidx)
    used = sorted(set(eidx.reshape(-1).tolist()) | {e_routed})
    remap = {e: j for j, e in enumerate(used)}
    stable = np.array([[remap[e] for e in row] + [remap[e_routed]] for row in eidx.tolist()])
    sub = [b[used].cpu().numpy() if b.dtype == torch.uint8 else to_bits(b[used]) for b in banks]
    cw = np.concatenate((ew, np.ones((len(sel), 1), np.float32)), 1)
    if weights == "w4a16":
        act = OW.swiglu(x[sel], stable, sub[0], sub[1], sub[2], sub[3], 128)
        ey = OM.w2_combine(act, stable, cw, sub[4], sub[5], 128)
    else:
        act = X.swiglu(x[sel], stable, sub[0], sub[1], sub[2], sub[3])
        eo = X.grouped(act.reshape(len(sel) * (k + 1), -1), stable.reshape(-1, 1), sub[4], sub[5])
        ey = OM.combine(eo.reshape(len(sel), k + 1, -1), cw)
    assert_close_bf16(to_bits(y)[sel], ey, what=f"{weights} split SwiGLU T={tokens}")
