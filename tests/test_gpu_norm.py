"""GPU parity of the decode norm kernels (local_kimi_amd/csrc/norm.hip) with oracle/norm.py.

Tolerance, stated once for every test here: within two units in the last
place of the input dtype (four for fp32) of the oracle, the bound at which
the oracle itself agrees with torch's CPU evaluation of the reference
expressions (tests/test_oracle_norm.py): the kernel's fp32 mean square is
summed in another order than the oracle's, which can flip the rounding of a
normalised value. The gated norm in fp32 end to end allows eight: the
kernel's fp32 exp in the sigmoid (an ulp or two against the oracle's
correctly rounded one) adds to the chain. That is far inside the path's 1e-2
relative / 2e-2 absolute bar, which every result is also checked against. The residual sums
are bit-exact; reruns are bit-identical; graph replays equal eager calls.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import norm as N
from oracle.kda import round_to

pytestmark = pytest.mark.gpu

DEV = "cuda"
_NAMES = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}


@pytest.fixture(scope="module", autouse=True)
def _require_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from local_kimi_amd import _lib

    _lib.load()


def _rand(rng, shape, dtype, std=1.0, mean=0.0):
    vals = round_to(mean + std * rng.normal(size=shape), _NAMES[dtype])
    return torch.from_numpy(vals).to(DEV, dtype), vals


def _ulp(values, dtype_name):
    bits = {"bfloat16": 8, "float16": 11, "float32": 24}[dtype_name]
    mag = np.maximum(np.abs(values), np.finfo(np.float32).tiny)
    return 2.0 ** (np.floor(np.log2(mag)) - (bits - 1))


def _check(got: torch.Tensor, want: np.ndarray, in_dtype_name: str, what: str, fp32_ulps=4):
    g = got.detach().double().cpu().numpy()
    assert g.shape == want.shape, (what, g.shape, want.shape)
    assert np.isfinite(g).all(), what
    k = fp32_ulps if in_dtype_name == "float32" else 2
    err = np.abs(g - want)
    bad = err > k * _ulp(want, in_dtype_name)
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond {k} ulps, worst {err.max():.3g}"
    assert np.all(err <= 2e-2 + 1e-2 * np.abs(want)), what


WIDTHS = [8, 120, 128, 136, 2304, 4096, 8192]


@pytest.mark.parametrize("width", WIDTHS)
@pytest.mark.parametrize("rows", [1, 7, 2048])
def test_rms_norm_matches_oracle(rng, rows, width):
    from local_kimi_amd.kernels import rms_norm

    if rows * width > 2048 * 2304:
        rows = 2048 * 2304 // width
    x, xv = _rand(rng, (rows, width), torch.bfloat16)
    w, wv = _rand(rng, (width,), torch.bfloat16, 0.1, 1.0)
    got = rms_norm(x, w, 1e-6)
    assert got.dtype == torch.bfloat16
    _check(got, N.rms_norm(xv, wv, 1e-6, "bfloat16", "bfloat16"), "bfloat16", f"{rows}x{width}")
    assert torch.equal(got, rms_norm(x, w, 1e-6))


@pytest.mark.parametrize("xd,wd", [(torch.float16, torch.float16), (torch.float32, torch.float32),
                                   (torch.bfloat16, torch.float32), (torch.float16, torch.bfloat16),
                                   (torch.float32, torch.bfloat16)])
def test_rms_norm_dtypes_follow_torch_promotion(rng, xd, wd):
    from local_kimi_amd.kernels import rms_norm

    x, xv = _rand(rng, (3, 5, 2304), xd)
    w, wv = _rand(rng, (2304,), wd, 0.1, 1.0)
    got = rms_norm(x, w, 1e-5)
    assert got.dtype == (xd if xd == wd else torch.float32) and got.shape == x.shape
    want = N.rms_norm(xv, wv, 1e-5, _NAMES[xd], _NAMES[wd])
    _check(got, want, _NAMES[xd], f"{xd}/{wd}")


def test_rms_norm_zero_rows_and_eps(rng):
    from local_kimi_amd.kernels import rms_norm

    w, _ = _rand(rng, (256,), torch.bfloat16, 0.1, 1.0)
    out = rms_norm(torch.zeros((4, 256), dtype=torch.bfloat16, device=DEV), w, 1e-6)
    assert torch.equal(out, torch.zeros_like(out))
    assert rms_norm(torch.zeros((0, 256), dtype=torch.bfloat16, device=DEV), w, 1e-6).shape == (0, 256)


def test_rms_norm_hand_computed_rounding_case():
    """width 2, x = [1, 0], weight 1.046875: 1.4765625 (the oracle's KAT)."""
    from local_kimi_amd.kernels import rms_norm

    x = torch.tensor([[1.0, 0, 0, 0, 0, 0, 0, 0]], dtype=torch.bfloat16, device=DEV)
    w = torch.tensor([1.046875] + [1.0] * 7, dtype=torch.bfloat16, device=DEV)
    # width 8, one-hot: n = bf16(sqrt 8) = 2.828125; w * n = 2.96069... -> 2.953125
    got = rms_norm(x, w, 0.0).float().cpu().numpy()
    assert got[0, 0] == 2.953125 and not got[0, 1:].any()


@pytest.mark.parametrize("rows,width", [(1, 2304), (64, 2304), (2048, 2304), (5, 128)])
def test_add_rms_norm_matches_oracle(rng, rows, width):
    from local_kimi_amd.kernels import add_rms_norm

    r, rv = _rand(rng, (rows, width), torch.bfloat16)
    d, dv = _rand(rng, (rows, width), torch.bfloat16, 4.0)
    w, wv = _rand(rng, (width,), torch.bfloat16, 0.1, 1.0)
    hidden, normed = add_rms_norm(r, d, w, 1e-6)
    want_h, want = N.add_rms_norm(rv, dv, wv, 1e-6, "bfloat16", "bfloat16")
    assert np.array_equal(hidden.double().cpu().numpy(), want_h)
    _check(normed, want, "bfloat16", f"add {rows}x{width}")


def test_add_rms_norm_in_place_sum_through_the_c_abi(rng):
    """sum_out may alias the residual (the residual stream updated in place)."""
    from local_kimi_amd import _lib

    r, rv = _rand(rng, (3, 2304), torch.bfloat16)
    d, dv = _rand(rng, (3, 2304), torch.bfloat16)
    w, wv = _rand(rng, (2304,), torch.bfloat16, 0.1, 1.0)
    y = torch.empty_like(r)
    _lib.call("lk_add_rms_norm", r.data_ptr(), d.data_ptr(), w.data_ptr(), r.data_ptr(),
              y.data_ptr(), 3, 2304, 1e-6, 2, 2, torch.cuda.current_stream().cuda_stream)
    want_h, want = N.add_rms_norm(rv, dv, wv, 1e-6, "bfloat16", "bfloat16")
    assert np.array_equal(r.double().cpu().numpy(), want_h)
    _check(y, want, "bfloat16", "in place")


@pytest.mark.parametrize("vd,ind,gd,wd", [
    (torch.bfloat16, torch.bfloat16, torch.bfloat16, torch.bfloat16),
    (torch.float32, torch.bfloat16, torch.bfloat16, torch.bfloat16),
    (torch.float32, torch.float32, torch.float32, torch.float32),
    (torch.bfloat16, torch.bfloat16, torch.float32, torch.float32),
    (torch.float16, torch.float16, torch.float16, torch.float16)])
@pytest.mark.parametrize("shape", [(1, 1, 32, 128), (2, 3, 32, 128), (7, 72), (4, 2304)])
def test_rms_gated_norm_matches_oracle(rng, vd, ind, gd, wd, shape):
    from local_kimi_amd.kernels import rms_gated_norm

    v, vv = _rand(rng, shape, vd)
    g, gv = _rand(rng, shape, gd, 2.0)
    w, wv = _rand(rng, shape[-1:], wd, 0.1, 1.0)
    got = rms_gated_norm(v, g, w, 1e-5, input_dtype=ind)
    assert got.dtype == ind
    want = N.rms_gated_norm(vv, gv, wv, 1e-5, _NAMES[ind])
    _check(got, want, _NAMES[ind], f"gated {shape} {vd}/{ind}/{gd}/{wd}", fp32_ulps=8)
    assert torch.equal(got, rms_gated_norm(v, g, w, 1e-5, input_dtype=ind))


def test_modules_and_the_layer_tail(rng):
    """RMSNorm / RMSGatedNorm modules equal the functions; MoELayerTail equals
    add + norm + MoE + add (+ the next layer's norm) composed from the ops."""
    from local_kimi_amd.checkpoint import MoeBanks
    from local_kimi_amd.kernels import add_rms_norm, rms_norm, w4a16_moe_block
    from local_kimi_amd.klinear import KLinearMoE, MoELayerTail, RMSGatedNorm, RMSNorm
    from local_kimi_amd.quant import quantise

    h, inter, experts = 512, 256, 8
    ln = RMSNorm(h, 1e-5, device=DEV, dtype=torch.bfloat16)
    nxt = RMSNorm(h, 1e-5, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        ln.weight.copy_(_rand(rng, (h,), torch.bfloat16, 0.1, 1.0)[0])
        nxt.weight.copy_(_rand(rng, (h,), torch.bfloat16, 0.1, 1.0)[0])
    x, _ = _rand(rng, (2, h), torch.bfloat16)
    assert torch.equal(ln(x), rms_norm(x, ln.weight.detach(), 1e-5))
    gn = RMSGatedNorm(128, device=DEV, dtype=torch.bfloat16)
    v, _ = _rand(rng, (2, 128), torch.float32)
    gate, _ = _rand(rng, (2, 128), torch.bfloat16)
    assert gn(v, gate, torch.bfloat16).dtype == torch.bfloat16

    def bank(n, k):
        encs = [quantise((torch.randn(n, k, device=DEV) * 0.02).bfloat16(), group_size=128)
                for _ in range(experts + 1)]
        return torch.stack([e.packed for e in encs]), torch.stack([e.scales for e in encs])

    banks = MoeBanks(*bank(inter, h), *bank(inter, h), *bank(h, inter))
    gate_w = (torch.randn(experts, h, device=DEV) * 0.05).bfloat16()
    moe = KLinearMoE(gate_w, None, banks, top_k=2, routed_scaling_factor=2.446)
    tail = MoELayerTail(moe, ln)
    attended, _ = _rand(rng, (2, h), torch.bfloat16)
    hidden, ff_in = add_rms_norm(x, attended, ln.weight.detach(), 1e-5)
    ff = moe(ff_in)
    assert torch.equal(tail(x, attended), hidden + ff)
    got_h, got_n = tail(x, attended, nxt)
    want_h, want_n = add_rms_norm(hidden, ff, nxt.weight.detach(), 1e-5)
    assert torch.equal(got_h, want_h) and torch.equal(got_n, want_n)
    assert torch.equal(moe(ff_in), w4a16_moe_block(ff_in, moe.router_logits(ff_in), None,
                                                   *banks.as_tuple(), 2, 2.446)[0])


def test_graph_replays_match_eager(rng):
    from local_kimi_amd.kernels import add_rms_norm, rms_gated_norm

    r, _ = _rand(rng, (1, 2304), torch.bfloat16)
    d, _ = _rand(rng, (1, 2304), torch.bfloat16)
    w, _ = _rand(rng, (2304,), torch.bfloat16, 0.1, 1.0)
    v, _ = _rand(rng, (1, 32, 128), torch.float32)
    g, _ = _rand(rng, (1, 32, 128), torch.bfloat16)
    gw, _ = _rand(rng, (128,), torch.bfloat16, 0.1, 1.0)
    eager = (*add_rms_norm(r, d, w, 1e-6), rms_gated_norm(v, g, gw, 1e-5, input_dtype=torch.bfloat16))
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        add_rms_norm(r, d, w, 1e-6)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = (*add_rms_norm(r, d, w, 1e-6), rms_gated_norm(v, g, gw, 1e-5,
                                                            input_dtype=torch.bfloat16))
    for rep in range(3):
        for t in out:
            t.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(out, eager):
            assert torch.equal(a, b), rep
        _ = (r.float() * 2).sum().item()  # unrelated eager work between replays
