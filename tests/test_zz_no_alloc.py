"""The allocation-free MoE block entry point, lk_w4a16_moe_forward_static,
against lk_w4a16_moe_forward (workspace from the caller) on the same inputs,
both called through the C ABI: outputs, selections and combine weights must be
bit-identical (the same kernels on the same tables). Two calls in a row, the
second smaller, so the second runs on scratch the first left behind; then a
decode-sized call (the token-major W2 tail) and a call past the scratch size,
which is refused before any launch."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from local_kimi_amd import _lib

from ._helpers import random_bf16_bits

pytestmark = pytest.mark.gpu

DEV = "cuda"
H, INTER, ROUTED, TOP_K, G = 2304, 1024, 256, 8, 128


@pytest.fixture(scope="module")
def banks():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from local_kimi_amd.quant import quantise

    _lib.load()
    gen = torch.Generator(device=DEV).manual_seed(20260807)

    def bank(n, k):
        packed = torch.empty((ROUTED + 1, n, k // 2), dtype=torch.uint8, device=DEV)
        scales = torch.empty((ROUTED + 1, n, k // G), dtype=torch.bfloat16, device=DEV)
        for e in range(ROUTED + 1):
            enc = quantise((torch.randn(n, k, device=DEV, generator=gen) * 0.02)
                           .to(torch.bfloat16), group_size=G)
            packed[e].copy_(enc.packed)
            scales[e].copy_(enc.scales)
        return packed, scales

    return (*bank(INTER, H), *bank(INTER, H), *bank(H, INTER))


def _inputs(rng, tokens):
    from local_kimi_amd.workloads import zipf_router_logits

    x = torch.from_numpy(random_bf16_bits(rng, (tokens, H)).view(np.int16)).view(torch.bfloat16)
    logits = torch.from_numpy(zipf_router_logits(rng, tokens, ROUTED))
    return x.to(DEV), logits.to(DEV)


def _run(static: bool, x, logits, banks):
    tokens = x.shape[0]
    y = torch.full((tokens, H), float("nan"), dtype=torch.bfloat16, device=DEV)
    idx = torch.full((tokens, TOP_K), -5, dtype=torch.long, device=DEV)
    w = torch.full((tokens, TOP_K), float("nan"), dtype=torch.float32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    ptrs = [b.data_ptr() for b in banks]
    tail = (tokens, ROUTED + 1, H, INTER, TOP_K, 2.446, 1, G, stream)
    if static:
        _lib.call("lk_w4a16_moe_forward_static", x.data_ptr(), logits.data_ptr(), None, *ptrs,
                  y.data_ptr(), idx.data_ptr(), w.data_ptr(), *tail)
    else:
        nbytes = _lib.query("lk_w4a16_moe_forward_workspace", tokens, ROUTED + 1, H, INTER, TOP_K)
        ws = torch.empty((nbytes,), dtype=torch.uint8, device=DEV)
        _lib.call("lk_w4a16_moe_forward", x.data_ptr(), logits.data_ptr(), None, *ptrs,
                  y.data_ptr(), idx.data_ptr(), w.data_ptr(), ws.data_ptr(), nbytes, *tail)
    torch.cuda.synchronize()
    return y, idx, w


def test_static_scratch_matches_the_workspace_entry_point(banks):
    rng = np.random.default_rng(20260808)
    for tokens in (128, 37, 4, 1):  # each call smaller than the one before
        x, logits = _inputs(rng, tokens)
        want = _run(False, x, logits, banks)
        got = _run(True, x, logits, banks)
        for a, b, name in zip(got, want, ("y", "expert indices", "weights")):
            assert torch.equal(a, b), f"{name} differ at {tokens} tokens"
        assert torch.isfinite(got[0].float()).all()


def test_static_scratch_refuses_calls_past_its_size(banks):
    cap = _lib.query("lk_w4a16_moe_forward_static_capacity")
    too_many = 161
    assert _lib.query("lk_w4a16_moe_forward_workspace", too_many, ROUTED + 1, H, INTER,
                      TOP_K) > cap
    x, logits = _inputs(np.random.default_rng(1), too_many)
    with pytest.raises(RuntimeError, match="static scratch holds"):
        _run(True, x, logits, banks)
