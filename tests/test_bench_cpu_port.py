"""The CPU baseline of bench.py is a torch restatement of the reference path
(dequantise, F.linear, bf16 SwiGLU, fp32 combine + shared expert). It is what
the GPU numbers are compared with, so it must compute the same block as the
oracle: decoders bit-exact, block outputs within the quantized-matmul
tolerance (1e-2 relative / 2e-2 absolute in bf16)."""

from __future__ import annotations

import numpy as np
import torch

import bench
from oracle import moe as OM
from oracle import mxfp4 as OX
from oracle import w4a16 as OW
from oracle.bf16 import bf16_bits_to_f32

from ._helpers import assert_close_bf16, random_bf16_bits


def _t(a):
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a))


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_w4a16_dequant_is_bit_exact(rng):
    p, s = OW.quantise(random_bf16_bits(rng, (96, 512), 0.02), 128)
    assert np.array_equal(_bits(bench.cpu_dequant_w4a16(_t(p), _t(s))), OW.dequantise(p, s, 128))


def test_mxfp4_dequant_is_bit_exact(rng):
    p, s = OX.quantize(bf16_bits_to_f32(random_bf16_bits(rng, (64, 256), 0.02)))
    from oracle.bf16 import f32_to_bf16_bits

    want = f32_to_bf16_bits(OX.dequantize(p, s))
    assert np.array_equal(_bits(bench.cpu_dequant_mxfp4(_t(p), _t(s))), want)


def test_block_matches_oracle(rng, monkeypatch):
    e_routed, h, inter, top_k, tokens = 12, 256, 128, 4, 5
    monkeypatch.setattr(bench, "H", h)
    monkeypatch.setattr(bench, "E_ROUTED", e_routed)
    monkeypatch.setattr(bench, "TOP_K", top_k)
    banks = []
    for n, k in ((inter, h), (inter, h), (h, inter)):
        pairs = [OW.quantise(random_bf16_bits(rng, (n, k), 0.02), 128) for _ in range(e_routed + 1)]
        banks += [np.stack([a for a, _ in pairs]), np.stack([b for _, b in pairs])]
    x = random_bf16_bits(rng, (tokens, h))
    logits = rng.normal(0, 1, (tokens, e_routed)).astype(np.float32)
    cpu = bench.CpuMoe([_t(b) for b in banks], "w4a16")
    got = cpu.step(_t(x), _t(logits))
    want, _, _ = OM.moe_block(x, logits, None, *banks, top_k=top_k, routed_scaling_factor=2.446,
                              group_size=128)
    assert_close_bf16(_bits(got), want, what="bench CPU port")
    # a stride sample of the routed experts plus the rest is the same work split differently
    union = torch.unique(bench.cpu_router(_t(logits))[0])
    assert union.numel() > 1
