"""GPU parity of the MXFP4 path against the numpy oracle.

Bit-exact: the codec (quantise against the oracle's OCP encoder, dequantise
against the reference decode in fp32 and bf16). Tolerance (stated here, from
the quantized-matmul contract): bf16 outputs within 1e-2 relative / 2e-2
absolute of the oracle's dequantise-then-linear path; fp16 outputs within the
same bound.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as OM
from oracle import mxfp4 as X
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

from local_kimi_amd._lib import forced_path

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


def _encode(rng, n, k, std=0.02):
    w = random_bf16_bits(rng, (n, k), std)
    return X.quantize(bf16_bits_to_f32(w))


def _bank(rng, e, n, k):
    enc = [_encode(rng, n, k) for _ in range(e)]
    return np.stack([p for p, _ in enc]), np.stack([s for _, s in enc])


# ---------------------------------------------------------------------------
# codec


def test_quantise_is_bit_exact(rng):
    from local_kimi_amd.quant import quantize_mxfp4

    w = random_bf16_bits(rng, (64, 512), 0.02)
    w[0, :32] = 0                                                   # all-zero block -> 127
    w[1, :32] = f32_to_bf16_bits(np.full(32, 1e-39, np.float32))   # subnormal block -> 0
    w[2, :32] = f32_to_bf16_bits(np.full(32, 3e38, np.float32))    # huge block -> 254
    ties = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 4.0] * 4, np.float32)
    ties[1::2] *= -1
    w[3, :32] = f32_to_bf16_bits(ties)                              # amax 5 -> scale 1: grid midpoints
    w[4, :32] = 0x8000                                              # negative zeros
    packed, scale = quantize_mxfp4(_dev(w))
    ep, es = X.quantize(bf16_bits_to_f32(w))
    assert np.array_equal(scale.cpu().numpy(), es)
    assert np.array_equal(packed.cpu().numpy(), ep)


def test_dequantise_is_bit_exact_for_every_code_and_exponent():
    from local_kimi_amd.quant import dequantize_mxfp4

    exps = np.array([0, 1, 100, 120, 127, 128, 200, 253, 254, 255], np.uint8)
    packed = np.tile(np.arange(256, dtype=np.uint8), (len(exps), 1))        # [10, 256] -> K = 512
    scale = np.repeat(exps[:, None], 16, axis=1).astype(np.uint8)
    want = X.dequantize(packed, scale)
    got = dequantize_mxfp4(_dev(packed), _dev(scale)).cpu().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    got16 = to_bits(dequantize_mxfp4(_dev(packed), _dev(scale), dtype=torch.bfloat16))
    want16 = f32_to_bf16_bits(want)
    assert np.array_equal(got16[~nan], want16[~nan])


# ---------------------------------------------------------------------------
# GEMM


@pytest.mark.parametrize("form", ["default", "lds"])  # streaming 64-row kernel / LDS-staged GEMM
@pytest.mark.parametrize("m,n,k", [(1, 96, 256), (16, 64, 512), (64, 2048, 2304), (100, 200, 1024),
                                   (37, 48, 96)])
def test_gemm_matches_oracle(rng, monkeypatch, m, n, k, form):
    from local_kimi_amd.kernels import mxfp4_gemm, mxfp4_gemm_reference

    p, s = _encode(rng, n, k)
    x = random_bf16_bits(rng, (m, k))
    want = X.linear(x, p, s)
    with forced_path("dense_gemm", "lds" if form == "lds" else "auto"):
        y = mxfp4_gemm(_dev(x), _dev(p), _dev(s))
        again = mxfp4_gemm(_dev(x), _dev(p), _dev(s))
    assert_close_bf16(to_bits(y), want, what=f"mxfp4 gemm {m}x{n}x{k}")
    assert torch.equal(y, again)
    yr = mxfp4_gemm_reference(_dev(x), _dev(p), _dev(s))
    assert_close_bf16(to_bits(yr), want, what="mxfp4 reference variant")


def test_gemm_across_scale_exponents(rng):
    """Blocks spread over E8M0 exponents 20..230: the scaled decode stays exact."""
    from local_kimi_amd.kernels import mxfp4_gemm

    n, k, m = 64, 1024, 32
    codes = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scale = rng.choice(np.array([20, 60, 100, 120, 127, 140, 160, 200, 230], np.uint8),
                       size=(n, k // 32)).astype(np.uint8)
    x = random_bf16_bits(rng, (m, k))
    want = X.linear(x, codes, scale)
    got = to_bits(mxfp4_gemm(_dev(x), _dev(codes), _dev(scale)))
    # compare relative to each row's magnitude (outputs span many binades)
    a = bf16_bits_to_f32(got).astype(np.float64)
    e = bf16_bits_to_f32(want).astype(np.float64)
    mag = np.abs(e).max(axis=1, keepdims=True)
    assert np.all(np.abs(a - e) <= 2e-2 * mag + 1e-2 * np.abs(e))


@pytest.mark.parametrize("form", ["default", "lds"])
@pytest.mark.parametrize("m", [1, 64])
def test_gemm_fp16_activations(rng, monkeypatch, m, form):
    from local_kimi_amd.kernels import mxfp4_gemm

    n, k = 128, 1024
    p, s = _encode(rng, n, k)
    xf = rng.normal(0, 1, (m, k)).astype(np.float16)
    with forced_path("dense_gemm", "lds" if form == "lds" else "auto"):
        y = mxfp4_gemm(torch.from_numpy(xf).to(DEV), _dev(p), _dev(s))
    assert y.dtype == torch.float16
    got = y.cpu().numpy().astype(np.float64)
    want = X.linear_f16(xf.view(np.uint16), p, s).view(np.float16).astype(np.float64)
    assert np.all(np.abs(got - want) <= 2e-2 + 1e-2 * np.abs(want))


def test_gemm_validation_messages():
    from local_kimi_amd.kernels import mxfp4_gemm

    x = torch.zeros((2, 64), dtype=torch.float32, device=DEV)
    p = torch.zeros((8, 32), dtype=torch.uint8, device=DEV)
    s = torch.zeros((8, 2), dtype=torch.uint8, device=DEV)
    with pytest.raises(TypeError, match="float16 or torch.bfloat16"):
        mxfp4_gemm(x, p, s)
    with pytest.raises(ValueError, match="one byte per 32"):
        mxfp4_gemm(x.bfloat16(), p, s[:, :1])


# ---------------------------------------------------------------------------
# grouped, MoE block, expert MLP


@pytest.mark.parametrize("k", [256, 160])  # 16-byte (k % 128 == 0) and 4-byte weight loads
def test_grouped_and_swiglu_gemm_match_oracle(rng, k):
    from local_kimi_amd.kernels import grouped_mxfp4_gemm, grouped_mxfp4_swiglu_gemm

    t, r, e, n = 40, 3, 6, 96
    x = random_bf16_bits(rng, (t, k))
    idx = rng.integers(0, e, (t, r)).astype(np.int64)
    idx[5, 2] = -1
    bad = idx < 0
    safe = np.where(bad, 0, idx)
    p, s = _bank(rng, e, n, k)
    out = to_bits(grouped_mxfp4_gemm(_dev(x), _dev(idx), _dev(p), _dev(s)))
    want = X.grouped(x, safe, p, s)
    want[bad] = 0
    assert_close_bf16(out, want, what="mxfp4 grouped")
    p3, s3 = _bank(rng, e, n, k)
    act = to_bits(grouped_mxfp4_swiglu_gemm(_dev(x), _dev(idx), _dev(p), _dev(s), _dev(p3),
                                            _dev(s3)))
    want = X.swiglu(x, safe, p, s, p3, s3)
    want[bad] = 0
    assert_close_bf16(act, want, what="mxfp4 swiglu")


@pytest.mark.parametrize("tokens", [1, 6, 33])
def test_moe_block_matches_oracle_small_bank(rng, tokens):
    from local_kimi_amd.kernels import mxfp4_moe_block, mxfp4_moe_block_reference

    e_routed, h, inter, k = 16, 512, 256, 4
    banks = (*_bank(rng, e_routed + 1, inter, h), *_bank(rng, e_routed + 1, inter, h),
             *_bank(rng, e_routed + 1, h, inter))
    x = random_bf16_bits(rng, (tokens, h))
    logits = rng.normal(0, 1, (tokens, e_routed)).astype(np.float32)
    ey, eidx, ew = X.moe_block(x, logits, None, *banks, top_k=k, routed_scaling_factor=2.446)
    args = (_dev(x), _dev(logits), None, *(_dev(b) for b in banks), k, 2.446)
    y, idx, w = mxfp4_moe_block(*args)
    assert np.array_equal(idx.cpu().numpy(), eidx)
    assert_close_bf16(to_bits(y), ey, what=f"mxfp4 moe block T={tokens}")
    yr, idxr, _ = mxfp4_moe_block_reference(*args)
    assert torch.equal(idxr, idx)
    assert_close_bf16(to_bits(yr), ey, what="mxfp4 moe block reference")


@pytest.fixture(scope="module")
def kimi_mx_banks():
    """MXFP4 Kimi-Linear banks: hidden 2304, 256 routed + 1 shared experts,
    intermediate 1024, weights N(0, 0.02) quantised on the GPU."""
    from local_kimi_amd.quant import quantize_mxfp4

    e_total, h, i = 257, 2304, 1024
    gen = torch.Generator(device=DEV).manual_seed(20260732)

    def bank(n, k):
        packed = torch.empty((e_total, n, k // 2), dtype=torch.uint8, device=DEV)
        scale = torch.empty((e_total, n, k // 32), dtype=torch.uint8, device=DEV)
        for e in range(e_total):
            w = (torch.randn(n, k, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
            p, s = quantize_mxfp4(w)
            packed[e].copy_(p)
            scale[e].copy_(s)
        return packed, scale

    return (*bank(i, h), *bank(i, h), *bank(h, i))


@pytest.mark.parametrize("tokens,zipf", [(64, True), (2048, False)])
def test_moe_block_full_size(rng, kimi_mx_banks, tokens, zipf):
    """Batched decode (M=64, Zipf routing) and prefill (2048 tokens) with MXFP4 experts."""
    from local_kimi_amd.kernels import mxfp4_moe_block
    from local_kimi_amd.workloads import normal_router_logits, zipf_router_logits

    x = random_bf16_bits(rng, (tokens, 2304))
    logits = (zipf_router_logits if zipf else normal_router_logits)(rng, tokens, 256)
    y, idx, _ = mxfp4_moe_block(_dev(x), _dev(logits), None, *kimi_mx_banks, 8, 2.446)
    # 64 tokens: every token against the oracle; 2048 tokens: 6 sampled (the
    # designed-bank prefill tests check every token)
    sel = (np.arange(tokens) if tokens <= 64
           else np.unique(rng.choice(tokens, size=6, replace=False)))
    eidx, ew = OM.route(logits[sel], None, 8, routed_scaling_factor=2.446)
    assert np.array_equal(idx.cpu().numpy()[sel], eidx)
    e_total = 257
    used = sorted(set(eidx.reshape(-1).tolist()) | {e_total - 1})
    remap = {e: j for j, e in enumerate(used)}
    sub = [b[used].cpu().numpy() for b in kimi_mx_banks]
    stable = np.array([[remap[e] for e in row] + [remap[e_total - 1]] for row in eidx.tolist()])
    act = X.swiglu(x[sel], stable, sub[0], sub[1], sub[2], sub[3])
    eo = X.grouped(act.reshape(-1, act.shape[-1]), stable.reshape(-1, 1), sub[4],
                   sub[5]).reshape(len(sel), 9, -1)
    cw = np.concatenate((ew, np.ones((len(sel), 1), np.float32)), 1)
    worst = assert_close_bf16(to_bits(y)[sel], OM.combine(eo, cw), what=f"mxfp4 block T={tokens}")
    print(f"mxfp4 block T={tokens}: {sel.size} tokens checked, worst {worst:.3f} of the tolerance")
    assert worst < 0.75


@pytest.mark.parametrize("linear_beta", [25.0, None])
def test_expert_mlp_situ_matches_oracle(rng, linear_beta):
    from types import SimpleNamespace

    from local_kimi_amd.kernels import mxfp4_expert_mlp

    m, h, i = 32, 512, 256
    w1, w3, w2 = _encode(rng, i, h, 0.05), _encode(rng, i, h, 0.05), _encode(rng, h, i, 0.05)
    x = random_bf16_bits(rng, (m, h))
    weights = SimpleNamespace(w1_packed=_dev(w1[0]), w1_scale=_dev(w1[1]), w3_packed=_dev(w3[0]),
                              w3_scale=_dev(w3[1]), w2_packed=_dev(w2[0]), w2_scale=_dev(w2[1]))
    y = mxfp4_expert_mlp(_dev(x), weights, situ_beta=4.0, situ_linear_beta=linear_beta)
    want = X.expert_mlp(x, *w1, *w3, *w2, 4.0, linear_beta)
    assert_close_bf16(to_bits(y), want, what="mxfp4 expert mlp (SiTU)")


@pytest.mark.parametrize("op", ["mxfp4_gemm", "mxfp4_grouped"])
def test_mxfp4_variants_match_the_reference_variant(op):
    from local_kimi_amd.kernels import equivalence

    def make(device):
        g = torch.Generator().manual_seed(20260733)
        k, n, e = 512, 64, 4
        x = torch.randn((5, k), generator=g).to(torch.bfloat16)

        def packed(*shape):
            return torch.randint(0, 256, shape, generator=g, dtype=torch.uint8)

        def scale(*shape):
            return torch.randint(118, 124, shape, generator=g, dtype=torch.uint8)

        if op == "mxfp4_gemm":
            return x, packed(n, k // 2), scale(n, k // 32)
        idx = torch.tensor([[0, 3], [2, 2], [1, 0], [3, 3], [0, 1]])
        return x, idx, packed(e, n, k // 2), scale(e, n, k // 32)

    reports = equivalence.assert_equivalent(op, make, rtol=1e-2, atol=2e-2, device=DEV)
    assert reports and all(r.passed for r in reports)


# ---------------------------------------------------------------------------
# scaled fp4 MFMA: fp8 hi/lo activation split and both MFMA forms of the block

def test_split_activations_bit_exact(rng):
    from local_kimi_amd.kernels import split_activations_fp8

    x = (rng.normal(0, 1, (48, 512)) * np.exp(rng.normal(0, 3, (48, 1)))).astype(np.float32)
    x[3] = 0.0
    x[5, :40] = -0.0
    x[7, 32:64] = 1.0 + 1.0 / 16.0  # midpoints between E4M3 neighbours: ties to even
    bits = f32_to_bf16_bits(x)
    hi, lo, sc = split_activations_fp8(_dev(bits))
    ehi, elo, esc = X.split_fp8(bits)
    assert np.array_equal(hi.cpu().numpy(), ehi)
    assert np.array_equal(lo.cpu().numpy(), elo)
    assert np.array_equal(sc.cpu().numpy().view(np.uint16), esc)


@pytest.mark.parametrize("form", ["scaled-fp4", "bf16"])
@pytest.mark.parametrize("tokens", [1, 40])
def test_moe_block_both_mfma_forms_match_oracle(rng, monkeypatch, form, tokens):
    from local_kimi_amd.kernels import mxfp4_moe_block

    e_routed, h, inter, k = 12, 384, 256, 4
    banks = (*_bank(rng, e_routed + 1, inter, h), *_bank(rng, e_routed + 1, inter, h),
             *_bank(rng, e_routed + 1, h, inter))
    x = random_bf16_bits(rng, (tokens, h))
    logits = rng.normal(0, 1, (tokens, e_routed)).astype(np.float32)
    ey, eidx, _ = X.moe_block(x, logits, None, *banks, top_k=k, routed_scaling_factor=2.446)
    with forced_path("mxfp4_mfma", "bf16" if form == "bf16" else "fp4"):
        y, idx, _ = mxfp4_moe_block(_dev(x), _dev(logits), None, *(_dev(b) for b in banks), k,
                                    2.446)
    assert np.array_equal(idx.cpu().numpy(), eidx)
    assert_close_bf16(to_bits(y), ey, what=f"mxfp4 moe block ({form}, T={tokens})")


@pytest.fixture(scope="module")
def designed_mx_prefill():
    """2048 tokens at H = 2304, I = 1024 with 32 routed + 1 shared MXFP4
    experts, routed so that expert tiles take every shape (designed_counts);
    the oracle output of every token."""
    from local_kimi_amd.quant import quantize_mxfp4

    from ._helpers import designed_counts, designed_router_logits

    tokens, routed, h, i = 2048, 32, 2304, 1024
    rng = np.random.default_rng(20260806)
    gen = torch.Generator(device=DEV).manual_seed(20260806)

    def bank(n, k):
        pairs = [quantize_mxfp4((torch.randn(n, k, device=DEV, generator=gen) * 0.02)
                                .to(torch.bfloat16)) for _ in range(routed + 1)]
        return torch.stack([p for p, _ in pairs]), torch.stack([s for _, s in pairs])

    banks = (*bank(i, h), *bank(i, h), *bank(h, i))
    counts = designed_counts(tokens, routed, 8)
    logits = designed_router_logits(rng, counts, tokens, 8)
    x = random_bf16_bits(rng, (tokens, h))
    ey, eidx, _ = X.moe_block(x, logits, None, *(b.cpu().numpy() for b in banks), top_k=8,
                              routed_scaling_factor=2.446)
    return x, logits, banks, counts, ey, eidx


@pytest.mark.parametrize("form", ["scaled-fp4", "bf16"])
def test_prefill_every_token_matches_oracle(designed_mx_prefill, form):
    """MXFP4 prefill on 64-row tiles in both MFMA forms (scaled fp4 with the
    fp8 hi + lo activation split, and bf16 on decoded weights): every token,
    so every tile shape of both kernels (full, partial 64-row, the 16-row
    tail path) is under the oracle."""
    from local_kimi_amd.kernels import mxfp4_moe_block

    x, logits, banks, counts, ey, eidx = designed_mx_prefill
    with forced_path("mxfp4_mfma", "bf16" if form == "bf16" else "fp4"):
        y, idx, _ = mxfp4_moe_block(_dev(x), _dev(logits), None, *banks, 8, 2.446)
    assert np.array_equal(idx.cpu().numpy(), eidx)
    assert np.array_equal(np.bincount(idx.cpu().numpy().reshape(-1), minlength=counts.size),
                          counts)
    assert_close_bf16(to_bits(y), ey, what=f"mxfp4 prefill ({form}), every token")
