"""Host-side validation raises the reference's exception types before any GPU work."""

from __future__ import annotations

import pytest
import torch

from local_kimi_amd.kernels import (fused_w2_combine, grouped_w4a16_gemv, grouped_w4a16_swiglu_gemv,
                                    moe_router, w4a16_dense)
from local_kimi_amd.quant import W4A16Tensor, quantise


def test_dense_rejects_wrong_dtypes_and_cpu_tensors():
    x = torch.zeros((1, 64), dtype=torch.bfloat16)
    p = torch.zeros((8, 32), dtype=torch.uint8)
    s = torch.zeros((8, 2), dtype=torch.bfloat16)
    with pytest.raises(TypeError):
        w4a16_dense(x.float(), p, s)
    with pytest.raises(TypeError):
        w4a16_dense(x, p.to(torch.int8), s)
    with pytest.raises(TypeError):
        w4a16_dense(x, p, s.float())
    with pytest.raises(ValueError, match="requires CUDA"):
        w4a16_dense(x, p, s)


def test_grouped_rejects_bad_indices_dtype_and_shapes():
    x = torch.zeros((1, 64), dtype=torch.bfloat16)
    p = torch.zeros((3, 8, 32), dtype=torch.uint8)
    s = torch.zeros((3, 8, 2), dtype=torch.bfloat16)
    with pytest.raises(TypeError, match="int64"):
        grouped_w4a16_gemv(x, torch.zeros((1, 2), dtype=torch.int32), p, s)
    with pytest.raises(ValueError, match="rank three"):
        grouped_w4a16_gemv(x, torch.zeros((1, 2), dtype=torch.long), p[0], s[0])
    with pytest.raises(ValueError, match="requires CUDA"):
        grouped_w4a16_gemv(x, torch.zeros((1, 2), dtype=torch.long), p, s)


def test_swiglu_and_combine_reject_mismatched_inputs():
    x = torch.zeros((1, 64), dtype=torch.bfloat16)
    idx = torch.zeros((1, 2), dtype=torch.long)
    p = torch.zeros((3, 8, 32), dtype=torch.uint8)
    s = torch.zeros((3, 8, 2), dtype=torch.bfloat16)
    with pytest.raises(TypeError):
        grouped_w4a16_swiglu_gemv(x, idx, p, s.float(), p, s)
    act = torch.zeros((1, 2, 64), dtype=torch.bfloat16)
    with pytest.raises(TypeError, match="float32"):
        fused_w2_combine(act, idx, torch.zeros((1, 2), dtype=torch.float64), p, s)


def test_router_rejects_bad_arguments():
    with pytest.raises(TypeError):
        moe_router(torch.zeros((1, 8), dtype=torch.float64), None, 2)
    with pytest.raises(ValueError, match="requires CUDA"):
        moe_router(torch.zeros((1, 8)), None, 2)


def test_codec_validation():
    with pytest.raises(TypeError):
        quantise(torch.zeros((2, 64)))
    with pytest.raises(ValueError, match="divisible"):
        quantise(torch.zeros((2, 48), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="power-of-two"):
        quantise(torch.zeros((2, 96), dtype=torch.bfloat16), group_size=96)
    with pytest.raises(ValueError, match="requires a CUDA"):
        quantise(torch.zeros((2, 64), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="scale shape"):
        W4A16Tensor(torch.zeros((2, 64), dtype=torch.uint8), torch.zeros((2, 3), dtype=torch.bfloat16),
                    (2, 128), group_size=32)


def test_kda_ops_validate_like_the_reference_before_any_launch():
    """engine/kernels/kda_step.py:140-170 and kda_prepare.py:378-431, 541-587:
    the same exception types and messages, raised on CPU tensors before any
    kernel runs."""
    from local_kimi_amd.kernels import fused_kda_gates, fused_short_conv_triple, kda_decode_step

    st = torch.zeros((1, 2, 4, 4))
    z3 = torch.zeros((1, 2, 4))
    b = torch.zeros((1, 2))
    with pytest.raises(ValueError, match=r"state must have shape"):
        kda_decode_step(st[0], z3, z3, z3, z3, b, scale=1.0)
    with pytest.raises(TypeError, match="float32"):
        kda_decode_step(st.double(), z3, z3, z3, z3, b, scale=1.0)
    with pytest.raises(ValueError, match=r"beta must have shape"):
        kda_decode_step(st, z3, z3, z3, z3, z3, scale=1.0)
    with pytest.raises(ValueError, match="requires CUDA"):
        kda_decode_step(st, z3, z3, z3, z3, b, scale=1.0)

    x = torch.zeros((2, 1, 8))
    s4 = torch.zeros((2, 8, 4))
    w = torch.zeros((8, 1, 4))
    with pytest.raises(ValueError, match="sequence length one"):
        fused_short_conv_triple(*(torch.zeros((2, 2, 8)),) * 3, s4, s4, s4, w, w, w)
    with pytest.raises(ValueError, match=r"state must have shape \[batch, channels, 4\]"):
        fused_short_conv_triple(x, x, x, s4[:, :, :3], s4, s4, w, w, w)
    with pytest.raises(TypeError, match="share a dtype"):
        fused_short_conv_triple(x, x, x, s4.half(), s4, s4, w, w, w)
    with pytest.raises(ValueError, match="requires CUDA"):
        fused_short_conv_triple(x, x, x, s4, s4, s4, w, w, w)

    rd = torch.zeros((1, 1, 2, 4))
    with pytest.raises(ValueError, match="head_dim at most 1024"):
        fused_kda_gates(rd, torch.zeros(8), torch.zeros((1, 1, 2, 1)), torch.zeros((1, 1, 2)),
                        torch.zeros((1, 1, 8)), torch.zeros((1, 1, 8)), num_heads=2,
                        head_dim=2048, eps=1e-6)
    with pytest.raises(ValueError, match="eps must be positive"):
        fused_kda_gates(rd, torch.zeros(8), torch.zeros((1, 1, 2, 1)), torch.zeros((1, 1, 2)),
                        torch.zeros((1, 1, 8)), torch.zeros((1, 1, 8)), num_heads=2,
                        head_dim=4, eps=0.0)
    with pytest.raises(ValueError, match="contiguous without transposition"):
        q = torch.zeros((1, 1, 16))[..., ::2]
        fused_kda_gates(rd, torch.zeros(8), torch.zeros((1, 1, 2, 1)), torch.zeros((1, 1, 2)),
                        q, q, num_heads=2, head_dim=4, eps=1e-6)
    with pytest.raises(ValueError, match="require CUDA"):
        fused_kda_gates(rd, torch.zeros(8), torch.zeros((1, 1, 2, 1)), torch.zeros((1, 1, 2)),
                        torch.zeros((1, 1, 8)), torch.zeros((1, 1, 8)), num_heads=2,
                        head_dim=4, eps=1e-6)


def test_norm_wrappers_refuse_bad_inputs_before_any_launch():
    from local_kimi_amd.kernels import add_rms_norm, rms_gated_norm, rms_norm

    x = torch.zeros((2, 16), dtype=torch.bfloat16)
    w = torch.ones(16, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="shape \\[16\\]"):
        rms_norm(x, torch.ones(8, dtype=torch.bfloat16), 1e-6)
    with pytest.raises(ValueError, match="multiple of 8"):
        rms_norm(torch.zeros((2, 12), dtype=torch.bfloat16), torch.ones(12, dtype=torch.bfloat16), 1e-6)
    with pytest.raises(TypeError, match="float32, float16 or bfloat16"):
        rms_norm(x.to(torch.int32), w, 1e-6)
    with pytest.raises(ValueError, match="require CUDA"):
        rms_norm(x, w, 1e-6)
    with pytest.raises(TypeError, match="share one dtype"):
        add_rms_norm(x, x.float(), w, 1e-6)
    with pytest.raises(ValueError, match="same shape"):
        add_rms_norm(x, x[:1], w, 1e-6)
    with pytest.raises(ValueError, match="same shape"):
        rms_gated_norm(x, x[:, :8], w, 1e-5)
    with pytest.raises(TypeError, match="input_dtype"):
        rms_gated_norm(x, x, w, 1e-5, input_dtype=torch.int8)
