"""Decode normalisations on HIP: RMSNorm, residual add + RMSNorm, gated RMSNorm.

``rms_norm(hidden_states, weight, eps)`` has the name, signature and result
dtype of engine/klinear/norm.py:9-13; ``rms_gated_norm(values, gate, weight,
eps)`` computes ``RMSGatedNorm.forward`` (norm.py:45-52). ``add_rms_norm``
fuses the residual add of engine/klinear/layer.py:156/:170 with the RMSNorm
that reads its result (post_attention_layernorm, or the next layer's
input_layernorm) and returns both. Each is one launch of
``local_kimi_amd/csrc/norm.hip``; outputs are allocated from the torch caching
allocator on the input's device, inputs are never mutated, and nothing
synchronises, so the calls can be captured in a HIP graph.

Inputs must be float32, float16 or bfloat16 CUDA tensors whose last dimension
(the normalised one) is a multiple of 8 up to 8192; other layouts are copied
to dense ones first.
"""

from __future__ import annotations

import torch

from .. import _lib
from . import w4a16 as _w

NORM_MAX_WIDTH = 8192
_DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def _code(t: torch.Tensor, what: str) -> int:
    code = _DTYPE_CODES.get(t.dtype)
    if code is None:
        raise TypeError(f"{what} must be float32, float16 or bfloat16, got {t.dtype}")
    return code


def _dense(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() and t.data_ptr() % 16 == 0 else t.contiguous()


def _check_rows(x: torch.Tensor, weight: torch.Tensor, what: str) -> int:
    if x.ndim < 1:
        raise ValueError(f"{what} must have at least one dimension")
    width = x.shape[-1]
    if weight.ndim != 1 or weight.shape[0] != width:
        raise ValueError(f"the norm weight must have shape [{width}], got {tuple(weight.shape)}")
    if width == 0 or width % 8 or width > NORM_MAX_WIDTH:
        raise ValueError(f"the normalised width must be a positive multiple of 8 up to "
                         f"{NORM_MAX_WIDTH}, got {width}")
    if x.device.type != "cuda":
        raise ValueError("the HIP norm kernels require CUDA tensors")
    if weight.device != x.device:
        raise ValueError("norm inputs must share one device")
    return width


def _result_dtype(x: torch.Tensor, weight: torch.Tensor) -> torch.dtype:
    return x.dtype if x.dtype == weight.dtype else torch.float32


def rms_norm(hidden_states: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``weight * (x.float() * rsqrt(mean(x.float()^2) + eps)).to(x.dtype)``
    (engine/klinear/norm.py:9-13), in torch's promoted dtype."""
    xc, wc = _code(hidden_states, "hidden states"), _code(weight, "the norm weight")
    width = _check_rows(hidden_states, weight, "hidden states")
    if eps < 0:
        raise ValueError("eps must be non-negative")
    x, w = _dense(hidden_states), _dense(weight)
    out = torch.empty(hidden_states.shape, dtype=_result_dtype(x, w), device=x.device)
    rows = x.numel() // width
    if rows:
        with torch.cuda.device(x.device):
            _lib.call("lk_rms_norm", x.data_ptr(), w.data_ptr(), out.data_ptr(), rows, width,
                      float(eps), xc, wc, _w._stream(x.device))
    return out


def add_rms_norm(residual: torch.Tensor, delta: torch.Tensor, weight: torch.Tensor,
                 eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """``hidden = residual + delta`` (rounded to their dtype), then
    ``rms_norm(hidden, weight, eps)``; returns ``(hidden, normed)``
    (engine/klinear/layer.py:156-160)."""
    if residual.dtype != delta.dtype:
        raise TypeError("residual and delta must share one dtype")
    if residual.shape != delta.shape:
        raise ValueError("residual and delta must have the same shape")
    xc, wc = _code(residual, "the residual stream"), _code(weight, "the norm weight")
    width = _check_rows(residual, weight, "the residual stream")
    if delta.device != residual.device:
        raise ValueError("norm inputs must share one device")
    if eps < 0:
        raise ValueError("eps must be non-negative")
    r, d, w = _dense(residual), _dense(delta), _dense(weight)
    hidden = torch.empty(residual.shape, dtype=residual.dtype, device=r.device)
    out = torch.empty(residual.shape, dtype=_result_dtype(r, w), device=r.device)
    rows = r.numel() // width
    if rows:
        with torch.cuda.device(r.device):
            _lib.call("lk_add_rms_norm", r.data_ptr(), d.data_ptr(), w.data_ptr(),
                      hidden.data_ptr(), out.data_ptr(), rows, width, float(eps), xc, wc,
                      _w._stream(r.device))
    return hidden, out


def rms_gated_norm(values: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, eps: float,
                   *, input_dtype: torch.dtype | None = None) -> torch.Tensor:
    """``RMSGatedNorm.forward`` (engine/klinear/norm.py:45-52) over the last
    dimension: ``(v * rsqrt(mean(v^2) + eps) * weight.float() *
    sigmoid(gate.float())).to(input_dtype)`` with ``v = values.to(input_dtype).float()``.

    ``input_dtype`` defaults to ``values.dtype``; passing bf16 for fp32
    values folds the reference's ``.to(hidden_states.dtype)`` before o_norm
    (engine/klinear/attention.py:324) into the same launch.
    """
    in_dtype = values.dtype if input_dtype is None else input_dtype
    vc, gc = _code(values, "values"), _code(gate, "the gate")
    wc = _code(weight, "the norm weight")
    ic = _DTYPE_CODES.get(in_dtype)
    if ic is None:
        raise TypeError(f"input_dtype must be float32, float16 or bfloat16, got {in_dtype}")
    if gate.shape != values.shape:
        raise ValueError("values and gate must have the same shape")
    width = _check_rows(values, weight, "values")
    if gate.device != values.device:
        raise ValueError("norm inputs must share one device")
    if eps < 0:
        raise ValueError("eps must be non-negative")
    v, g, w = _dense(values), _dense(gate), _dense(weight)
    out = torch.empty(values.shape, dtype=in_dtype, device=v.device)
    rows = v.numel() // width
    if rows:
        with torch.cuda.device(v.device):
            _lib.call("lk_rms_gated_norm", v.data_ptr(), g.data_ptr(), w.data_ptr(),
                      out.data_ptr(), rows, width, float(eps), vc, ic, gc, wc,
                      _w._stream(v.device))
    return out
