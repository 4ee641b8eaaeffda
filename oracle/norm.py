"""Oracle for the decode normalisations: RMSNorm, residual add + RMSNorm and
the gated RMSNorm of the KDA output.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates engine/klinear/norm.py:9-52 and the residual adds of
engine/klinear/layer.py:150-170 in numpy. Values are float64 arrays holding
numbers representable in the named storage dtype ('float32', 'float16',
'bfloat16'); every fp32 operation of the reference is an exact float64
operation followed by an explicit rounding to float32, and every ``.to(dtype)``
an explicit rounding to the storage dtype, so each rounding point is visible.
The mean square is summed in float64 (torch sums it in fp32 in an order of its
own; the difference is far below the tests' tolerance).

Pinning (tests/test_oracle_norm.py): hand-computed cases (the [3, 4] row; a
one-hot row normalises to sqrt(width); the rounding-order case width 2,
weight 1.046875 -> 1.4765625, which the product-then-round order gets as
1.484375; sigmoid(0) = 1/2 halves the gated output), scale invariance, the
zero row under eps, torch's CPU evaluation of the reference expressions, and
planted mistakes (sum for mean, eps outside the root, weight before the
rounding, gate unsquashed) that fail those cases.
"""

from __future__ import annotations

import numpy as np

from .kda import round_to


def _f32(values) -> np.ndarray:
    return round_to(values, "float32")


def promoted(x_dtype: str, weight_dtype: str) -> str:
    """torch's result dtype of ``weight * x`` over {float32, float16, bfloat16}."""
    return x_dtype if x_dtype == weight_dtype else "float32"


def _inv_rms(v: np.ndarray, eps: float) -> np.ndarray:
    """fp32 rsqrt(mean(v^2) + eps) over the last axis (norm.py:12, :48-50)."""
    ms = _f32(np.mean(np.square(v), axis=-1, keepdims=True))
    return _f32(1.0 / _f32(np.sqrt(_f32(ms + _f32(eps)))))


def rms_norm(x, weight, eps: float, x_dtype: str, weight_dtype: str) -> np.ndarray:
    """engine/klinear/norm.py:9-13: ``weight * (fp32(x) * rsqrt(mean(x^2) + eps)).to(x.dtype)``;
    the product in torch's promoted dtype."""
    v = np.asarray(x, dtype=np.float64)
    n = round_to(_f32(v * _inv_rms(v, eps)), x_dtype)
    w = np.asarray(weight, dtype=np.float64)
    return round_to(_f32(w * n), promoted(x_dtype, weight_dtype))


def add_rms_norm(residual, delta, weight, eps: float, x_dtype: str, weight_dtype: str):
    """engine/klinear/layer.py:156-160: ``hidden = residual + attended`` (an fp32
    add rounded to the storage dtype) and the RMSNorm that follows; returns
    (hidden, normed)."""
    s = round_to(_f32(np.asarray(residual, dtype=np.float64) + np.asarray(delta, dtype=np.float64)),
                 x_dtype)
    return s, rms_norm(s, weight, eps, x_dtype, weight_dtype)


def sigmoid_f32(g) -> np.ndarray:
    g = np.asarray(g, dtype=np.float64)
    return _f32(1.0 / (1.0 + np.exp(-g)))


def rms_gated_norm(values, gate, weight, eps: float, input_dtype: str) -> np.ndarray:
    """engine/klinear/norm.py:45-52 (RMSGatedNorm.forward) on values first
    rounded to ``input_dtype`` (attention.py:324, ``.to(hidden_states.dtype)``):
    ``(v * rsqrt(mean(v^2) + eps) * fp32(weight) * sigmoid(fp32(gate))).to(input_dtype)``."""
    v = round_to(values, input_dtype)
    n = _f32(v * _inv_rms(v, eps))
    w = np.asarray(weight, dtype=np.float64)
    out = _f32(_f32(n * w) * sigmoid_f32(gate))
    return round_to(out, input_dtype)
