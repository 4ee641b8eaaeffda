"""Kimi Delta Attention decode kernels, restated in numpy (test infrastructure).

Only the tests, ``__graft_entry__.smoke()`` and the bench's CPU leg use this
module, as the checker of the HIP kernels; nothing in the product path calls it.

Three functions, each in float64 so it serves as the exact answer the fp32
kernels are held to:

* ``decode_step``  — engine/kernels/kda_step.py:173-196 (the eager recurrence):
  S ← S·exp(decay) row-wise; pred = Sᵀk; S ← S + β·k·(v − pred)ᵀ;
  out = Sᵀ(q·scale). State [B, H, dk, dv], q/k/decay [B, H, dk], v [B, H, dv],
  beta [B, H].
* ``short_conv_triple`` — engine/kernels/kda_prepare.py:434-476: per channel
  the width-4 window (state[1:], token), conv = Σ window·weight in fp32,
  SiLU, rounded to the input dtype; the window becomes the new state.
* ``gates`` — engine/kernels/kda_prepare.py:590-627: decay = −exp(A_log[h]) ·
  softplus(raw_decay + dt_bias) (softplus(x) = x above 20, as torch's
  threshold and the fused kernel's SOFTPLUS_THRESHOLD, kda_prepare.py:22),
  beta = sigmoid(raw_beta), q and k scaled by rsqrt(Σx² + eps) per head.

Pinned by the reference's hand-computed cases (tests/test_kda_step.py:13-90,
tests/test_kda_prepare.py:26-123) and by closed forms and invariants in
tests/test_oracle_kda.py.
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits

CONV_WIDTH = 4
SOFTPLUS_THRESHOLD = 20.0


def decode_step(state: np.ndarray, q: np.ndarray, k: np.ndarray, v: np.ndarray,
                decay: np.ndarray, beta: np.ndarray, scale: float
                ) -> tuple[np.ndarray, np.ndarray]:
    """One recurrence step (kda_step.py:186-195). Returns (new state, output),
    both float64; the inputs are not modified."""
    s = np.asarray(state, dtype=np.float64)
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    g = np.exp(np.asarray(decay, dtype=np.float64))
    b = np.asarray(beta, dtype=np.float64)
    cand = s * g[..., :, None]                           # decay each key row
    pred = np.einsum("bhkv,bhk->bhv", cand, k)           # what the state recalls for k
    delta = v - pred
    cand = cand + b[..., None, None] * k[..., :, None] * delta[..., None, :]
    out = np.einsum("bhkv,bhk->bhv", cand, q * scale)
    return cand, out


def silu(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


def round_to(values: np.ndarray, dtype: str) -> np.ndarray:
    """float64 -> the storage dtype ('float32', 'float16' or 'bfloat16'), as
    float64 values; torch's casts round to nearest even."""
    v = np.asarray(values, dtype=np.float64)
    if dtype == "float32":
        return v.astype(np.float32).astype(np.float64)
    if dtype == "float16":
        return v.astype(np.float16).astype(np.float64)
    if dtype == "bfloat16":
        return bf16_bits_to_f32(f32_to_bf16_bits(v.astype(np.float32))).astype(np.float64)
    raise ValueError(f"unsupported dtype {dtype}")


def short_conv(values: np.ndarray, state: np.ndarray, weight: np.ndarray, dtype: str
               ) -> tuple[np.ndarray, np.ndarray]:
    """One width-4 causal convolution step (kda_prepare.py:434-445).

    values [B, 1, C] and state [B, C, 4] hold numbers representable in
    ``dtype``; weight is [C, 4] or [C, 1, 4]. Returns (output [B, 1, C] rounded
    to dtype, new state [B, C, 4]) as float64. The sum of four products is
    exact enough in float64 that it stands for the fp32 sum within the
    tolerance the tests state."""
    w = np.asarray(weight, dtype=np.float64)
    if w.ndim == 3:
        w = w[:, 0, :]
    st = np.asarray(state, dtype=np.float64)
    token = np.asarray(values, dtype=np.float64)[:, 0]
    shifted = np.concatenate((st[:, :, 1:], token[:, :, None]), axis=-1)
    conv = (shifted * w[None, :, :]).sum(axis=-1)
    return round_to(silu(conv), dtype)[:, None, :], shifted


def short_conv_triple(q_in, k_in, v_in, q_state, k_state, v_state, q_weight, k_weight,
                      v_weight, dtype: str):
    """The three convolutions of kda_prepare.py:448-476: ((q, k, v) outputs,
    (q, k, v) new states)."""
    q, qs = short_conv(q_in, q_state, q_weight, dtype)
    k, ks = short_conv(k_in, k_state, k_weight, dtype)
    v, vs = short_conv(v_in, v_state, v_weight, dtype)
    return (q, k, v), (qs, ks, vs)


def softplus(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    return np.where(x > SOFTPLUS_THRESHOLD, x,
                    np.log1p(np.exp(np.minimum(x, SOFTPLUS_THRESHOLD))))


def gates(raw_decay: np.ndarray, dt_bias: np.ndarray, a_log: np.ndarray,
          raw_beta: np.ndarray, q: np.ndarray, k: np.ndarray, num_heads: int,
          head_dim: int, eps: float):
    """kda_prepare.py:603-627: (decay [B, S, H, D], beta [B, S, H], q and k
    normalised [B, S, H, D]), float64. q and k may be flat [B, S, H*D]."""
    rd = np.asarray(raw_decay, dtype=np.float64)
    b, s = rd.shape[:2]
    biased = rd + np.asarray(dt_bias, dtype=np.float64).reshape(num_heads, head_dim)
    rate = np.exp(np.asarray(a_log, dtype=np.float64).reshape(1, 1, num_heads, 1))
    decay = -rate * softplus(biased)
    beta = 1.0 / (1.0 + np.exp(-np.asarray(raw_beta, dtype=np.float64)))
    qn = np.asarray(q, dtype=np.float64).reshape(b, s, num_heads, head_dim)
    kn = np.asarray(k, dtype=np.float64).reshape(b, s, num_heads, head_dim)
    qn = qn / np.sqrt((qn * qn).sum(axis=-1, keepdims=True) + eps)
    kn = kn / np.sqrt((kn * kn).sum(axis=-1, keepdims=True) + eps)
    return decay, beta, qn, kn
