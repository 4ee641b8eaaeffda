"""W4A16 codec and projections, restated in numpy.

Layout (quant/w4a16.py:1-6, 46-47, 94-99): ``packed[N, K/2]`` uint8 where
byte j holds reduction index 2j in the LOW nibble and 2j+1 in the HIGH nibble;
codes are 4-bit two's complement (v >= 8 -> v - 16); ``scales[N, K/G]`` bf16.
The reference hard-codes G=32 (quant/w4a16.py:14,36-37); here G is a
parameter because the workloads use G=128.
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32, bf16_tiny, f32_to_bf16_bits, round_bf16

QMIN = -7
QMAX = 7


def _check_group(k: int, group_size: int) -> None:
    if group_size <= 0 or k % group_size:
        raise ValueError(f"reduction width {k} must be divisible by group size {group_size}")


def quantise(weight_bits: np.ndarray, group_size: int) -> tuple[np.ndarray, np.ndarray]:
    """Quantise a bf16 ``[N, K]`` matrix (uint16 bits) along K.

    Follows quant/w4a16.py:68-105: per group absmax in fp32, ``bf16(absmax/7)``,
    all-zero group -> scale 1, non-zero scales clamped to bf16 tiny, codes =
    round-half-even(w / stored_scale) clamped to [-7, 7], low nibble first.
    Returns ``(packed uint8 [N, K/2], scales uint16 bf16 bits [N, K/G])``.
    """
    w = bf16_bits_to_f32(weight_bits)
    if w.ndim != 2:
        raise ValueError("weight must have shape [out_features, in_features]")
    if not np.isfinite(w).all():
        raise ValueError("weight must contain only finite values")
    n, k = w.shape
    _check_group(k, group_size)
    groups = w.reshape(n, k // group_size, group_size)
    absmax = np.abs(groups).max(axis=-1).astype(np.float32)
    raw = (absmax / np.float32(QMAX)).astype(np.float32)
    stored = round_bf16(raw)
    scales_f = np.where(absmax == 0, np.float32(1.0), np.maximum(stored, np.float32(bf16_tiny())))
    scales_bits = f32_to_bf16_bits(scales_f)
    scales_f = bf16_bits_to_f32(scales_bits)
    codes = np.rint(groups / scales_f[..., None]).astype(np.float32)
    codes = np.clip(codes, QMIN, QMAX).astype(np.int16).reshape(n, k)
    nibbles = (codes & 0xF).astype(np.uint8)
    packed = (nibbles[:, 0::2] | (nibbles[:, 1::2] << 4)).astype(np.uint8)
    return np.ascontiguousarray(packed), np.ascontiguousarray(scales_bits)


def unpack_codes(packed: np.ndarray) -> np.ndarray:
    """Signed int4 codes ``[..., K]`` from ``[..., K/2]`` bytes (quant/w4a16.py:118-122)."""
    p = np.asarray(packed, dtype=np.uint8)
    low = (p & 0xF).astype(np.int16)
    high = (p >> 4).astype(np.int16)
    nib = np.stack((low, high), axis=-1).reshape(*p.shape[:-1], p.shape[-1] * 2)
    return np.where(nib >= 8, nib - 16, nib).astype(np.int16)


def dequantise(packed: np.ndarray, scales_bits: np.ndarray, group_size: int,
               *, dtype: str = "bf16") -> np.ndarray:
    """Decode to bf16 bits (``dtype='bf16'``) or float32 (quant/w4a16.py:108-129).

    Value is ``bf16(float(q) * float(scale))``; the float32 product is exact
    and the bf16 cast is the single rounding.
    """
    codes = unpack_codes(packed)
    k = codes.shape[-1]
    _check_group(k, group_size)
    s = bf16_bits_to_f32(scales_bits)
    if s.shape[-1] * group_size != k:
        raise ValueError("scale shape does not match the reduction width")
    restored = codes.astype(np.float32).reshape(*codes.shape[:-1], k // group_size, group_size)
    restored = (restored * s[..., None]).reshape(codes.shape)
    if dtype == "bf16":
        return f32_to_bf16_bits(restored)
    if dtype == "f32":
        return restored.astype(np.float32)
    raise TypeError("dequantise output dtype must be 'bf16' or 'f32'")


def _matmul_bf16_out(x_f32: np.ndarray, w_f32: np.ndarray) -> np.ndarray:
    """``bf16(x @ w.T)`` accumulated in float64 (every product is exact)."""
    acc = np.asarray(x_f32, dtype=np.float64) @ np.asarray(w_f32, dtype=np.float64).T
    return f32_to_bf16_bits(acc.astype(np.float32))


def dense(x_bits: np.ndarray, packed: np.ndarray, scales_bits: np.ndarray,
          group_size: int) -> np.ndarray:
    """``y[M, N] = x @ bf16(dequant W).T``, fp32-class accumulate, bf16 out.

    Restates the registered reference of op ``w4a16_dense``
    (kernels/__init__.py:92-104 -> quant/triton_w4a16.py:105-113, 151-188):
    weights decoded to bf16 before the dot, fp32 accumulation, bf16 store.
    """
    w = bf16_bits_to_f32(dequantise(packed, scales_bits, group_size))
    return _matmul_bf16_out(bf16_bits_to_f32(x_bits), w)


def grouped(x_bits: np.ndarray, expert_indices: np.ndarray, packed: np.ndarray,
            scales_bits: np.ndarray, group_size: int) -> np.ndarray:
    """``out[t, r, :] = x[t] @ bf16(dequant W[idx[t, r]]).T`` -> bf16 ``[T, R, N]``.

    Restates op ``w4a16_grouped`` (kernels/w4a16_grouped.py:121-194 and
    kernels/w4a16_gemv.py:56-174, 610-635): one GEMV per (token, route).
    """
    x = bf16_bits_to_f32(x_bits)
    idx = np.asarray(expert_indices, dtype=np.int64)
    t_count, r_count = idx.shape
    n = packed.shape[1]
    out = np.empty((t_count, r_count, n), dtype=np.uint16)
    # each output row is its own float64 dot product; rows that share an
    # expert are evaluated together (one decode of the expert per call)
    for e in np.unique(idx):
        tok, slot = np.nonzero(idx == e)
        w = bf16_bits_to_f32(dequantise(packed[int(e)], scales_bits[int(e)], group_size))
        out[tok, slot] = _matmul_bf16_out(x[tok], w)
    return out


def silu_bf16(gate_bits: np.ndarray) -> np.ndarray:
    """``F.silu`` on a bf16 tensor: fp32 ``g / (1 + exp(-g))`` rounded to bf16."""
    g = bf16_bits_to_f32(gate_bits)
    with np.errstate(over="ignore"):
        act = (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32)
    return f32_to_bf16_bits(act)


def mul_bf16(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """bf16 * bf16 in torch: fp32 product rounded once to bf16."""
    return f32_to_bf16_bits(bf16_bits_to_f32(a_bits) * bf16_bits_to_f32(b_bits))


def add_bf16(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """bf16 + bf16 in torch: fp32 sum rounded once to bf16."""
    return f32_to_bf16_bits(bf16_bits_to_f32(a_bits) + bf16_bits_to_f32(b_bits))


def swiglu(x_bits, expert_indices, w1_packed, w1_scales, w3_packed, w3_scales,
           group_size: int) -> np.ndarray:
    """``act = bf16(bf16(silu(bf16(W1 x))) * bf16(W3 x))`` -> bf16 ``[T, R, I]``.

    Restates op ``w4a16_swiglu``'s reference (kernels/__init__.py:182-197):
    two grouped calls (each rounded to bf16), ``F.silu`` on bf16, bf16 multiply.
    The same contract as the fused kernel's ``_rounded_silu_mul``
    (kernels/w4a16_gemv.py:214-221).
    """
    gate = grouped(x_bits, expert_indices, w1_packed, w1_scales, group_size)
    up = grouped(x_bits, expert_indices, w3_packed, w3_scales, group_size)
    return mul_bf16(silu_bf16(gate), up)


def fused_qkv(x_bits, q_packed, q_scales, k_packed, k_scales, v_packed, v_scales,
              group_size: int):
    """Three dense projections (kernels/w4a16_fused_qkv.py:257-271)."""
    return (
        dense(x_bits, q_packed, q_scales, group_size),
        dense(x_bits, k_packed, k_scales, group_size),
        dense(x_bits, v_packed, v_scales, group_size),
    )
