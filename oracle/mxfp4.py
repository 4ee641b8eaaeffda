"""OCP MXFP4 codec and linear, restated in numpy.

Decode follows engine/k3ref/dequant.py:18-73 and kernels/reference.py:29-80:
E2M1 nibbles, low nibble first, sign bit 3 (negative zero kept), one E8M0
exponent per 32 values along K, value = e2m1 * 2**(e8m0 - 127).

The reference has no encoder. :func:`quantize` is this project's encoder,
written from the OCP Microscaling Formats v1.0 definition: shared exponent
``floor(log2(amax)) - emax_elem`` with ``emax_elem = 2`` for E2M1, elements
rounded to nearest (ties to even) on the E2M1 grid and saturated to +-6.
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits

GROUP = 32
EXP_BIAS = 127
E2M1_POSITIVE = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)
E2M1_CODEBOOK = np.concatenate((E2M1_POSITIVE, -E2M1_POSITIVE)).astype(np.float32)


def unpack(packed: np.ndarray) -> np.ndarray:
    """Decode E2M1 nibbles to float32 (low nibble first, -0.0 preserved)."""
    p = np.asarray(packed, dtype=np.uint8)
    codes = np.stack((p & 0xF, p >> 4), axis=-1).reshape(*p.shape[:-1], p.shape[-1] * 2)
    return E2M1_CODEBOOK[codes]


def dequantize(packed: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """Float32 weights ``[N, K]`` from ``packed [N, K/2]`` and ``scale [N, K/32]`` u8."""
    values = unpack(packed)
    k = values.shape[-1]
    s = np.asarray(scale, dtype=np.uint8)
    if s.shape[-1] * GROUP != k:
        raise ValueError("MXFP4 scale shape must provide one exponent for every 32 decoded values")
    exps = np.ldexp(np.float32(1.0), s.astype(np.int32) - EXP_BIAS).astype(np.float32)
    return (values.reshape(*values.shape[:-1], k // GROUP, GROUP) * exps[..., None]).reshape(values.shape)


def _e2m1_code(v: np.ndarray) -> np.ndarray:
    """Nearest E2M1 code (ties to even code, saturating) for float32 values."""
    a = np.minimum(np.abs(v), np.float32(6.0))
    # Decision boundaries between consecutive grid points; at an exact midpoint
    # the even code wins: 0.25->0, 0.75->2(1.0), 1.25->2(1.0), 1.75->4(2.0),
    # 2.5->4(2.0), 3.5->6(4.0), 5.0->6(4.0).
    mag = np.zeros(a.shape, dtype=np.uint8)
    mag = np.where(a > 0.25, 1, mag)
    mag = np.where(a >= 0.75, 2, mag)
    mag = np.where(a > 1.25, 3, mag)
    mag = np.where(a >= 1.75, 4, mag)
    mag = np.where(a > 2.5, 5, mag)
    mag = np.where(a >= 3.5, 6, mag)
    mag = np.where(a > 5.0, 7, mag)
    sign = np.signbit(v).astype(np.uint8) << 3
    return (mag.astype(np.uint8) | sign).astype(np.uint8)


def quantize(weight_f32: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Encode ``[N, K]`` float32 to ``(packed [N, K/2] u8, scale [N, K/32] u8)``.

    Shared exponent per 32 values: ``floor(log2(amax)) - 2`` biased by 127 and
    clamped to [0, 254]; an all-zero block uses 127. Elements are
    ``w / 2**exp`` rounded to the E2M1 grid.
    """
    w = np.asarray(weight_f32, dtype=np.float32)
    n, k = w.shape
    if k % GROUP:
        raise ValueError("MXFP4 reduction dimension must be divisible by 32")
    blocks = w.reshape(n, k // GROUP, GROUP)
    amax = np.abs(blocks).max(axis=-1)
    # floor(log2(amax)) exactly: frexp gives amax = m * 2**fe with m in [0.5, 1).
    _, fe = np.frexp(np.where(amax > 0, amax, 1.0).astype(np.float32))
    e = (fe.astype(np.int64) - 1)
    biased = np.clip(e - 2 + EXP_BIAS, 0, 254)
    biased = np.where(amax > 0, biased, EXP_BIAS).astype(np.uint8)
    scale_f = np.ldexp(np.float32(1.0), biased.astype(np.int32) - EXP_BIAS).astype(np.float32)
    scaled = (blocks / scale_f[..., None]).astype(np.float32)
    codes = _e2m1_code(scaled).reshape(n, k)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    return np.ascontiguousarray(packed), np.ascontiguousarray(biased)


def linear(x_bits: np.ndarray, packed: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """``F.linear(x, bf16(dequant W))`` -> bf16 bits (kernels/reference.py:67-80).

    The decoded weight is cast to the activation dtype (bf16); e2m1 * 2**k is
    exactly representable there, so the cast is lossless unless it leaves the
    bf16 range. Accumulation is float64, output rounded to bf16.
    """
    w = bf16_bits_to_f32(f32_to_bf16_bits(dequantize(packed, scale)))
    x = bf16_bits_to_f32(x_bits)
    acc = x.astype(np.float64) @ w.astype(np.float64).T
    return f32_to_bf16_bits(acc.astype(np.float32))
