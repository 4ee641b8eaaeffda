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


def linear_f16(x_f16_bits: np.ndarray, packed: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """The same linear with fp16 activations: the decoded weight cast to fp16
    (kernels/reference.py:75-80 with ``dtype=float16``), float64 accumulation,
    fp16 output bits."""
    w = dequantize(packed, scale).astype(np.float16).astype(np.float64)
    x = np.asarray(x_f16_bits, dtype=np.uint16).view(np.float16).astype(np.float64)
    return (x @ w.T).astype(np.float16).view(np.uint16)


def grouped(x_bits, expert_indices, packed_bank, scale_bank) -> np.ndarray:
    """``out[t, r] = linear(x[t], expert idx[t, r])`` -> bf16 bits ``[T, R, N]``.

    The per-route evaluation of kernels/reference.py:119-165 with
    ``mxfp4_linear_reference`` as the expert function.
    """
    x = np.asarray(x_bits)
    idx = np.asarray(expert_indices, dtype=np.int64)
    t_count, r_count = idx.shape
    n = packed_bank.shape[1]
    out = np.empty((t_count, r_count, n), dtype=np.uint16)
    # each output row is its own float64 dot product; rows that share an
    # expert are evaluated together (one decode of the expert per call)
    for e in np.unique(idx):
        tok, slot = np.nonzero(idx == e)
        w = bf16_bits_to_f32(f32_to_bf16_bits(dequantize(packed_bank[int(e)], scale_bank[int(e)])))
        acc = bf16_bits_to_f32(x[tok]).astype(np.float64) @ w.astype(np.float64).T
        out[tok, slot] = f32_to_bf16_bits(acc.astype(np.float32))
    return out


def swiglu(x_bits, expert_indices, w1_packed, w1_scale, w3_packed, w3_scale) -> np.ndarray:
    """``bf16(bf16(silu(gate)) * up)`` with MXFP4 gate / up projections (the
    SwiGLU contract of engine/kernels/__init__.py:182-197)."""
    from .w4a16 import mul_bf16, silu_bf16

    gate = grouped(x_bits, expert_indices, w1_packed, w1_scale)
    up = grouped(x_bits, expert_indices, w3_packed, w3_scale)
    return mul_bf16(silu_bf16(gate), up)


def moe_block(x_bits, logits, bias, w1_packed, w1_scale, w3_packed, w3_scale, w2_packed,
              w2_scale, *, top_k: int, routed_scaling_factor: float, renormalize: bool = True):
    """The Kimi-Linear grouped MoE block (klinear/moe.py:278-334, 375-398) with
    MXFP4 expert banks: route, shared expert appended as the last bank entry,
    SwiGLU, W2 per route, fp32 weighted sum -> bf16, + shared expert (bf16).
    Returns ``(y bf16 bits [T, H], idx [T, k], w [T, k])``."""
    from . import moe as OM

    num_routed = w1_packed.shape[0] - 1
    idx, w = OM.route(logits, bias, top_k, routed_scaling_factor=routed_scaling_factor,
                      renormalize=renormalize)
    stable = OM.shape_stable_expert_indices(idx, num_routed)
    act = swiglu(x_bits, stable, w1_packed, w1_scale, w3_packed, w3_scale)
    t_count = act.shape[0]
    eo = grouped(act.reshape(t_count * (top_k + 1), -1), stable.reshape(-1, 1), w2_packed,
                 w2_scale).reshape(t_count, top_k + 1, -1)
    full_w = np.concatenate((w, np.ones((t_count, 1), dtype=np.float32)), axis=1)
    return OM.combine(eo, full_w), idx, w


def situ(gate_bits, up_bits, beta: float = 4.0, linear_beta: float | None = 25.0) -> np.ndarray:
    """K3's SiTU in float32, rounded once to bf16 (kernels/moe_grouped.py:163-178):
    ``beta * tanh(g / beta) * sigmoid(g) * (linear_beta * tanh(u / linear_beta))``;
    without ``linear_beta`` the up term is ``u``."""
    g = bf16_bits_to_f32(gate_bits).astype(np.float32)
    u = bf16_bits_to_f32(up_bits).astype(np.float32)
    b = np.float32(beta)
    with np.errstate(over="ignore"):
        sig = (np.float32(1.0) / (np.float32(1.0) + np.exp(-g))).astype(np.float32)
    ag = (b * np.tanh(g / b)).astype(np.float32) * sig
    if linear_beta is not None:
        lb = np.float32(linear_beta)
        u = (lb * np.tanh(u / lb)).astype(np.float32)
    return f32_to_bf16_bits((ag * u).astype(np.float32))


def expert_mlp(x_bits, w1_packed, w1_scale, w3_packed, w3_scale, w2_packed, w2_scale,
               beta: float = 4.0, linear_beta: float | None = 25.0) -> np.ndarray:
    """One packed expert: gate / up projections, SiTU, down projection
    (kernels/moe_grouped.py:181-194, kernels/reference.py:101-116)."""
    gate = linear(x_bits, w1_packed, w1_scale)
    up = linear(x_bits, w3_packed, w3_scale)
    act = situ(gate, up, beta, linear_beta)
    return linear(act, w2_packed, w2_scale)


# ---------------------------------------------------------------------------
# fp8 activation split for the scaled fp4 MFMA. This build's own encoding (the
# reference multiplies bf16 activations by decoded weights and has no fp8
# step): per block of 32 values along K, x ~= hi * 2**e_hi + lo * 2**e_lo with
# hi and lo OCP FP8 E4M3 codes and E8M0 exponents e + 127.
#   e     = clamp(E(amax) - 7, -127, 127), E(a) = the float32 exponent field
#           minus 127 (floor(log2 a) for normal a, -127 for zero/subnormal),
#           so the scaled block max lies in [128, 256) and never saturates;
#   codes = round to nearest, ties to even, on the E4M3 grid; magnitudes below
#           2**-6 (the smallest normal) flush to a signed zero;
#   lo    = the same encoding of the exact residual x - hi * 2**e_hi.
# Pinned in tests by brute force over the E4M3 grid and by reconstruction
# bounds; the scaled MFMA consumes it (gfx950 v_mfma_scale_f32_16x16x128_f8f6f4).

E4M3_MIN_NORMAL = 2.0 ** -6


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """float64 values of OCP E4M3 codes (bias 7, subnormals m/8 * 2**-6)."""
    c = np.asarray(codes, dtype=np.int64)
    e = (c >> 3) & 15
    m = c & 7
    mag = np.where(e > 0, np.ldexp(1.0 + m / 8.0, e - 7), np.ldexp(m / 8.0, -6))
    return np.where(c & 0x80, -mag, mag)


def e4m3_encode(v: np.ndarray) -> np.ndarray:
    """E4M3 codes of float32 values with |v| < 448: nearest, ties to even,
    |v| < 2**-6 flushed to signed zero (float32 bit arithmetic)."""
    u = np.asarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    sign = (u >> 24) & 0x80
    a = u & 0x7FFFFFFF
    r = a + 0x7FFFF + ((a >> 20) & 1)
    code = sign | ((((r >> 23) - 120) & 15) << 3) | ((r >> 20) & 7)
    return np.where(a < 0x3C800000, sign, code).astype(np.uint8)


def _block_exponent(amax: np.ndarray) -> np.ndarray:
    field = (np.asarray(amax, dtype=np.float32).view(np.uint32) >> 23).astype(np.int64) & 0xFF
    return np.clip(field - 127 - 7, -127, 127)


def _split_once(x: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(codes [M, K], exponents [M, K/32], exact residual float32 [M, K])."""
    m, k = x.shape
    xb = x.reshape(m, k // GROUP, GROUP)
    e = _block_exponent(np.abs(xb).max(-1))
    scaled = (xb * np.ldexp(np.float32(1.0), -e)[..., None].astype(np.float32)).astype(np.float32)
    codes = e4m3_encode(scaled)
    val = (e4m3_decode(codes) * np.ldexp(1.0, e)[..., None]).astype(np.float32)
    resid = (xb - val).astype(np.float32)
    return codes.reshape(m, k), e, resid.reshape(m, k)


def split_fp8(x_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """bf16 bits [M, K] -> (hi u8 [M, K], lo u8 [M, K], scales u16 [M, K/32] with
    byte 0 = hi exponent + 127 and byte 1 = lo exponent + 127)."""
    x = bf16_bits_to_f32(np.asarray(x_bits, dtype=np.uint16))
    if x.shape[-1] % GROUP:
        raise ValueError("the fp8 split needs K % 32 == 0")
    hi, e_hi, resid = _split_once(x)
    lo, e_lo, _ = _split_once(resid)
    sc = ((e_hi + EXP_BIAS) | ((e_lo + EXP_BIAS) << 8)).astype(np.uint16)
    return hi, lo, sc


def split_decode(hi: np.ndarray, lo: np.ndarray, sc: np.ndarray) -> np.ndarray:
    """float64 hi * 2**e_hi + lo * 2**e_lo."""
    s = np.asarray(sc, dtype=np.int64)
    e_hi = np.repeat((s & 0xFF) - EXP_BIAS, GROUP, axis=-1)
    e_lo = np.repeat((s >> 8) - EXP_BIAS, GROUP, axis=-1)
    return e4m3_decode(hi) * np.ldexp(1.0, e_hi) + e4m3_decode(lo) * np.ldexp(1.0, e_lo)
