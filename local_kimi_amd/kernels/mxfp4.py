"""MXFP4 expert ops on HIP: the GEMM op, grouped banks, the MoE block, the K3 expert MLP.

``mxfp4_gemm`` keeps the reference op's signature and validation
(engine/kernels/mxfp4_gemm.py:158-226): ``activations [M, K]`` bf16 or fp16,
``weight_packed [N, K/2]`` uint8 E2M1 (low nibble first), ``weight_scale
[N, K/32]`` uint8 E8M0 -> ``[M, N]`` in the activation dtype. Weights are
decoded by the gfx950 scaled convert (exact) and multiplied on the bf16 / fp16
matrix cores with fp32 accumulation.

Grouped banks stack experts on a leading axis; the MoE block is the
Kimi-Linear SwiGLU block of :mod:`.moe` with MXFP4 banks (shared expert
last). Its expert GEMMs run bf16 MFMA on weights decoded by the scaled
convert; the path knob ``mxfp4_mfma=fp4`` selects the gfx950 scaled fp4 MFMA
instead (raw E2M1 weights with their E8M0 exponents, activations split into
fp8 hi + lo by :func:`split_activations_fp8` so the product keeps bf16
activation precision), which measured slower at every batch size.
``mxfp4_expert_mlp`` is the K3 packed expert with SiTU
(engine/kernels/moe_grouped.py:163-194).
"""

from __future__ import annotations

import torch

from .. import _lib
from . import moe as _moe
from . import w4a16 as _w

MXFP4_GROUP_SIZE = 32


def _validate_gemm(activations, weight_packed, weight_scale) -> tuple[int, int, int]:
    """engine/kernels/mxfp4_gemm.py:158-188, message for message."""
    if activations.ndim != 2:
        raise ValueError("activations must have shape [tokens, reduction]")
    if weight_packed.ndim != 2 or weight_scale.ndim != 2:
        raise ValueError("packed weights and scales must both be matrices")
    if activations.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("activations must use torch.float16 or torch.bfloat16")
    if weight_packed.dtype != torch.uint8 or weight_scale.dtype != torch.uint8:
        raise TypeError("packed weights and scales must both use torch.uint8")
    if activations.device.type != "cuda":
        raise ValueError("the fused MXFP4 GEMM requires CUDA activations")
    if not (activations.device == weight_packed.device == weight_scale.device):
        raise ValueError("activations, packed weights, and scales must share a device")
    m, k = activations.shape
    n, packed_k = weight_packed.shape
    if k == 0 or n == 0:
        raise ValueError("reduction and output dimensions must be nonzero")
    if k % MXFP4_GROUP_SIZE != 0:
        raise ValueError("MXFP4 reduction dimension must be divisible by 32")
    if packed_k * 2 != k:
        raise ValueError("packed weight shape does not match the reduction dimension")
    if weight_scale.shape != (n, k // MXFP4_GROUP_SIZE):
        raise ValueError("scale shape must provide one byte per 32 reduction values")
    return m, n, k


def _gemm(entry: str, activations, weight_packed, weight_scale) -> torch.Tensor:
    m, n, k = _validate_gemm(activations, weight_packed, weight_scale)
    out = torch.empty((m, n), dtype=activations.dtype, device=activations.device)
    if m == 0:
        return out
    x, p, s = _w._c(activations), _w._c(weight_packed), _w._c(weight_scale)
    with torch.cuda.device(activations.device):
        _lib.call(entry, x.data_ptr(), p.data_ptr(), s.data_ptr(), out.data_ptr(), m, n, k,
                  int(activations.dtype == torch.float16), _w._stream(activations.device))
    return out


def mxfp4_gemm(activations: torch.Tensor, weight_packed: torch.Tensor,
               weight_scale: torch.Tensor) -> torch.Tensor:
    """``activations @ dequant(weight).T`` without a decoded weight tensor."""
    return _gemm("lk_mxfp4_gemm", activations, weight_packed, weight_scale)


def mxfp4_linear(activations, weight_packed, weight_scale) -> torch.Tensor:
    """Linear-style name for callers that store weights as output-by-input."""
    return mxfp4_gemm(activations, weight_packed, weight_scale)


def mxfp4_gemm_reference(activations, weight_packed, weight_scale) -> torch.Tensor:
    """Decode each weight to the activation dtype, fp32 dot (one thread per output)."""
    return _gemm("lk_mxfp4_gemm_reference", activations, weight_packed, weight_scale)


def check_mx_bank(packed: torch.Tensor, scale: torch.Tensor, what: str) -> tuple[int, int, int]:
    """``(E, N, K)`` of a grouped MXFP4 bank ``[E, N, K/2]`` + ``[E, N, K/32]``."""
    if packed.ndim != 3 or scale.ndim != 3:
        raise ValueError(f"{what} packed weights and scales must be rank three")
    if packed.dtype != torch.uint8 or scale.dtype != torch.uint8:
        raise TypeError(f"{what} packed weights and scales must both use torch.uint8")
    if packed.device != scale.device:
        raise ValueError(f"{what} packed weights and scales must share a device")
    e, n, packed_k = packed.shape
    k = packed_k * 2
    if e == 0 or n == 0 or k == 0:
        raise ValueError(f"{what} bank requires nonzero dimensions")
    if k % MXFP4_GROUP_SIZE:
        raise ValueError("MXFP4 reduction dimension must be divisible by 32")
    if scale.shape != (e, n, k // MXFP4_GROUP_SIZE):
        raise ValueError(f"{what} scale shape must provide one byte per 32 reduction values")
    return e, n, k


def _validate_grouped(activations, expert_indices, packed, scale, what="grouped MXFP4"):
    if activations.ndim != 2 or activations.dtype != torch.bfloat16:
        raise TypeError("activations must be a BF16 [tokens, reduction] matrix")
    if expert_indices.ndim != 2 or expert_indices.dtype != torch.long:
        raise TypeError("expert_indices must be an int64 [tokens, routes] matrix")
    if activations.device.type != "cuda":
        raise ValueError("grouped MXFP4 requires CUDA")
    e, n, k = check_mx_bank(packed, scale, what)
    if not (activations.device == expert_indices.device == packed.device):
        raise ValueError("grouped MXFP4 inputs must share one device")
    t, kk = activations.shape
    if expert_indices.shape[0] != t:
        raise ValueError("expert routing must have one row per token")
    if expert_indices.shape[1] == 0:
        raise ValueError("grouped MXFP4 requires nonzero dimensions")
    if kk != k:
        raise ValueError("packed grouped weights have the wrong reduction width")
    return t, expert_indices.shape[1], e, n, k


def grouped_mxfp4_gemm(activations, expert_indices, packed, scale) -> torch.Tensor:
    """``out[t, r] = x[t] @ dequant(W[idx[t, r]]).T`` -> ``[T, R, N]`` bf16, expert-major.

    Indices outside ``[0, E)`` give zero rows.
    """
    t, r, e, n, k = _validate_grouped(activations, expert_indices, packed, scale)
    out = torch.empty((t, r, n), dtype=torch.bfloat16, device=activations.device)
    if t == 0:
        return out
    x, idx, p, s = (_w._c(a) for a in (activations, expert_indices, packed, scale))
    with torch.cuda.device(x.device):
        ws = _w.workspace(_lib.query("lk_w4a16_grouped_gemm_workspace", t, r, e), x.device)
        _lib.call("lk_mxfp4_grouped_gemm", x.data_ptr(), idx.data_ptr(), p.data_ptr(),
                  s.data_ptr(), out.data_ptr(), t, r, e, n, k, ws.data_ptr(), ws.numel(),
                  _w._stream(x.device))
    return out


def grouped_mxfp4_swiglu_gemm(activations, expert_indices, w1_packed, w1_scale, w3_packed,
                              w3_scale) -> torch.Tensor:
    """``bf16(bf16(silu(bf16(x W1^T))) * bf16(x W3^T))`` per route, MXFP4 banks."""
    dims = _validate_grouped(activations, expert_indices, w1_packed, w1_scale, "W1")
    if _validate_grouped(activations, expert_indices, w3_packed, w3_scale, "W3") != dims:
        raise ValueError("grouped W1 and W3 dimensions must match")
    t, r, e, n, k = dims
    out = torch.empty((t, r, n), dtype=torch.bfloat16, device=activations.device)
    if t == 0:
        return out
    x, idx = _w._c(activations), _w._c(expert_indices)
    banks = [_w._c(a) for a in (w1_packed, w1_scale, w3_packed, w3_scale)]
    with torch.cuda.device(x.device):
        ws = _w.workspace(_lib.query("lk_w4a16_grouped_gemm_workspace", t, r, e), x.device)
        _lib.call("lk_mxfp4_swiglu_gemm", x.data_ptr(), idx.data_ptr(),
                  *(b.data_ptr() for b in banks), out.data_ptr(), t, r, e, n, k, ws.data_ptr(),
                  ws.numel(), _w._stream(x.device))
    return out


def split_activations_fp8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """bf16 ``[M, K]`` -> ``(hi uint8 [M, K], lo uint8 [M, K], scales int16 [M, K/32])``:
    per 32 values x ~= hi * 2**e_hi + lo * 2**e_lo (OCP E4M3 codes; scale word
    byte 0 = e_hi + 127, byte 1 = e_lo + 127)."""
    if x.ndim != 2 or x.dtype != torch.bfloat16:
        raise TypeError("the fp8 split takes a BF16 [rows, reduction] matrix")
    if x.device.type != "cuda":
        raise ValueError("the fp8 split requires CUDA tensors")
    m, k = x.shape
    if k == 0 or k % MXFP4_GROUP_SIZE:
        raise ValueError("the fp8 split needs a reduction width that is a nonzero multiple of 32")
    xc = _w._c(x)
    hi = torch.empty((m, k), dtype=torch.uint8, device=x.device)
    lo = torch.empty((m, k), dtype=torch.uint8, device=x.device)
    sc = torch.empty((m, k // MXFP4_GROUP_SIZE), dtype=torch.int16, device=x.device)
    if m:
        with torch.cuda.device(x.device):
            _lib.call("lk_mxfp4_split_activations", xc.data_ptr(), hi.data_ptr(), lo.data_ptr(),
                      sc.data_ptr(), m, k, _w._stream(x.device))
    return hi, lo, sc


def mxfp4_moe_block(hidden, logits, bias, w1_packed, w1_scale, w3_packed, w3_scale, w2_packed,
                    w2_scale, top_k: int, routed_scaling_factor: float = 1.0,
                    renormalize: bool = True):
    """Kimi-Linear MoE block (router, SwiGLU experts + shared expert, W2,
    combine) with MXFP4 banks ``[E_routed + 1, ...]``, expert-major on HIP.

    Returns ``(y bf16 [T, H], expert_indices int64 [T, k], weights float32 [T, k])``.
    """
    if hidden.ndim != 2 or hidden.dtype != torch.bfloat16:
        raise TypeError("hidden states must be a BF16 [tokens, hidden] matrix")
    tokens, h = hidden.shape
    _moe._validate_router(logits, bias, top_k)
    e1, inter, k1 = check_mx_bank(w1_packed, w1_scale, "W1")
    if check_mx_bank(w3_packed, w3_scale, "W3") != (e1, inter, k1):
        raise ValueError("grouped W1 and W3 dimensions must match")
    e2, h2, k2 = check_mx_bank(w2_packed, w2_scale, "W2")
    if k1 != h or (e2, h2, k2) != (e1, h, inter):
        raise ValueError("W1/W3 must map hidden -> intermediate and W2 back, with one expert count")
    if logits.shape != (tokens, e1 - 1):
        raise ValueError("banks must hold every routed expert plus the shared expert last")
    if len({t.device for t in (hidden, logits, w1_packed, w3_packed, w2_packed)}) != 1:
        raise ValueError("MoE inputs must share one device")
    dev = hidden.device
    y = torch.empty((tokens, h), dtype=torch.bfloat16, device=dev)
    idx = torch.empty((tokens, top_k), dtype=torch.long, device=dev)
    w = torch.empty((tokens, top_k), dtype=torch.float32, device=dev)
    if tokens == 0:
        return y, idx, w
    x, lg = _w._c(hidden), _w._c(logits)
    b = _w._c(bias) if bias is not None else None
    banks = [_w._c(a) for a in (w1_packed, w1_scale, w3_packed, w3_scale, w2_packed, w2_scale)]
    with torch.cuda.device(dev):
        ws = _w.workspace(_lib.query("lk_mxfp4_moe_forward_workspace", tokens, e1, h, inter,
                                     top_k), dev)
        _lib.call("lk_mxfp4_moe_forward", x.data_ptr(), lg.data_ptr(),
                  b.data_ptr() if b is not None else None, *(a.data_ptr() for a in banks),
                  y.data_ptr(), idx.data_ptr(), w.data_ptr(), ws.data_ptr(), ws.numel(), tokens,
                  e1, h, inter, top_k, float(routed_scaling_factor), int(bool(renormalize)),
                  _w._stream(dev))
    return y, idx, w


def mxfp4_expert_mlp(hidden_states: torch.Tensor, weights, *, situ_beta: float = 4.0,
                     situ_linear_beta: float | None = 25.0) -> torch.Tensor:
    """One K3 routed expert with packed weights (moe_grouped.py:181-194).

    ``weights`` carries ``w1_packed, w1_scale, w3_packed, w3_scale, w2_packed,
    w2_scale`` as in the reference's ``PackedExpertWeights``.
    """
    if hidden_states.ndim != 2 or hidden_states.dtype != torch.bfloat16:
        raise TypeError("hidden states must be a BF16 [tokens, hidden] matrix")
    m, h = hidden_states.shape
    mats = [weights.w1_packed, weights.w1_scale, weights.w3_packed, weights.w3_scale,
            weights.w2_packed, weights.w2_scale]
    i = _validate_gemm(hidden_states, mats[0], mats[1])[1]
    if _validate_gemm(hidden_states, mats[2], mats[3])[1] != i:
        raise ValueError("gate and up projections must have the same width")
    probe = torch.empty((0, i), dtype=torch.bfloat16, device=hidden_states.device)
    if _validate_gemm(probe, mats[4], mats[5])[1] != h:
        raise ValueError("down projection must map back to the hidden size")
    if situ_beta == 0:
        raise ValueError("situ_beta must be nonzero")
    dev = hidden_states.device
    y = torch.empty((m, h), dtype=torch.bfloat16, device=dev)
    if m == 0:
        return y
    act = torch.empty((m, i), dtype=torch.bfloat16, device=dev)
    x = _w._c(hidden_states)
    mats = [_w._c(a) for a in mats]
    lb = -1.0 if situ_linear_beta is None else float(situ_linear_beta)
    if situ_linear_beta is not None and situ_linear_beta <= 0:
        raise ValueError("situ_linear_beta must be positive or None")
    with torch.cuda.device(dev):
        _lib.call("lk_mxfp4_expert_mlp", x.data_ptr(), *(a.data_ptr() for a in mats), y.data_ptr(),
                  act.data_ptr(), m, h, i, float(situ_beta), lb, _w._stream(dev))
    return y


def grouped_mxfp4_reference(activations, expert_indices, packed, scale) -> torch.Tensor:
    """Per-expert reference GEMMs over the gathered rows (kernels/reference.py:119-165)."""
    t, r, e, n, k = _validate_grouped(activations, expert_indices, packed, scale)
    out = torch.zeros((t, r, n), dtype=torch.bfloat16, device=activations.device)
    flat = expert_indices.reshape(-1)
    rows = activations.repeat_interleave(r, dim=0)
    for expert in torch.unique(flat).tolist():
        if not 0 <= expert < e:
            continue
        sel = (flat == expert).nonzero().reshape(-1)
        out.view(t * r, n)[sel] = mxfp4_gemm_reference(rows[sel].contiguous(), packed[expert],
                                                       scale[expert])
    return out


def mxfp4_moe_block_reference(hidden, logits, bias, w1_packed, w1_scale, w3_packed, w3_scale,
                              w2_packed, w2_scale, top_k: int, routed_scaling_factor: float = 1.0,
                              renormalize: bool = True):
    """The same block from reference GEMMs: router, gate / up, silu * up, W2, combine."""
    e_total = w1_packed.shape[0]
    idx, w = _moe.moe_router(logits, bias, top_k, routed_scaling_factor=routed_scaling_factor,
                             renormalize=renormalize)
    stable = _moe.shape_stable_expert_indices(idx, e_total - 1)
    gate = grouped_mxfp4_reference(hidden, stable, w1_packed, w1_scale)
    up = grouped_mxfp4_reference(hidden, stable, w3_packed, w3_scale)
    act = _w.silu_mul(gate, up)
    t, r, i = act.shape
    eo = grouped_mxfp4_reference(act.reshape(t * r, i), stable.reshape(-1, 1), w2_packed,
                                 w2_scale).reshape(t, r, -1)
    cw = torch.cat((w, torch.ones((t, 1), dtype=torch.float32, device=w.device)), dim=1)
    return _w.route_combine(eo, cw), idx, w
