"""Router and the whole W4A16 MoE block on HIP.

``moe_router`` restates engine/klinear/router.py:47-85 on precomputed fp32
logits; ``w4a16_moe_block`` is the grouped branch of KLinearMoE.forward
(engine/klinear/moe.py:278-334, 375-398): route, gate/up + SwiGLU over the
top-k routes and the shared expert, W2, weighted combine plus shared expert.
Batch-1 decode runs in two launches (router + gate/up + SwiGLU, then W2 +
combine). From ``MOE_EXPERT_MAJOR_MIN_TOKENS`` tokens the block runs
expert-major: router, a counting-sort schedule of the routes by expert
(engine/kernels/moe_grouped.py:77-160), an MFMA gate/up + SwiGLU GEMM over
64-row expert tiles, the down GEMM scattered back to (token, route) rows and
the combine. The reference variant composes the reference ops.

Expert banks hold the routed experts first and the shared expert last
(``[E_routed + 1, ...]``), exactly as ``prepare_grouped_w4a16`` stacks them
(engine/klinear/moe.py:253-267).
"""

from __future__ import annotations

import torch

from .. import _lib
from . import w4a16 as _w


# tokens from which the MoE block runs expert-major (each expert read once).
# Below it the token-major kernels win: at the Kimi-Linear shape with
# Zipf(1.1) routing, 3 tokens take 39.3 us token-major vs 44.1 us
# expert-major, 4 tokens 47.7 us vs 46.2 us, 6 tokens 65.8 us vs 51.9 us (the
# expert-major chain has a floor of about 40 us: router, schedule, two
# persistent GEMMs, combine).
MOE_EXPERT_MAJOR_MIN_TOKENS = 4
# bank entries (routed + shared) the expert-major schedule supports
MOE_EXPERT_MAJOR_MAX_EXPERTS = 512


def moe_schedule(expert_indices: torch.Tensor, experts: int, shared_expert: int = -1,
                 tile_rows: int = 64):
    """Expert-major schedule of a route table on the GPU.

    Returns ``(offsets int32 [E+2], perm int32 [T*R], tiles int32 [n, 4],
    tile_count int32 [1])`` with ``R = routes (+1 if shared_expert >= 0)``;
    see ``lk_moe_schedule`` in include/lk_w4a16.h for the table contracts.
    """
    if expert_indices.ndim != 2 or expert_indices.dtype != torch.long:
        raise TypeError("expert_indices must be an int64 [tokens, routes] matrix")
    if expert_indices.device.type != "cuda":
        raise ValueError("the HIP schedule requires CUDA")
    tokens, routes = expert_indices.shape
    r_total = routes + (1 if shared_expert >= 0 else 0)
    max_tiles, ws_bytes = _lib.schedule_sizes(tokens, r_total, experts)
    dev = expert_indices.device
    offsets = torch.empty((experts + 2,), dtype=torch.int32, device=dev)
    perm = torch.empty((tokens * r_total,), dtype=torch.int32, device=dev)
    tiles = torch.empty((max_tiles, 4), dtype=torch.int32, device=dev)
    count = torch.empty((1,), dtype=torch.int32, device=dev)
    ws = _w.workspace(ws_bytes, dev)
    idx = _w._c(expert_indices)
    with torch.cuda.device(dev):
        _lib.call("lk_moe_schedule", idx.data_ptr(), tokens, routes, experts, shared_expert,
                  tile_rows, offsets.data_ptr(), perm.data_ptr(), tiles.data_ptr(), count.data_ptr(),
                  ws.data_ptr(), ws.numel(), _w._stream(dev))
    return offsets, perm, tiles, count


def shape_stable_expert_indices(expert_indices: torch.Tensor, shared_expert_id: int) -> torch.Tensor:
    """Append the shared expert as one fixed route for every token (moe.py:23-36)."""
    if expert_indices.ndim != 2:
        raise ValueError("expert_indices must have shape [tokens, routes]")
    shared = torch.full((expert_indices.shape[0], 1), shared_expert_id,
                        dtype=expert_indices.dtype, device=expert_indices.device)
    return torch.cat((expert_indices, shared), dim=1)


def _validate_router(logits: torch.Tensor, bias: torch.Tensor | None, top_k: int):
    if logits.ndim != 2 or logits.dtype != torch.float32:
        raise TypeError("router logits must be a float32 [tokens, experts] matrix")
    if logits.device.type != "cuda":
        raise ValueError("the HIP router requires CUDA")
    tokens, experts = logits.shape
    if experts == 0 or experts > 1024:
        raise ValueError("the HIP router supports 1..1024 experts")
    if not 0 < top_k <= min(32, experts):
        raise ValueError(f"top_k must be in 1..{min(32, experts)}, got {top_k}")
    if bias is not None:
        if bias.dtype != torch.float32 or bias.shape != (experts,):
            raise TypeError("router bias must be a float32 [experts] vector")
        if bias.device != logits.device:
            raise ValueError("router bias must share the logits device")
    return tokens, experts


def moe_router(logits: torch.Tensor, bias: torch.Tensor | None, top_k: int, *,
               routed_scaling_factor: float = 1.0, renormalize: bool = True,
               num_expert_group: int = 1,
               topk_group: int = 1) -> tuple[torch.Tensor, torch.Tensor]:
    """Sigmoid top-k routing: ``(idx int64 [T, k], weights float32 [T, k])``.

    Selections are ordered by descending ``sigmoid(logit) + bias``, ties to the
    lower expert id; weights are the un-biased sigmoid scores, renormalised by
    ``sum + 1e-20`` (when ``top_k > 1`` and ``renormalize``) and scaled.
    ``num_expert_group > 1`` is the grouped top-k of router.py:62-80: groups
    ranked by the sum of their two largest choice scores, the best
    ``topk_group`` kept, every other expert's choice masked to 0.0.
    """
    tokens, experts = _validate_router(logits, bias, top_k)
    num_expert_group, topk_group = int(num_expert_group), int(topk_group)
    if num_expert_group < 1 or experts % num_expert_group:
        raise ValueError("num_experts must be divisible by num_expert_group")
    if num_expert_group > 1 and not 1 <= topk_group <= num_expert_group:
        raise ValueError("topk_group must lie in 1..num_expert_group")
    idx = torch.empty((tokens, top_k), dtype=torch.long, device=logits.device)
    w = torch.empty((tokens, top_k), dtype=torch.float32, device=logits.device)
    if tokens == 0:
        return idx, w
    lg = _w._c(logits)
    b = _w._c(bias) if bias is not None else None
    with torch.cuda.device(logits.device):
        if num_expert_group > 1:
            _lib.call("lk_moe_router_grouped", lg.data_ptr(),
                      b.data_ptr() if b is not None else None, idx.data_ptr(), w.data_ptr(),
                      tokens, experts, top_k, num_expert_group, topk_group,
                      float(routed_scaling_factor), int(bool(renormalize)),
                      _w._stream(logits.device))
        else:
            _lib.call("lk_moe_router", lg.data_ptr(), b.data_ptr() if b is not None else None,
                      idx.data_ptr(), w.data_ptr(), tokens, experts, top_k,
                      float(routed_scaling_factor), int(bool(renormalize)),
                      _w._stream(logits.device))
    return idx, w


def router_logits(hidden: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``fp32(hidden) @ fp32(weight).T`` -> float32 ``[T, E]`` (router.py:50-51).

    bf16 ``hidden [T, H]`` with ``H % 8 == 0`` and ``H <= 4096``, and a router
    ``weight [E, H]`` in bf16 or fp32 (fp16 is widened to fp32 first, which is
    exact), on the GPU: one HIP launch for any token count. Every logit is
    summed in the same fixed order whatever the batch size, so a token's
    logits, and therefore its expert selection, do not depend on how many
    tokens share the call.
    """
    if hidden.ndim != 2 or weight.ndim != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError("router logits need hidden [T, H] and weight [E, H]")
    if hidden.dtype != torch.bfloat16:
        raise TypeError("router logits need BF16 hidden states")
    if weight.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError("the router weight must be BF16, FP16 or FP32")
    if hidden.device != weight.device:
        raise ValueError("router inputs must share one device")
    if hidden.device.type != "cuda":
        raise ValueError("the HIP router logits require CUDA")
    tokens, h = hidden.shape
    experts = weight.shape[0]
    if h % 8 or h > 4096 or experts == 0:
        raise ValueError(f"router logits need 0 < experts and hidden % 8 == 0, hidden <= 4096; "
                         f"got hidden {h}, experts {experts}")
    out = torch.empty((tokens, experts), dtype=torch.float32, device=hidden.device)
    if tokens == 0:
        return out
    if weight.dtype == torch.float16:
        weight = weight.float()
    x, w = _w._c(hidden), _w._c(weight)
    with torch.cuda.device(hidden.device):
        _lib.call("lk_router_logits", x.data_ptr(), w.data_ptr(), out.data_ptr(), tokens, experts, h,
                  int(w.dtype == torch.float32), _w._stream(hidden.device))
    return out


def _validate_stage1(hidden, logits, bias, w1_packed, w1_scales, w3_packed, w3_scales, top_k):
    if hidden.ndim != 2 or hidden.dtype != torch.bfloat16:
        raise TypeError("hidden states must be a BF16 [tokens, hidden] matrix")
    tokens, h = hidden.shape
    _validate_router(logits, bias, top_k)
    if logits.shape[0] != tokens:
        raise ValueError("router logits must have one row per token")
    e1, inter, k1, g1 = _w.check_bank(w1_packed, w1_scales, "W1")
    e3, inter3, k3, g3 = _w.check_bank(w3_packed, w3_scales, "W3")
    if (e1, inter, k1, g1) != (e3, inter3, k3, g3):
        raise ValueError("grouped W1 and W3 dimensions must match")
    if k1 != h:
        raise ValueError("W1/W3 reduction width must equal the hidden size")
    if logits.shape[1] != e1 - 1:
        raise ValueError("banks must hold every routed expert plus the shared expert last")
    if w1_packed.device != hidden.device or w3_packed.device != hidden.device or \
            logits.device != hidden.device:
        raise ValueError("MoE inputs must share one device")
    return tokens, e1, h, inter, g1


def _validate_block(hidden, logits, bias, w1_packed, w1_scales, w3_packed, w3_scales,
                    w2_packed, w2_scales, top_k):
    tokens, e_total, h, inter, g1 = _validate_stage1(hidden, logits, bias, w1_packed, w1_scales,
                                                     w3_packed, w3_scales, top_k)
    e2, h2, k2, g2 = _w.check_bank(w2_packed, w2_scales, "W2")
    if e2 != e_total:
        raise ValueError("W2 bank must have the same expert count as W1/W3")
    if h2 != h or k2 != inter:
        raise ValueError("W2 must map the intermediate size back to the hidden size")
    if g1 != g2:
        raise ValueError("W1/W3 and W2 must use the same group size")
    if w2_packed.device != hidden.device:
        raise ValueError("MoE inputs must share one device")
    return tokens, e_total, h, inter, g1


def w4a16_moe_block(hidden: torch.Tensor, logits: torch.Tensor, bias: torch.Tensor | None,
                    w1_packed, w1_scales, w3_packed, w3_scales, w2_packed, w2_scales, top_k: int,
                    routed_scaling_factor: float = 1.0, renormalize: bool = True, *,
                    num_expert_group: int = 1, topk_group: int = 1):
    """Router + SwiGLU experts + W2 + combine + shared expert on HIP.

    Fewer than ``MOE_EXPERT_MAJOR_MIN_TOKENS`` tokens: two launches per call
    (token-major decode). More tokens: the expert-major path
    (:func:`w4a16_moe_forward`). Grouped top-k routing (``num_expert_group >
    1``) routes with :func:`moe_router` first, then runs
    :func:`w4a16_moe_routed` on those routes.
    Returns ``(y bf16 [T, H], expert_indices int64 [T, k], weights float32 [T, k])``.
    """
    if num_expert_group != 1:
        _validate_block(hidden, logits, bias, w1_packed, w1_scales, w3_packed, w3_scales,
                        w2_packed, w2_scales, top_k)
        idx, w = moe_router(logits, bias, top_k, routed_scaling_factor=routed_scaling_factor,
                            renormalize=renormalize, num_expert_group=num_expert_group,
                            topk_group=topk_group)
        y = w4a16_moe_routed(hidden, idx, w, w1_packed, w1_scales, w3_packed, w3_scales,
                             w2_packed, w2_scales)
        return y, idx, w
    expert_major_fits = hidden.ndim == 2 and w1_packed.ndim == 3 and \
        w1_packed.shape[0] <= MOE_EXPERT_MAJOR_MAX_EXPERTS
    if expert_major_fits and (hidden.shape[0] >= MOE_EXPERT_MAJOR_MIN_TOKENS or
                              not decode_supported(w1_packed, top_k)):
        return w4a16_moe_forward(hidden, logits, bias, w1_packed, w1_scales, w3_packed, w3_scales,
                                 w2_packed, w2_scales, top_k, routed_scaling_factor, renormalize)
    return w4a16_moe_decode(hidden, logits, bias, w1_packed, w1_scales, w3_packed, w3_scales,
                            w2_packed, w2_scales, top_k, routed_scaling_factor, renormalize)


def w4a16_moe_routed(hidden: torch.Tensor, expert_indices: torch.Tensor,
                     combine_weights: torch.Tensor, w1_packed, w1_scales, w3_packed, w3_scales,
                     w2_packed, w2_scales) -> torch.Tensor:
    """The block on routes chosen elsewhere (klinear/moe.py:278-334's sequence).

    ``expert_indices`` int64 ``[T, k]`` into the routed experts and
    ``combine_weights`` float32 ``[T, k]``; the shared expert (bank entry
    ``E - 1``) is appended as a last route of weight 1. Gate/up + SwiGLU on the
    ``[T, k + 1]`` routes (GEMV or expert-major GEMM by size), then W2 with the
    weighted combine in one launch for small batches, or the grouped W2 over
    ``[T (k + 1), I]`` single-route rows and the route combine.
    Returns ``y`` bf16 ``[T, H]``.
    """
    e_total = w1_packed.shape[0]
    if expert_indices.ndim != 2 or expert_indices.dtype != torch.long:
        raise TypeError("expert_indices must be an int64 [tokens, top_k] matrix")
    if combine_weights.dtype != torch.float32 or combine_weights.shape != expert_indices.shape:
        raise TypeError("combine_weights must be a float32 matrix shaped like expert_indices")
    tokens, top_k = expert_indices.shape
    if hidden.ndim != 2 or hidden.shape[0] != tokens:
        raise ValueError("hidden states must be [tokens, hidden] with one row per route row")
    stable = shape_stable_expert_indices(expert_indices, e_total - 1)
    act = _w.grouped_w4a16_swiglu_gemv(hidden, stable, w1_packed, w1_scales, w3_packed,
                                       w3_scales)
    cw = torch.cat((combine_weights,
                    torch.ones((tokens, 1), dtype=torch.float32, device=combine_weights.device)),
                   dim=1)
    inter = act.shape[-1]
    if tokens < MOE_EXPERT_MAJOR_MIN_TOKENS and decode_supported(w1_packed, top_k):
        return _w.fused_w2_combine(act.reshape(tokens, top_k + 1, inter), stable, cw, w2_packed,
                                   w2_scales)
    eo = _w.grouped_w4a16_gemv(act.reshape(tokens * (top_k + 1), inter),
                               stable.reshape(tokens * (top_k + 1), 1), w2_packed, w2_scales)
    return _w.route_combine(eo.reshape(tokens, top_k + 1, -1), cw)


def decode_supported(w1_packed: torch.Tensor, top_k: int) -> bool:
    """Whether the token-major decode path takes ``top_k + 1`` routes at this bank's
    intermediate size (its W2 + combine launch has a route limit; the
    expert-major path has none)."""
    if w1_packed.ndim != 3:
        return False
    experts, inter, packed_h = w1_packed.shape
    return int(_lib.load().lk_w4a16_moe_decode_workspace(1, experts, packed_h * 2, inter,
                                                          top_k)) >= 0


def w4a16_moe_forward(hidden: torch.Tensor, logits: torch.Tensor, bias: torch.Tensor | None,
                      w1_packed, w1_scales, w3_packed, w3_scales, w2_packed, w2_scales,
                      top_k: int, routed_scaling_factor: float = 1.0, renormalize: bool = True):
    """The expert-major block (router, schedule, two MFMA GEMMs, combine)."""
    tokens, e_total, h, inter, g = _validate_block(hidden, logits, bias, w1_packed, w1_scales,
                                                   w3_packed, w3_scales, w2_packed, w2_scales, top_k)
    dev = hidden.device
    y = torch.empty((tokens, h), dtype=torch.bfloat16, device=dev)
    idx = torch.empty((tokens, top_k), dtype=torch.long, device=dev)
    w = torch.empty((tokens, top_k), dtype=torch.float32, device=dev)
    if tokens == 0:
        return y, idx, w
    ws = _w.workspace(_lib.query("lk_w4a16_moe_forward_workspace", tokens, e_total, h, inter,
                                 top_k), dev)
    c = _w._c
    x, lg = c(hidden), c(logits)
    b = c(bias) if bias is not None else None
    args = [c(t) for t in (w1_packed, w1_scales, w3_packed, w3_scales, w2_packed, w2_scales)]
    with torch.cuda.device(dev):
        _lib.call("lk_w4a16_moe_forward", x.data_ptr(), lg.data_ptr(),
                  b.data_ptr() if b is not None else None, *(t.data_ptr() for t in args),
                  y.data_ptr(), idx.data_ptr(), w.data_ptr(), ws.data_ptr(), ws.numel(), tokens,
                  e_total, h, inter, top_k, float(routed_scaling_factor), int(bool(renormalize)),
                  g, _w._stream(dev))
    return y, idx, w


def w4a16_moe_decode(hidden: torch.Tensor, logits: torch.Tensor, bias: torch.Tensor | None,
                     w1_packed, w1_scales, w3_packed, w3_scales, w2_packed, w2_scales, top_k: int,
                     routed_scaling_factor: float = 1.0, renormalize: bool = True):
    """The token-major block in two launches (any token count; fastest at one).

    Its W2 + combine launch takes ``top_k + 1`` routes with either intermediate
    size 1024 and at most 16 routes, or at most 32 routes whose staged
    activations fit 64 KiB (``routes * (I / 32 * 68 + 32)`` bytes); other
    shapes raise ValueError (``w4a16_moe_block`` sends them expert-major).
    """
    tokens, e_total, h, inter, g = _validate_block(hidden, logits, bias, w1_packed, w1_scales,
                                                   w3_packed, w3_scales, w2_packed, w2_scales, top_k)
    if _lib.load().lk_w4a16_moe_decode_workspace(tokens, e_total, h, inter, top_k) < 0:
        raise ValueError(f"the token-major decode path does not take top_k={top_k} at "
                         f"intermediate size {inter}; use w4a16_moe_forward")
    dev = hidden.device
    y = torch.empty((tokens, h), dtype=torch.bfloat16, device=dev)
    idx = torch.empty((tokens, top_k), dtype=torch.long, device=dev)
    w = torch.empty((tokens, top_k), dtype=torch.float32, device=dev)
    if tokens == 0:
        return y, idx, w
    act = torch.empty((tokens, top_k + 1, inter), dtype=torch.bfloat16, device=dev)
    c = _w._c
    x, lg = c(hidden), c(logits)
    b = c(bias) if bias is not None else None
    args = [c(t) for t in (w1_packed, w1_scales, w3_packed, w3_scales, w2_packed, w2_scales)]
    with torch.cuda.device(dev):
        _lib.call("lk_w4a16_moe_decode", x.data_ptr(), lg.data_ptr(),
                  b.data_ptr() if b is not None else None, *(t.data_ptr() for t in args),
                  y.data_ptr(), idx.data_ptr(), w.data_ptr(), act.data_ptr(), tokens, e_total, h,
                  inter, top_k, float(routed_scaling_factor), int(bool(renormalize)), g,
                  _w._stream(dev))
    return y, idx, w


def w4a16_moe_gateup(hidden: torch.Tensor, logits: torch.Tensor, bias: torch.Tensor | None,
                     w1_packed, w1_scales, w3_packed, w3_scales, top_k: int,
                     routed_scaling_factor: float = 1.0, renormalize: bool = True):
    """First stage of the block in one launch: router + gate/up + SwiGLU.

    Returns ``(activated bf16 [T, k+1, I], expert_indices [T, k], weights [T, k])``;
    route ``k`` of ``activated`` is the shared expert.
    """
    tokens, e_total, h, inter, g = _validate_stage1(hidden, logits, bias, w1_packed, w1_scales,
                                                    w3_packed, w3_scales, top_k)
    dev = hidden.device
    act = torch.empty((tokens, top_k + 1, inter), dtype=torch.bfloat16, device=dev)
    idx = torch.empty((tokens, top_k), dtype=torch.long, device=dev)
    w = torch.empty((tokens, top_k), dtype=torch.float32, device=dev)
    if tokens == 0:
        return act, idx, w
    c = _w._c
    x, lg = c(hidden), c(logits)
    b = c(bias) if bias is not None else None
    args = [c(t) for t in (w1_packed, w1_scales, w3_packed, w3_scales)]
    with torch.cuda.device(dev):
        _lib.call("lk_w4a16_moe_gateup", x.data_ptr(), lg.data_ptr(),
                  b.data_ptr() if b is not None else None, *(t.data_ptr() for t in args),
                  idx.data_ptr(), w.data_ptr(), act.data_ptr(), tokens, e_total, h, inter, top_k,
                  float(routed_scaling_factor), int(bool(renormalize)), g, _w._stream(dev))
    return act, idx, w


def w4a16_moe_block_reference(hidden, logits, bias, w1_packed, w1_scales, w3_packed, w3_scales,
                              w2_packed, w2_scales, top_k: int, routed_scaling_factor: float = 1.0,
                              renormalize: bool = True, *, num_expert_group: int = 1,
                              topk_group: int = 1):
    """The same block composed from the reference-rounding ops (moe.py:278-334)."""
    tokens, e_total, h, inter, _ = _validate_block(hidden, logits, bias, w1_packed, w1_scales,
                                                   w3_packed, w3_scales, w2_packed, w2_scales, top_k)
    idx, w = moe_router(logits, bias, top_k, routed_scaling_factor=routed_scaling_factor,
                        renormalize=renormalize, num_expert_group=num_expert_group,
                        topk_group=topk_group)
    stable = shape_stable_expert_indices(idx, e_total - 1)
    gate = _w.grouped_w4a16_reference(hidden, stable, w1_packed, w1_scales)
    up = _w.grouped_w4a16_reference(hidden, stable, w3_packed, w3_scales)
    act = _w.silu_mul(gate, up)
    cw = torch.cat((w, torch.ones((tokens, 1), dtype=torch.float32, device=w.device)), dim=1)
    y = _w.fused_w2_combine_reference(act, stable, cw, w2_packed, w2_scales)
    return y, idx, w
