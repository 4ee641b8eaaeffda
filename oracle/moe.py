"""Router, route bookkeeping, W2 combine and the whole W4A16 MoE block (numpy).

Selection order policy: the reference takes ``topk(..., sorted=False)``
(klinear/router.py:81), whose slot order is implementation-defined. The oracle
(and the HIP router) fix one documented order: descending choice score, ties
to the lower expert id. Parity on indices compares per-token sets or uses this
order on both sides.
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from .w4a16 import add_bf16, grouped, swiglu


def sigmoid_f32(logits: np.ndarray) -> np.ndarray:
    x = np.asarray(logits, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (np.float32(1.0) / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


def router_logits(hidden_bits: np.ndarray, weight_f32: np.ndarray) -> np.ndarray:
    """``F.linear(x.float(), W.float())`` (klinear/router.py:50-51)."""
    x = bf16_bits_to_f32(hidden_bits).astype(np.float64)
    return (x @ np.asarray(weight_f32, dtype=np.float64).T).astype(np.float32)


def topk_desc(values: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest per row: descending value, ties -> lower index."""
    v = np.asarray(values)
    order = np.lexsort((np.broadcast_to(np.arange(v.shape[-1]), v.shape), -v.astype(np.float64)), axis=-1)
    return order[..., :k].astype(np.int64)


def route(logits: np.ndarray, bias: np.ndarray | None, top_k: int, *,
          routed_scaling_factor: float = 1.0, renormalize: bool = True,
          num_expert_group: int = 1, topk_group: int = 1
          ) -> tuple[np.ndarray, np.ndarray]:
    """Sigmoid top-k router on precomputed fp32 logits ``[T, E]``.

    Follows klinear/router.py:52-85: ``s = sigmoid(logits)``; choice =
    ``s + bias`` (out of place); grouped top-k (group score = sum of the top
    ``min(2, E/groups)`` choice scores, keep ``topk_group`` groups, others
    masked to 0.0); ``idx = topk(choice, k)``; ``w = s.gather(idx)``,
    renormalised by ``sum + 1e-20`` when ``top_k > 1``; times the scaling
    factor. Returns ``(idx int64 [T, k], w float32 [T, k])``.
    """
    lg = np.asarray(logits, dtype=np.float32)
    t_count, e_count = lg.shape
    if e_count % num_expert_group:
        raise ValueError("num_experts must be divisible by num_expert_group")
    scores = sigmoid_f32(lg)
    b = np.zeros(e_count, dtype=np.float32) if bias is None else np.asarray(bias, dtype=np.float32)
    choice = (scores + b[None, :]).astype(np.float32)
    if num_expert_group > 1:
        per = e_count // num_expert_group
        grouped_scores = choice.reshape(t_count, num_expert_group, per)
        width = min(2, per)
        top = np.sort(grouped_scores, axis=-1)[..., ::-1][..., :width]
        group_scores = top.astype(np.float32).sum(axis=-1, dtype=np.float32)
        keep = topk_desc(group_scores, topk_group)
        mask = np.zeros((t_count, num_expert_group), dtype=bool)
        np.put_along_axis(mask, keep, True, axis=1)
        full = np.repeat(mask, per, axis=1)
        choice = np.where(full, choice, np.float32(0.0)).astype(np.float32)
    idx = topk_desc(choice, top_k)
    w = np.take_along_axis(scores, idx, axis=1).astype(np.float32)
    if top_k > 1 and renormalize:
        denom = (w.astype(np.float32).sum(axis=-1, keepdims=True, dtype=np.float32)
                 + np.float32(1e-20)).astype(np.float32)
        w = (w / denom).astype(np.float32)
    return idx, (w * np.float32(routed_scaling_factor)).astype(np.float32)


def shape_stable_expert_indices(expert_indices: np.ndarray, shared_expert_id: int) -> np.ndarray:
    """Append the shared expert as a last fixed route (klinear/moe.py:23-36)."""
    idx = np.asarray(expert_indices, dtype=np.int64)
    if idx.ndim != 2:
        raise ValueError("expert_indices must have shape [tokens, routes]")
    shared = np.full((idx.shape[0], 1), shared_expert_id, dtype=np.int64)
    return np.concatenate((idx, shared), axis=1)


def combine(expert_outputs_bits: np.ndarray, combine_weights: np.ndarray) -> np.ndarray:
    """``bf16(bf16(sum_{r<R-1} eo_r * w_r) + eo_{R-1})``; last route has weight 1.

    Follows klinear/moe.py:327-334 and kernels/moe_combine.py:252-261: the
    routed sum is fp32 then cast to the activation dtype, and the shared expert
    is added as a bf16 + bf16 add. ``combine_weights[:, -1]`` is ignored.
    """
    eo = bf16_bits_to_f32(expert_outputs_bits).astype(np.float64)
    w = np.asarray(combine_weights, dtype=np.float32).astype(np.float64)
    r_count = eo.shape[1]
    routed = (eo[:, : r_count - 1] * w[:, : r_count - 1, None]).sum(axis=1)
    routed_bits = f32_to_bf16_bits(routed.astype(np.float32))
    return add_bf16(routed_bits, expert_outputs_bits[:, r_count - 1])


def w2_combine(activated_bits, expert_indices, combine_weights, w2_packed, w2_scales,
               group_size: int) -> np.ndarray:
    """W2 for every route, then :func:`combine` (kernels/moe_combine.py:209-261)."""
    act = np.asarray(activated_bits)
    t_count, r_count, i_size = act.shape
    idx = np.asarray(expert_indices, dtype=np.int64)
    eo = grouped(act.reshape(t_count * r_count, i_size), idx.reshape(-1, 1), w2_packed,
                 w2_scales, group_size).reshape(t_count, r_count, -1)
    return combine(eo, combine_weights)


def moe_block(x_bits, logits, bias, w1_packed, w1_scales, w3_packed, w3_scales,
              w2_packed, w2_scales, *, top_k: int, routed_scaling_factor: float,
              group_size: int, renormalize: bool = True, num_expert_group: int = 1,
              topk_group: int = 1):
    """The grouped W4A16 MoE block with its router.

    Follows KLinearMoE.forward's grouped branch (klinear/moe.py:375-398,
    278-334): route, append the shared expert (bank entry E, the last one),
    SwiGLU over [T, top_k+1] routes, W2 per route, weighted combine plus the
    shared expert. Returns ``(y bf16 bits [T, H], idx [T, k], w [T, k])``.
    """
    num_routed = w1_packed.shape[0] - 1
    idx, w = route(logits, bias, top_k, routed_scaling_factor=routed_scaling_factor,
                   renormalize=renormalize, num_expert_group=num_expert_group,
                   topk_group=topk_group)
    stable = shape_stable_expert_indices(idx, num_routed)
    act = swiglu(x_bits, stable, w1_packed, w1_scales, w3_packed, w3_scales, group_size)
    t_count = act.shape[0]
    eo = grouped(act.reshape(t_count * (top_k + 1), -1), stable.reshape(-1, 1), w2_packed,
                 w2_scales, group_size).reshape(t_count, top_k + 1, -1)
    full_w = np.concatenate((w, np.ones((t_count, 1), dtype=np.float32)), axis=1)
    return combine(eo, full_w), idx, w


# ---------------------------------------------------------------------------
# Expert-major schedule (kernels/moe_grouped.py:77-160)


def build_expert_schedule(expert_indices: np.ndarray):
    """Sorted union of routed experts with (token, slot) occurrences per expert.

    Follows kernels/moe_grouped.py:77-95: ``-1`` is the empty-route sentinel;
    occurrences are listed in row-major (token, slot) order. Returns a list of
    ``(expert_id, token_indices, route_slots)``.
    """
    idx = np.asarray(expert_indices)
    if idx.ndim != 2:
        raise ValueError("expert_indices must have shape [tokens, routes]")
    if (idx < -1).any():
        raise ValueError("expert indices may use only -1 as the empty-route sentinel")
    valid = idx[idx >= 0]
    out = []
    for e in np.unique(valid):
        tok, slot = np.nonzero(idx == e)
        out.append((int(e), tok.astype(np.int64), slot.astype(np.int64)))
    return out


def schedule_tables(expert_indices: np.ndarray, num_experts: int):
    """Counting-sort view of the schedule: counts, offsets and the permutation.

    ``perm`` lists flat positions ``t * R + r`` grouped by expert id (ascending)
    and row-major within an expert, i.e. exactly the occurrence order of
    :func:`build_expert_schedule` laid end to end; ``offsets[e]:offsets[e+1]``
    is expert e's segment. Sentinel routes (-1) are left out.
    """
    idx = np.asarray(expert_indices, dtype=np.int64)
    flat = idx.reshape(-1)
    counts = np.bincount(flat[flat >= 0], minlength=num_experts).astype(np.int64)
    offsets = np.concatenate(([0], np.cumsum(counts))).astype(np.int64)
    valid_pos = np.nonzero(flat >= 0)[0]
    order = np.argsort(flat[valid_pos], kind="stable")
    perm = valid_pos[order].astype(np.int64)
    return counts, offsets, perm


def expert_major_moe(hidden: np.ndarray, expert_indices: np.ndarray,
                     routing_weights: np.ndarray, expert_fn, output_size: int | None = None):
    """Apply each expert once to its rows, scatter to slots, weighted fp32 sum.

    Follows kernels/moe_grouped.py:103-160 on float32 tensors. Returns
    ``(values float32 [T, out], union_size, expert_token_counts)``.
    """
    h = np.asarray(hidden, dtype=np.float32)
    idx = np.asarray(expert_indices)
    w = np.asarray(routing_weights, dtype=np.float32)
    if idx.shape != w.shape:
        raise ValueError("expert_indices and routing_weights must have the same shape")
    out = h.shape[1] if output_size is None else output_size
    sched = build_expert_schedule(idx)
    slot_out = np.zeros((idx.shape[0], idx.shape[1], out), dtype=np.float32)
    for e, tok, slot in sched:
        slot_out[tok, slot] = expert_fn(e, h[tok])
    valid_w = np.where(idx >= 0, w, np.float32(0.0))
    values = (slot_out.astype(np.float64) * valid_w[..., None]).sum(axis=1).astype(np.float32)
    return values, len(sched), tuple((e, len(tok)) for e, tok, _ in sched)


def naive_token_major_moe(hidden, expert_indices, routing_weights, expert_fn, output_size=None):
    """Per-token, per-slot oracle (kernels/reference.py:119-165)."""
    h = np.asarray(hidden, dtype=np.float32)
    idx = np.asarray(expert_indices)
    w = np.asarray(routing_weights, dtype=np.float32)
    out = h.shape[1] if output_size is None else output_size
    slot_out = np.zeros((idx.shape[0], idx.shape[1], out), dtype=np.float32)
    for t in range(idx.shape[0]):
        for r in range(idx.shape[1]):
            e = int(idx[t, r])
            if e >= 0:
                slot_out[t, r] = expert_fn(e, h[t:t + 1])[0]
    valid_w = np.where(idx >= 0, w, np.float32(0.0))
    return (slot_out.astype(np.float64) * valid_w[..., None]).sum(axis=1).astype(np.float32)
