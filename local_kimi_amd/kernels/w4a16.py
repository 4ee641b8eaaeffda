"""Host wrappers of the W4A16 ops: validate like the reference, then call HIP.

Each public function keeps the positional signature of the reference op it
replaces (engine/kernels/__init__.py:82-86 and the modules cited per
function), raises the same exception types for the same mistakes, allocates
its outputs with the torch caching allocator on the input's device and
launches on the current stream, so it is safe under HIP graph capture.

The group size is not an argument in the reference (it is fixed at 32,
engine/quant/w4a16.py:14). Here it is read from the scale tensor's last axis:
``G = K // scales.shape[-1]``; it must be a power-of-two multiple of 32.
"""

from __future__ import annotations

import torch

from .. import _lib


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _group_size(reduction: int, scale_columns: int, what: str) -> int:
    if scale_columns <= 0 or reduction % scale_columns:
        raise ValueError(f"{what} scales have the wrong shape")
    group = reduction // scale_columns
    if group % 32 or group & (group - 1):
        raise ValueError(f"{what} group size {group} must be a power-of-two multiple of 32")
    return group


def _c(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


# Row counts from which the expert-major / MFMA GEMM paths replace the
# per-route GEMV kernels (token-routes for the grouped ops, rows for dense).
GROUPED_GEMM_MIN_ROUTES = 32
DENSE_GEMM_MIN_ROWS = 16


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Scratch device memory from the torch caching allocator."""
    return torch.empty((max(int(nbytes), 1),), dtype=torch.uint8, device=device)


def check_bank(packed: torch.Tensor, scales: torch.Tensor, what: str) -> tuple[int, int, int, int]:
    """Validate one grouped bank without touching its data: ``(E, N, K, G)``."""
    if packed.ndim != 3 or scales.ndim != 3:
        raise ValueError(f"{what} packed weights and scales must be rank three")
    if packed.dtype != torch.uint8:
        raise TypeError(f"{what} packed weights must use torch.uint8 storage")
    if scales.dtype != torch.bfloat16:
        raise TypeError(f"{what} scales must use torch.bfloat16 storage")
    if packed.device != scales.device:
        raise ValueError(f"{what} packed weights and scales must share a device")
    experts, output_size, packed_reduction = packed.shape
    reduction = packed_reduction * 2
    if experts == 0 or output_size == 0 or reduction == 0:
        raise ValueError(f"{what} bank requires nonzero dimensions")
    if scales.shape[:2] != (experts, output_size):
        raise ValueError(f"{what} scales have the wrong shape")
    group = _group_size(reduction, scales.shape[2], what)
    return experts, output_size, reduction, group


# ---------------------------------------------------------------------------
# op w4a16_dense (engine/kernels/w4a16_dense_gemv.py:167-198, 312-336)


def _validate_dense(activations, packed_weights, scales) -> tuple[int, int, int, int]:
    if activations.ndim != 2 or activations.dtype != torch.bfloat16:
        raise TypeError("activations must be a BF16 [tokens, reduction] matrix")
    if packed_weights.ndim != 2 or packed_weights.dtype != torch.uint8:
        raise TypeError("packed weights must be a uint8 [output, reduction / 2] matrix")
    if scales.ndim != 2 or scales.dtype != torch.bfloat16:
        raise TypeError("scales must be a BF16 [output, reduction / group] matrix")
    if activations.device.type != "cuda":
        raise ValueError("W4A16 dense GEMV requires CUDA")
    if not (activations.device == packed_weights.device == scales.device):
        raise ValueError("activations, packed weights, and scales must share a device")
    m, reduction = activations.shape
    output_size, packed_reduction = packed_weights.shape
    if output_size == 0 or reduction == 0:
        raise ValueError("W4A16 dense GEMV requires nonzero dimensions")
    if packed_reduction * 2 != reduction:
        raise ValueError("packed weights have the wrong reduction width")
    if scales.shape[0] != output_size:
        raise ValueError("W4A16 scales have the wrong shape")
    group = _group_size(reduction, scales.shape[1], "W4A16")
    return m, output_size, reduction, group


def _dense(entry: str, activations, packed_weights, scales):
    m, n, k, g = _validate_dense(activations, packed_weights, scales)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=activations.device)
    if m == 0:
        return out
    x, p, s = _c(activations), _c(packed_weights), _c(scales)
    with torch.cuda.device(activations.device):
        _lib.call(entry, x.data_ptr(), p.data_ptr(), s.data_ptr(), out.data_ptr(), m, n, k, g,
                  _stream(activations.device))
    return out


def _dense_gemm(activations, packed_weights, scales):
    """The MFMA GEMM with its direct-load workspace (the paired rows and their
    group sums, G = 128) from the torch caching allocator."""
    m, n, k, g = _validate_dense(activations, packed_weights, scales)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=activations.device)
    if m == 0:
        return out
    ws = workspace(_lib.query("lk_w4a16_dense_gemm_workspace", m, k, g), activations.device)
    x, p, s = _c(activations), _c(packed_weights), _c(scales)
    with torch.cuda.device(activations.device):
        _lib.call("lk_w4a16_dense_gemm_ws", x.data_ptr(), p.data_ptr(), s.data_ptr(),
                  out.data_ptr(), m, n, k, g, ws.data_ptr(), ws.numel(),
                  _stream(activations.device))
    return out


def w4a16_dense(activations: torch.Tensor, packed_weights: torch.Tensor,
                scales: torch.Tensor) -> torch.Tensor:
    """``y[M, N] = x @ dequant(W).T`` (registered as ``hip``).

    Decode rows use the K-split GEMV; from ``DENSE_GEMM_MIN_ROWS`` rows the
    MFMA GEMM (weights read once per 64-row tile).
    """
    if activations.ndim == 2 and activations.shape[0] >= DENSE_GEMM_MIN_ROWS:
        return _dense_gemm(activations, packed_weights, scales)
    return _dense("lk_w4a16_dense", activations, packed_weights, scales)


def w4a16_dense_gemm(activations: torch.Tensor, packed_weights: torch.Tensor,
                     scales: torch.Tensor) -> torch.Tensor:
    """The MFMA GEMM form of :func:`w4a16_dense` at any row count."""
    return _dense_gemm(activations, packed_weights, scales)


def w4a16_dense_reference(activations: torch.Tensor, packed_weights: torch.Tensor,
                          scales: torch.Tensor) -> torch.Tensor:
    """Reference-rounding dense op (bf16(q*s) weights, one thread per output)."""
    return _dense("lk_w4a16_dense_reference", activations, packed_weights, scales)


# ---------------------------------------------------------------------------
# op w4a16_grouped (engine/kernels/w4a16_gemv.py:449-488, 610-635)


def _validate_grouped(activations, expert_indices, packed_weights, scales):
    if activations.ndim != 2 or activations.dtype != torch.bfloat16:
        raise TypeError("activations must be a BF16 [tokens, reduction] matrix")
    if expert_indices.ndim != 2 or expert_indices.dtype != torch.long:
        raise TypeError("expert_indices must be an int64 [tokens, routes] matrix")
    if packed_weights.ndim != 3 or scales.ndim != 3:
        raise ValueError("grouped packed weights and scales must be rank three")
    if packed_weights.dtype != torch.uint8:
        raise TypeError("packed grouped weights must use torch.uint8 storage")
    if scales.dtype != torch.bfloat16:
        raise TypeError("grouped W4A16 scales must use torch.bfloat16 storage")
    if activations.device.type != "cuda":
        raise ValueError("grouped W4A16 decode requires CUDA")
    if not (activations.device == expert_indices.device == packed_weights.device == scales.device):
        raise ValueError("grouped W4A16 inputs must share one device")
    tokens, reduction = activations.shape
    route_tokens, routes = expert_indices.shape
    experts, output_size, packed_reduction = packed_weights.shape
    if route_tokens != tokens:
        raise ValueError("expert routing must have one row per token")
    if routes == 0 or experts == 0 or output_size == 0 or reduction == 0:
        raise ValueError("grouped W4A16 decode requires nonzero dimensions")
    if packed_reduction * 2 != reduction:
        raise ValueError("packed grouped weights have the wrong reduction width")
    if scales.shape[:2] != (experts, output_size):
        raise ValueError("grouped W4A16 scales have the wrong shape")
    group = _group_size(reduction, scales.shape[2], "grouped W4A16")
    return tokens, routes, experts, output_size, reduction, group


def _grouped(entry: str, activations, expert_indices, packed_weights, scales):
    t, r, e, n, k, g = _validate_grouped(activations, expert_indices, packed_weights, scales)
    out = torch.empty((t, r, n), dtype=torch.bfloat16, device=activations.device)
    if t == 0:
        return out
    x, idx, p, s = _c(activations), _c(expert_indices), _c(packed_weights), _c(scales)
    with torch.cuda.device(activations.device):
        if entry.endswith("_gemm"):
            ws = workspace(_lib.query("lk_w4a16_grouped_gemm_workspace", t, r, e), x.device)
            _lib.call(entry, x.data_ptr(), idx.data_ptr(), p.data_ptr(), s.data_ptr(),
                      out.data_ptr(), t, r, e, n, k, g, ws.data_ptr(), ws.numel(),
                      _stream(activations.device))
        else:
            _lib.call(entry, x.data_ptr(), idx.data_ptr(), p.data_ptr(), s.data_ptr(),
                      out.data_ptr(), t, r, e, n, k, g, _stream(activations.device))
    return out


def _use_grouped_gemm(activations, expert_indices) -> bool:
    return (expert_indices.ndim == 2 and activations.ndim == 2
            and expert_indices.shape[0] * expert_indices.shape[1] >= GROUPED_GEMM_MIN_ROUTES)


def grouped_w4a16_gemv(activations: torch.Tensor, expert_indices: torch.Tensor,
                       packed_weights: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """``out[t, r] = x[t] @ dequant(W[idx[t, r]]).T`` -> ``[T, R, N]`` bf16.

    Expert indices outside ``[0, E)`` are treated as empty routes (zeros) so a
    bad index cannot read past the bank. From ``GROUPED_GEMM_MIN_ROUTES``
    token-routes the routes are sorted by expert and run as an MFMA GEMM.
    """
    entry = "lk_w4a16_grouped_gemm" if _use_grouped_gemm(activations, expert_indices) \
        else "lk_w4a16_grouped"
    return _grouped(entry, activations, expert_indices, packed_weights, scales)


def grouped_w4a16_gemm(activations, expert_indices, packed_weights, scales):
    """The expert-major MFMA form of :func:`grouped_w4a16_gemv` at any size."""
    return _grouped("lk_w4a16_grouped_gemm", activations, expert_indices, packed_weights, scales)


def grouped_w4a16_reference(activations, expert_indices, packed_weights, scales):
    """Reference-rounding grouped op (engine/kernels/w4a16_grouped.py:121-194)."""
    return _grouped("lk_w4a16_grouped_reference", activations, expert_indices, packed_weights, scales)


# ---------------------------------------------------------------------------
# op w4a16_swiglu (engine/kernels/w4a16_gemv.py:638-658, 772-790)


def _validate_swiglu(activations, expert_indices, w1_packed, w1_scales, w3_packed, w3_scales):
    dims = _validate_grouped(activations, expert_indices, w1_packed, w1_scales)
    w3_dims = _validate_grouped(activations, expert_indices, w3_packed, w3_scales)
    if w3_dims != dims:
        raise ValueError("grouped W1 and W3 dimensions must match")
    if w3_packed.shape != w1_packed.shape:
        raise ValueError("grouped W1 and W3 packed shapes must match")
    if w3_scales.shape != w1_scales.shape:
        raise ValueError("grouped W1 and W3 scale shapes must match")
    return dims


def _swiglu(gemm: bool, activations, expert_indices, w1_packed, w1_scales, w3_packed,
            w3_scales) -> torch.Tensor:
    t, r, e, n, k, g = _validate_swiglu(activations, expert_indices, w1_packed, w1_scales,
                                        w3_packed, w3_scales)
    out = torch.empty((t, r, n), dtype=torch.bfloat16, device=activations.device)
    if t == 0:
        return out
    x, idx = _c(activations), _c(expert_indices)
    p1, s1, p3, s3 = _c(w1_packed), _c(w1_scales), _c(w3_packed), _c(w3_scales)
    args = [x.data_ptr(), idx.data_ptr(), p1.data_ptr(), s1.data_ptr(), p3.data_ptr(),
            s3.data_ptr(), out.data_ptr(), t, r, e, n, k, g]
    with torch.cuda.device(activations.device):
        if gemm:
            ws = workspace(_lib.query("lk_w4a16_grouped_gemm_workspace", t, r, e), x.device)
            _lib.call("lk_w4a16_swiglu_gemm", *args, ws.data_ptr(), ws.numel(),
                      _stream(activations.device))
        else:
            _lib.call("lk_w4a16_swiglu", *args, _stream(activations.device))
    return out


def grouped_w4a16_swiglu_gemv(activations, expert_indices, w1_packed, w1_scales, w3_packed,
                              w3_scales) -> torch.Tensor:
    """One launch: ``bf16(bf16(silu(bf16(x W1^T))) * bf16(x W3^T))`` per route.

    From ``GROUPED_GEMM_MIN_ROUTES`` token-routes: the expert-major MFMA GEMM.
    """
    return _swiglu(_use_grouped_gemm(activations, expert_indices), activations, expert_indices,
                   w1_packed, w1_scales, w3_packed, w3_scales)


def grouped_w4a16_swiglu_gemm(activations, expert_indices, w1_packed, w1_scales, w3_packed,
                              w3_scales) -> torch.Tensor:
    """The expert-major MFMA form of :func:`grouped_w4a16_swiglu_gemv`."""
    return _swiglu(True, activations, expert_indices, w1_packed, w1_scales, w3_packed, w3_scales)


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``F.silu(gate) * up`` on bf16 tensors (rounded like torch's two ops)."""
    if gate.dtype != torch.bfloat16 or up.dtype != torch.bfloat16:
        raise TypeError("gate and up must be BF16 tensors")
    if gate.shape != up.shape:
        raise ValueError("gate and up tensors must have the same shape")
    if gate.device.type != "cuda" or gate.device != up.device:
        raise ValueError("silu_mul requires CUDA tensors on one device")
    out = torch.empty_like(gate, memory_format=torch.contiguous_format)
    g, u = _c(gate), _c(up)
    with torch.cuda.device(gate.device):
        _lib.call("lk_silu_mul", g.data_ptr(), u.data_ptr(), out.data_ptr(), gate.numel(),
                  _stream(gate.device))
    return out


# ---------------------------------------------------------------------------
# fused W2 + combine (engine/kernels/moe_combine.py:156-206, 264-324)


def _validate_w2_combine(activated, expert_indices, combine_weights, w2_packed, w2_scales):
    if activated.ndim != 3 or activated.dtype != torch.bfloat16:
        raise TypeError("activated must be a BF16 [tokens, routes, reduction] tensor")
    if expert_indices.ndim != 2 or expert_indices.dtype != torch.long:
        raise TypeError("expert_indices must be an int64 [tokens, routes] matrix")
    if combine_weights.ndim != 2 or combine_weights.dtype != torch.float32:
        raise TypeError("combine_weights must be a float32 [tokens, routes] matrix")
    if w2_packed.ndim != 3 or w2_scales.ndim != 3:
        raise ValueError("grouped W2 packed weights and scales must be rank three")
    if w2_packed.dtype != torch.uint8:
        raise TypeError("grouped W2 packed weights must use torch.uint8 storage")
    if w2_scales.dtype != torch.bfloat16:
        raise TypeError("grouped W2 scales must use torch.bfloat16 storage")
    if activated.device.type != "cuda":
        raise ValueError("fused W2 combine requires CUDA")
    if not (activated.device == expert_indices.device == combine_weights.device
            == w2_packed.device == w2_scales.device):
        raise ValueError("fused W2 combine inputs must share one device")
    tokens, routes, reduction = activated.shape
    experts, output_size, packed_reduction = w2_packed.shape
    if expert_indices.shape != (tokens, routes):
        raise ValueError("expert_indices must match the activated token-route shape")
    if combine_weights.shape != (tokens, routes):
        raise ValueError("combine_weights must match the activated token-route shape")
    if routes == 0 or experts == 0 or output_size == 0 or reduction == 0:
        raise ValueError("fused W2 combine requires nonzero route and weight dimensions")
    if packed_reduction * 2 != reduction:
        raise ValueError("grouped W2 packed weights have the wrong reduction width")
    if w2_scales.shape[:2] != (experts, output_size):
        raise ValueError("grouped W2 scales have the wrong shape")
    group = _group_size(reduction, w2_scales.shape[2], "grouped W2")
    return tokens, routes, experts, output_size, reduction, group


def fused_w2_combine(activated, expert_indices, combine_weights, w2_packed, w2_scales):
    """W2 for every route and the weighted route sum plus shared expert, one launch.

    The last route is the shared expert, added with weight exactly 1; its entry
    in ``combine_weights`` is ignored (engine/kernels/moe_combine.py:216-221).
    """
    t, r, e, h, i, g = _validate_w2_combine(activated, expert_indices, combine_weights,
                                            w2_packed, w2_scales)
    out = torch.empty((t, h), dtype=torch.bfloat16, device=activated.device)
    if t == 0:
        return out
    a, idx, cw = _c(activated), _c(expert_indices), _c(combine_weights)
    p, s = _c(w2_packed), _c(w2_scales)
    with torch.cuda.device(activated.device):
        _lib.call("lk_w4a16_w2_combine", a.data_ptr(), idx.data_ptr(), cw.data_ptr(), p.data_ptr(),
                  s.data_ptr(), out.data_ptr(), t, r, e, h, i, g, _stream(activated.device))
    return out


def route_combine(expert_outputs: torch.Tensor, combine_weights: torch.Tensor) -> torch.Tensor:
    """``bf16(bf16(sum_{r<R-1} eo*w) + eo[:, -1])`` on precomputed route outputs."""
    if expert_outputs.ndim != 3 or expert_outputs.dtype != torch.bfloat16:
        raise TypeError("expert_outputs must be a BF16 [tokens, routes, hidden] tensor")
    if combine_weights.dtype != torch.float32 or combine_weights.shape != expert_outputs.shape[:2]:
        raise TypeError("combine_weights must be a float32 [tokens, routes] matrix")
    if expert_outputs.device.type != "cuda" or combine_weights.device != expert_outputs.device:
        raise ValueError("route_combine requires CUDA tensors on one device")
    t, r, h = expert_outputs.shape
    out = torch.empty((t, h), dtype=torch.bfloat16, device=expert_outputs.device)
    eo, cw = _c(expert_outputs), _c(combine_weights)
    with torch.cuda.device(expert_outputs.device):
        _lib.call("lk_route_combine", eo.data_ptr(), cw.data_ptr(), out.data_ptr(), t, r, h,
                  _stream(expert_outputs.device))
    return out


def fused_w2_combine_reference(activated, expert_indices, combine_weights, w2_packed, w2_scales):
    """Reference sequence: grouped W2 per route (reference rounding), then combine."""
    t, r, e, h, i, g = _validate_w2_combine(activated, expert_indices, combine_weights,
                                            w2_packed, w2_scales)
    eo = grouped_w4a16_reference(activated.reshape(t * r, i), expert_indices.reshape(t * r, 1),
                                 w2_packed, w2_scales).reshape(t, r, h)
    return route_combine(eo, combine_weights)


# ---------------------------------------------------------------------------
# fused QKV (engine/kernels/w4a16_fused_qkv.py:178-389)


def _validate_qkv(activations, q_packed, q_scales, k_packed, k_scales, v_packed, v_scales):
    if activations.ndim != 2 or activations.dtype != torch.bfloat16:
        raise TypeError("activations must be a BF16 [tokens, reduction] matrix")
    if activations.device.type != "cuda":
        raise ValueError("fused W4A16 QKV requires CUDA")
    if q_packed.ndim != 2:
        raise TypeError("q packed weights must be a uint8 [output, reduction / 2] matrix")
    output_size = q_packed.shape[0]
    reduction = activations.shape[1]
    if output_size == 0 or reduction == 0:
        raise ValueError("fused W4A16 QKV requires nonzero dimensions")
    for name, p, s in (("q", q_packed, q_scales), ("k", k_packed, k_scales), ("v", v_packed, v_scales)):
        if p.ndim != 2 or p.dtype != torch.uint8:
            raise TypeError(f"{name} packed weights must be a uint8 [output, reduction / 2] matrix")
        if s.ndim != 2 or s.dtype != torch.bfloat16:
            raise TypeError(f"{name} scales must be a BF16 [output, reduction / group] matrix")
        if p.device != activations.device or s.device != activations.device:
            raise ValueError("all fused QKV inputs must share a device")
        if p.shape != (output_size, reduction // 2):
            raise ValueError(f"{name} packed weights have the wrong shape")
        if s.shape[0] != output_size:
            raise ValueError(f"{name} scales have the wrong shape")
        _group_size(reduction, s.shape[1], name)


def fused_qkv_w4a16(activations, q_packed, q_scales, k_packed, k_scales, v_packed, v_scales):
    """Q, K and V projections of one activation matrix -> ``(q, k, v)``.

    One launch either way: from 16 rows the MFMA GEMM over all three
    matrices, for decode rows the K-split GEMV over the three matrices' row
    blocks (the reference's one-launch K7, w4a16_fused_qkv.py:342-389).
    """
    _validate_qkv(activations, q_packed, q_scales, k_packed, k_scales, v_packed, v_scales)
    m, k = activations.shape
    n = q_packed.shape[0]
    g = _group_size(k, q_scales.shape[1], "q")
    if _group_size(k, k_scales.shape[1], "k") != g or _group_size(k, v_scales.shape[1], "v") != g:
        raise ValueError("fused QKV projections must share one group size")
    dev = activations.device
    outs = [torch.empty((m, n), dtype=torch.bfloat16, device=dev) for _ in range(3)]
    if m == 0:
        return tuple(outs)
    x = _c(activations)
    w = [_c(t) for t in (q_packed, q_scales, k_packed, k_scales, v_packed, v_scales)]
    ws = workspace(_lib.query("lk_w4a16_dense_gemm_workspace", m, k, g), dev)
    with torch.cuda.device(dev):
        _lib.call("lk_w4a16_fused_qkv_ws", x.data_ptr(), *(t.data_ptr() for t in w),
                  *(o.data_ptr() for o in outs), m, n, k, g, ws.data_ptr(), ws.numel(),
                  _stream(dev))
    return tuple(outs)


def fused_qkv_w4a16_reference(activations, q_packed, q_scales, k_packed, k_scales, v_packed,
                              v_scales):
    """Three reference dense calls (engine/kernels/w4a16_fused_qkv.py:257-271)."""
    _validate_qkv(activations, q_packed, q_scales, k_packed, k_scales, v_packed, v_scales)
    return (w4a16_dense_reference(activations, q_packed, q_scales),
            w4a16_dense_reference(activations, k_packed, k_scales),
            w4a16_dense_reference(activations, v_packed, v_scales))
