"""Kimi Delta Attention decode ops on HIP: the recurrence step and its fused preparation.

Same names, signatures, validation and in-place semantics as the reference's
engine/kernels/kda_step.py:273-293 (``kda_decode_step``) and
engine/kernels/kda_prepare.py:479-538 (``fused_short_conv_triple``), :630-686
(``fused_kda_gates``); each runs one launch of ``local_kimi_amd/csrc/kda.hip``.
``kda_decode_layer`` (no reference counterpart) runs all three for one decode
token in a single launch.

Beyond the reference's checks: values and states of the short convolutions
and the q / k / raw inputs of the gates must be float32, float16 or bfloat16
(TypeError otherwise), and the recurrence takes d_k up to 256. Inputs the
kernels read in another layout are copied to dense ones first; a state that
is not dense is updated through a dense copy and written back, so every state
is still mutated in place.
"""

from __future__ import annotations

import torch

from .. import _lib
from . import w4a16 as _w

CONV_WIDTH = 4
KDA_MAX_KEY_DIM = 256

_DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def _code(t: torch.Tensor, what: str) -> int:
    code = _DTYPE_CODES.get(t.dtype)
    if code is None:
        raise TypeError(f"{what} must be float32, float16 or bfloat16, got {t.dtype}")
    return code


def _dense(t: torch.Tensor) -> torch.Tensor:
    dense = t.is_contiguous() and t.data_ptr() % 16 == 0
    return t if dense else t.contiguous()


# ---------------------------------------------------------------------------
# recurrence step (engine/kernels/kda_step.py:140-170 validation)


def _validate_step(state, q, k, v, decay, beta) -> tuple[int, int, int, int]:
    if state.ndim != 4:
        raise ValueError("state must have shape [batch, heads, d_k, d_v]")
    if any(t.dtype != torch.float32 for t in (state, q, k, v, decay, beta)):
        raise TypeError("KDA decode inputs must all use torch.float32")
    if not all(t.device == state.device for t in (q, k, v, decay, beta)):
        raise ValueError("KDA decode inputs must share one device")
    batch, heads, d_k, d_v = state.shape
    if batch == 0 or heads == 0 or d_k == 0 or d_v == 0:
        raise ValueError("KDA decode dimensions must be nonzero")
    if q.shape != (batch, heads, d_k):
        raise ValueError("q must have shape [batch, heads, d_k]")
    if k.shape != (batch, heads, d_k):
        raise ValueError("k must have shape [batch, heads, d_k]")
    if v.shape != (batch, heads, d_v):
        raise ValueError("v must have shape [batch, heads, d_v]")
    if decay.shape != (batch, heads, d_k):
        raise ValueError("decay must have shape [batch, heads, d_k]")
    if beta.shape != (batch, heads):
        raise ValueError("beta must have shape [batch, heads]")
    return batch, heads, d_k, d_v


def kda_decode_step(state: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    decay: torch.Tensor, beta: torch.Tensor, *, scale: float) -> torch.Tensor:
    """One KDA decode update; mutates ``state`` in place and returns the output.

    ``state`` [B, H, d_k, d_v], ``q``/``k``/``decay`` [B, H, d_k], ``v``
    [B, H, d_v], ``beta`` [B, H], all float32:
    S <- S * exp(decay) row-wise; S <- S + beta * k (v - S^T k)^T;
    returns S^T (q * scale) as float32 [B, H, d_v].
    """
    batch, heads, d_k, d_v = _validate_step(state, q, k, v, decay, beta)
    if state.device.type != "cuda":
        raise ValueError("fused KDA decode requires CUDA inputs")
    if d_k > KDA_MAX_KEY_DIM:
        raise ValueError(f"fused KDA decode supports d_k up to {KDA_MAX_KEY_DIM}, got {d_k}")
    work = _dense(state)
    qc, kc, vc, dc, bc = (_w._c(t) for t in (q, k, v, decay, beta))
    out = torch.empty((batch, heads, d_v), dtype=torch.float32, device=state.device)
    with torch.cuda.device(state.device):
        _lib.call("lk_kda_decode_step", work.data_ptr(), qc.data_ptr(), kc.data_ptr(),
                  vc.data_ptr(), dc.data_ptr(), bc.data_ptr(), out.data_ptr(), batch, heads,
                  d_k, d_v, float(scale), _w._stream(state.device))
    if work is not state:
        state.copy_(work)
    return out


# ---------------------------------------------------------------------------
# short convolutions (engine/kernels/kda_prepare.py:372-431 validation)


def _weight_view(weight: torch.Tensor) -> torch.Tensor:
    return weight[:, 0, :] if weight.ndim == 3 else weight


def _validate_conv(q_in, k_in, v_in, q_state, k_state, v_state, q_weight, k_weight,
                   v_weight) -> tuple[int, int]:
    values = (q_in, k_in, v_in)
    states = (q_state, k_state, v_state)
    weights = (q_weight, k_weight, v_weight)
    if any(value.ndim != 3 for value in values):
        raise ValueError("q_in, k_in, and v_in must have shape [batch, 1, channels]")
    if not (q_in.shape == k_in.shape == v_in.shape):
        raise ValueError("q_in, k_in, and v_in must have identical shapes")
    batch, sequence, channels = q_in.shape
    if batch == 0 or channels == 0 or sequence != 1:
        raise ValueError("fused short convolution requires nonempty sequence length one input")
    expected_state = (batch, channels, CONV_WIDTH)
    if any(tuple(state.shape) != expected_state for state in states):
        raise ValueError("each short convolution state must have shape [batch, channels, 4]")
    valid_weight_shapes = {(channels, CONV_WIDTH), (channels, 1, CONV_WIDTH)}
    if any(tuple(weight.shape) not in valid_weight_shapes for weight in weights):
        raise ValueError("each short convolution weight must have shape [channels, 1, 4]")
    tensors = values + states + weights
    if any(not tensor.is_floating_point() for tensor in tensors):
        raise TypeError("short convolution inputs, states, and weights must be floating point")
    if any(value.dtype != state.dtype for value, state in zip(values, states)):
        raise TypeError("each short convolution input and its state must share a dtype")
    if any(tensor.device != q_in.device for tensor in tensors[1:]):
        raise ValueError("all short convolution tensors must share one device")
    if q_in.device.type != "cuda":
        raise ValueError("fused short convolution requires CUDA tensors")
    strides = (q_in.stride(0), q_in.stride(2))
    if any((value.stride(0), value.stride(2)) != strides for value in values[1:]):
        raise ValueError("q_in, k_in, and v_in must use the same layout")
    if any(state.stride() != q_state.stride() for state in states[1:]):
        raise ValueError("q_state, k_state, and v_state must use the same layout")
    wstrides = (_weight_view(q_weight).stride(0), _weight_view(q_weight).stride(1))
    if any((_weight_view(w).stride(0), _weight_view(w).stride(1)) != wstrides for w in weights[1:]):
        raise ValueError("q_weight, k_weight, and v_weight must use the same layout")
    return batch, channels


def fused_short_conv_triple(q_in: torch.Tensor, k_in: torch.Tensor, v_in: torch.Tensor,
                            q_state: torch.Tensor, k_state: torch.Tensor, v_state: torch.Tensor,
                            q_weight: torch.Tensor, k_weight: torch.Tensor,
                            v_weight: torch.Tensor
                            ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The three width-4 decode convolutions in one launch; mutates the states.

    Per channel: window = (state[1], state[2], state[3], token); output =
    silu(sum window * weight) in float32, in the input dtype; the window
    becomes the state.
    """
    batch, channels = _validate_conv(q_in, k_in, v_in, q_state, k_state, v_state, q_weight,
                                     k_weight, v_weight)
    vcode = _code(q_in, "short convolution inputs and states")
    weights = [_weight_view(w) for w in (q_weight, k_weight, v_weight)]
    if weights[0].dtype not in _DTYPE_CODES or any(w.dtype != weights[0].dtype for w in weights):
        weights = [w.float() for w in weights]
    wcode = _DTYPE_CODES[weights[0].dtype]
    weights = [_w._c(w) for w in weights]
    ins = [_w._c(t) for t in (q_in, k_in, v_in)]
    states = [q_state, k_state, v_state]
    work = [s if s.is_contiguous() else s.contiguous() for s in states]
    outs = [torch.empty((batch, 1, channels), dtype=q_in.dtype, device=q_in.device)
            for _ in range(3)]
    with torch.cuda.device(q_in.device):
        _lib.call("lk_kda_short_conv_triple", *(t.data_ptr() for t in ins),
                  *(t.data_ptr() for t in work), *(t.data_ptr() for t in weights),
                  *(t.data_ptr() for t in outs), batch, channels, vcode, wcode,
                  _w._stream(q_in.device))
    for s, w in zip(states, work):
        if w is not s:
            s.copy_(w)
    return outs[0], outs[1], outs[2]


# ---------------------------------------------------------------------------
# gates (engine/kernels/kda_prepare.py:541-587 validation)


def _validate_gates(raw_decay, dt_bias, a_log, raw_beta, q, k, *, num_heads, head_dim,
                    eps) -> tuple[int, int]:
    if num_heads <= 0 or head_dim <= 0 or head_dim > 1024:
        raise ValueError("num_heads and head_dim must be positive, with head_dim at most 1024")
    if eps <= 0:
        raise ValueError("eps must be positive")
    if raw_decay.ndim != 4:
        raise ValueError("raw_decay must have shape [batch, sequence, heads, head_dim]")
    batch, sequence, decay_heads, decay_dim = raw_decay.shape
    if batch == 0 or sequence == 0:
        raise ValueError("KDA gate inputs must have nonempty batch and sequence dimensions")
    if (decay_heads, decay_dim) != (num_heads, head_dim):
        raise ValueError("raw_decay shape does not match num_heads and head_dim")
    if tuple(raw_beta.shape) != (batch, sequence, num_heads):
        raise ValueError("raw_beta must have shape [batch, sequence, num_heads]")
    if tuple(dt_bias.shape) != (num_heads * head_dim,):
        raise ValueError("dt_bias must be flat with num_heads * head_dim entries")
    if tuple(a_log.shape) != (1, 1, num_heads, 1):
        raise ValueError("a_log must have shape [1, 1, num_heads, 1]")
    flat = (batch, sequence, num_heads * head_dim)
    headed = (batch, sequence, num_heads, head_dim)
    if tuple(q.shape) not in (flat, headed):
        raise ValueError("q must be flat by projection or viewed as heads")
    if tuple(k.shape) != tuple(q.shape):
        raise ValueError("q and k must have identical shapes")
    tensors = (raw_decay, dt_bias, a_log, raw_beta, q, k)
    if any(not t.is_floating_point() for t in tensors):
        raise TypeError("KDA gate inputs must be floating point")
    if any(t.device != raw_decay.device for t in tensors[1:]):
        raise ValueError("all KDA gate tensors must share one device")
    if any(not t.is_contiguous() for t in tensors):
        raise ValueError("KDA gate tensors must be contiguous without transposition")
    if raw_decay.device.type != "cuda":
        raise ValueError("fused KDA gates require CUDA tensors")
    return batch, sequence


def fused_kda_gates(raw_decay: torch.Tensor, dt_bias: torch.Tensor, a_log: torch.Tensor,
                    raw_beta: torch.Tensor, q: torch.Tensor, k: torch.Tensor, *,
                    num_heads: int, head_dim: int, eps: float
                    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Decay, beta and per-head q / k normalisation in one launch.

    Returns float32 ``decay`` [B, S, H, D] = -exp(a_log) * softplus(raw_decay +
    dt_bias), ``beta`` [B, S, H] = sigmoid(raw_beta), and q and k [B, S, H, D]
    scaled by rsqrt(sum of squares over the head + eps).
    """
    batch, sequence = _validate_gates(raw_decay, dt_bias, a_log, raw_beta, q, k,
                                      num_heads=num_heads, head_dim=head_dim, eps=eps)
    dcode = _code(raw_decay, "raw_decay")
    bcode = _code(raw_beta, "raw_beta")
    if q.dtype != k.dtype:
        k = k.to(q.dtype)
    qcode = _code(q, "q and k")
    bias = dt_bias.float().contiguous()
    rate = a_log.float().reshape(num_heads).contiguous()
    dev = raw_decay.device
    decay = torch.empty(tuple(raw_decay.shape), dtype=torch.float32, device=dev)
    beta = torch.empty(tuple(raw_beta.shape), dtype=torch.float32, device=dev)
    q_out = torch.empty((batch, sequence, num_heads, head_dim), dtype=torch.float32, device=dev)
    k_out = torch.empty_like(q_out)
    with torch.cuda.device(dev):
        _lib.call("lk_kda_gates", raw_decay.data_ptr(), bias.data_ptr(), rate.data_ptr(),
                  raw_beta.data_ptr(), q.data_ptr(), k.data_ptr(), decay.data_ptr(),
                  beta.data_ptr(), q_out.data_ptr(), k_out.data_ptr(), batch * sequence,
                  num_heads, head_dim, float(eps), dcode, bcode, qcode, _w._stream(dev))
    return decay, beta, q_out, k_out


# ---------------------------------------------------------------------------
# the whole layer in one launch (no reference counterpart)

KDA_LAYER_MAX_DIM = 128


def kda_decode_layer(q_in: torch.Tensor, k_in: torch.Tensor, v_in: torch.Tensor,
                     q_state: torch.Tensor, k_state: torch.Tensor, v_state: torch.Tensor,
                     q_weight: torch.Tensor, k_weight: torch.Tensor, v_weight: torch.Tensor,
                     raw_decay: torch.Tensor, dt_bias: torch.Tensor, a_log: torch.Tensor,
                     raw_beta: torch.Tensor, state: torch.Tensor, *, num_heads: int,
                     head_dim: int, eps: float = 1e-6, scale: float | None = None,
                     conv_states_out: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None
                     ) -> torch.Tensor:
    """One KDA decode token: the short convolutions, the gates and the
    recurrence step in one launch (what engine/klinear/attention.py:193-271
    does with fused_short_conv_triple, fused_kda_gates and kda_decode_step).

    Arguments as those three functions take them, with ``state`` the fp32
    recurrent state [B, H, D, D]; ``scale`` defaults to D ** -0.5. ``state``
    is updated in place; returns the fp32 output [B, H, D] (``fused_output``
    of attention.py:268). head_dim: a multiple of 4 up to 128.

    Without ``conv_states_out`` the conv states are updated in place and one
    block works on each head. With ``conv_states_out`` (three dense tensors
    shaped like the states, none of them a state) the shifted conv states are
    written there instead and each head's value columns are split over blocks
    of 16 (a head's blocks all read the old conv states); callers alternate
    the two state sets from token to token.
    """
    batch, channels = _validate_conv(q_in, k_in, v_in, q_state, k_state, v_state, q_weight,
                                     k_weight, v_weight)
    ins = [_w._c(t) for t in (q_in, k_in, v_in)]  # strided projections (one fused buffer) are copied
    _validate_gates(raw_decay, dt_bias, a_log, raw_beta, ins[0], ins[1], num_heads=num_heads,
                    head_dim=head_dim, eps=eps)
    if raw_decay.shape[:2] != (batch, 1):
        raise ValueError("raw_decay must hold one token per batch row")
    if state.dtype != torch.float32:
        raise TypeError("KDA decode inputs must all use torch.float32")
    if tuple(state.shape) != (batch, num_heads, head_dim, head_dim):
        raise ValueError("state must have shape [batch, heads, head_dim, head_dim]")
    if state.device != q_in.device:
        raise ValueError("all KDA tensors must share one device")
    if head_dim > KDA_LAYER_MAX_DIM or head_dim % 4:
        raise ValueError(f"kda_decode_layer takes head_dim a multiple of 4 up to "
                         f"{KDA_LAYER_MAX_DIM}, got {head_dim}")
    vcode = _code(q_in, "short convolution inputs and states")
    weights = [_weight_view(w) for w in (q_weight, k_weight, v_weight)]
    if weights[0].dtype not in _DTYPE_CODES or any(w.dtype != weights[0].dtype for w in weights):
        weights = [w.float() for w in weights]
    wcode = _DTYPE_CODES[weights[0].dtype]
    weights = [_w._c(w) for w in weights]
    if conv_states_out is not None:
        return _layer_split(ins, [q_state, k_state, v_state], conv_states_out, weights, raw_decay,
                            dt_bias, a_log, raw_beta, state, batch, num_heads, head_dim, eps,
                            scale, vcode, wcode)
    conv_states = [q_state, k_state, v_state]
    conv_work = [s if s.is_contiguous() else s.contiguous() for s in conv_states]
    work = _dense(state)
    bias = dt_bias.float().contiguous()
    rate = a_log.float().reshape(num_heads).contiguous()
    out = torch.empty((batch, num_heads, head_dim), dtype=torch.float32, device=state.device)
    s = head_dim ** -0.5 if scale is None else float(scale)
    with torch.cuda.device(state.device):
        _lib.call("lk_kda_decode_layer", *(t.data_ptr() for t in ins),
                  *(t.data_ptr() for t in conv_work), *(t.data_ptr() for t in weights),
                  raw_decay.data_ptr(), bias.data_ptr(), rate.data_ptr(), raw_beta.data_ptr(),
                  work.data_ptr(), out.data_ptr(), batch, num_heads, head_dim, float(eps), s,
                  vcode, wcode, _code(raw_decay, "raw_decay"), _code(raw_beta, "raw_beta"),
                  _w._stream(state.device))
    for st, w in zip(conv_states, conv_work):
        if w is not st:
            st.copy_(w)
    if work is not state:
        state.copy_(work)
    return out


def _layer_split(ins, states, outs, weights, raw_decay, dt_bias, a_log, raw_beta, state, batch,
                 num_heads, head_dim, eps, scale, vcode, wcode):
    outs = tuple(outs)
    if len(outs) != 3:
        raise ValueError("conv_states_out must hold the q, k and v states")
    for st, o in zip(states, outs):
        if o.shape != st.shape or o.dtype != st.dtype or o.device != st.device:
            raise ValueError("each conv_states_out tensor must match its state's shape, dtype "
                             "and device")
        if not o.is_contiguous():
            raise ValueError("conv_states_out tensors must be contiguous")
    spans = [(t.data_ptr(), t.data_ptr() + t.numel() * t.element_size()) for t in (*states, *outs)]
    for i, (lo, hi) in enumerate(spans[3:]):
        if any(lo < h2 and l2 < hi for l2, h2 in spans[:3]):
            raise ValueError(f"conv_states_out[{i}] overlaps a state it is computed from")
    src = [s if s.is_contiguous() else s.contiguous() for s in states]
    work = _dense(state)
    bias = dt_bias.float().contiguous()
    rate = a_log.float().reshape(num_heads).contiguous()
    out = torch.empty((batch, num_heads, head_dim), dtype=torch.float32, device=state.device)
    s = head_dim ** -0.5 if scale is None else float(scale)
    with torch.cuda.device(state.device):
        _lib.call("lk_kda_decode_layer_split", *(t.data_ptr() for t in ins),
                  *(t.data_ptr() for t in src), *(t.data_ptr() for t in outs),
                  *(t.data_ptr() for t in weights), raw_decay.data_ptr(), bias.data_ptr(),
                  rate.data_ptr(), raw_beta.data_ptr(), work.data_ptr(), out.data_ptr(), batch,
                  num_heads, head_dim, float(eps), s, vcode, wcode, _code(raw_decay, "raw_decay"),
                  _code(raw_beta, "raw_beta"), _w._stream(state.device))
    if work is not state:
        state.copy_(work)
    return out
