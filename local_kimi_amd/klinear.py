"""Model-slice callers of the HIP ops, with the call shapes of the reference's.

* :class:`W4A16Linear` -- ``W4A16Linear.forward`` (engine/klinear/quantized.py:
  160-180): flatten the leading dimensions, call the ``w4a16_dense`` op
  resolved once per module, restore the shape.
* :class:`KLinearMoE` -- the grouped W4A16 route of ``KLinearMoE``
  (engine/klinear/moe.py:278-334) with the router of
  engine/klinear/router.py:47-85: ``logits = fp32(x) fp32(Wg)^T`` (one HIP
  launch for every batch size; the router weight in bf16, fp16 or fp32), then the ``w4a16_moe_block`` op (selection, SwiGLU experts, W2, combine,
  shared expert with weight 1) over banks with the shared expert last.
* :class:`MoEDecodeGraph` -- one MoE layer's decode step captured once in a
  HIP graph and replayed on a static input buffer, the counterpart of
  ``CUDAGraphDecodeRunner`` (engine/generate.py:226-306).
* :class:`RMSNorm`, :class:`RMSGatedNorm` -- engine/klinear/norm.py:16-52 on
  the HIP norm kernels (same constructor arguments and forward).
* :class:`MoELayerTail` -- the post-attention half of ``KLinearDecoderLayer.
  forward`` (engine/klinear/layer.py:155-170): residual add and
  post_attention_layernorm in one launch, the MoE, and the second residual
  add fused with the next layer's input_layernorm when one is given.
"""

from __future__ import annotations

import torch
from torch import nn

from .checkpoint import MoeBanks, W4A16Index, build_moe_banks
from .kernels import W4A16_DENSE, W4A16_MOE_BLOCK, registry, router_logits
from .kernels.norm import add_rms_norm, rms_gated_norm, rms_norm
from .quant.w4a16 import W4A16Tensor

HIDDEN = 2304         # Kimi-Linear hidden size (engine/klinear/config.py:42)
INTERMEDIATE = 1024   # moe_intermediate_size (config.py:62)
ROUTED_EXPERTS = 256  # config.py:59-61
TOP_K = 8             # config.py:60
ROUTED_SCALING_FACTOR = 2.446  # config.py:67
RMS_NORM_EPS = 1e-5   # config.py:49


class RMSNorm(nn.Module):
    """engine/klinear/norm.py:16-30 on ``lk_rms_norm``."""

    def __init__(self, hidden_size: int, eps: float = 1e-6, *,
                 device: torch.device | str | None = None, dtype: torch.dtype | None = None) -> None:
        super().__init__()
        self.variance_epsilon = eps
        self.weight = nn.Parameter(torch.ones(hidden_size, device=device, dtype=dtype))

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return rms_norm(hidden_states, self.weight.detach(), self.variance_epsilon)


class RMSGatedNorm(nn.Module):
    """engine/klinear/norm.py:33-52 on ``lk_rms_gated_norm``. ``input_dtype``
    rounds the values first (fp32 KDA outputs to bf16, attention.py:324)."""

    def __init__(self, hidden_size: int, eps: float = 1e-5, *,
                 device: torch.device | str | None = None, dtype: torch.dtype | None = None) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size, device=device, dtype=dtype))

    def forward(self, values: torch.Tensor, gate: torch.Tensor,
                input_dtype: torch.dtype | None = None) -> torch.Tensor:
        return rms_gated_norm(values, gate, self.weight.detach(), self.eps,
                              input_dtype=input_dtype)


class W4A16Linear(nn.Module):
    """A bias-free linear layer over W4A16 weights ``[N, K]``."""

    def __init__(self, encoded: W4A16Tensor) -> None:
        super().__init__()
        self.out_features, self.in_features = encoded.original_shape
        self.group_size = encoded.group_size
        self.register_buffer("packed_weight", encoded.packed, persistent=False)
        self.register_buffer("scales", encoded.scales, persistent=False)
        self._dense_kernel = None

    @classmethod
    def from_encoded(cls, encoded: W4A16Tensor) -> "W4A16Linear":
        return cls(encoded)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if hidden_states.shape[-1] != self.in_features:
            raise ValueError(f"linear input width {hidden_states.shape[-1]} does not match "
                             f"{self.in_features}")
        original_shape = hidden_states.shape[:-1]
        flattened = hidden_states.reshape(-1, self.in_features)
        if self._dense_kernel is None:  # resolved once per module, not per call
            self._dense_kernel = registry.resolve(W4A16_DENSE)
        out = self._dense_kernel(flattened, self.packed_weight, self.scales)
        return out.reshape(*original_shape, self.out_features)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, G={self.group_size}"


class KLinearMoE(nn.Module):
    """Sigmoid top-k router + W4A16 routed experts + shared expert, one layer."""

    def __init__(self, gate_weight: torch.Tensor, e_score_correction_bias: torch.Tensor | None,
                 banks: MoeBanks, *, top_k: int = TOP_K,
                 routed_scaling_factor: float = ROUTED_SCALING_FACTOR,
                 renormalize: bool = True, num_expert_group: int = 1,
                 topk_group: int = 1) -> None:
        super().__init__()
        experts, hidden = gate_weight.shape
        if banks.w1_packed.shape[0] != experts + 1:
            raise ValueError("banks must hold every routed expert plus the shared expert last")
        if banks.w1_packed.shape[2] * 2 != hidden:
            raise ValueError("router and expert banks disagree on the hidden size")
        self.num_experts = experts
        self.hidden_size = hidden
        self.top_k = top_k
        self.routed_scaling_factor = routed_scaling_factor
        self.renormalize = renormalize
        # grouped top-k (router.py:62-80); Kimi-Linear uses one group
        if num_expert_group < 1 or experts % num_expert_group:
            raise ValueError("num_experts must be divisible by num_expert_group")
        self.num_expert_group = num_expert_group
        self.topk_group = topk_group
        # the router computes in fp32 (router.py:51) from the weight as stored:
        # bf16 in the checkpoint layout; fp16 is widened once here (exactly)
        if gate_weight.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise TypeError("the router weight must be BF16, FP16 or FP32")
        if hidden % 8 or hidden > 4096:
            raise ValueError(f"the HIP router needs hidden % 8 == 0 and hidden <= 4096, got {hidden}")
        if gate_weight.dtype == torch.float16:
            gate_weight = gate_weight.float()
        self.register_buffer("gate_weight", gate_weight.contiguous(), persistent=False)
        bias = None if e_score_correction_bias is None else e_score_correction_bias.float().contiguous()
        self.register_buffer("e_score_correction_bias", bias, persistent=False)
        self.banks = banks
        self._block = None

    @classmethod
    def from_checkpoint(cls, index: W4A16Index, layer: int, *, device: torch.device | str,
                        num_experts: int = ROUTED_EXPERTS, hidden: int = HIDDEN,
                        intermediate: int = INTERMEDIATE, top_k: int = TOP_K,
                        routed_scaling_factor: float = ROUTED_SCALING_FACTOR) -> "KLinearMoE":
        """Router weights and the layer's banks from a W4A16 checkpoint."""
        prefix = f"model.layers.{layer}.block_sparse_moe.gate."
        gate = index.load(prefix + "weight", device=device)
        bias_name = prefix + "e_score_correction_bias"
        bias = index.load(bias_name, device=device) if bias_name in index.names else None
        banks = build_moe_banks(index, layer, num_experts=num_experts, hidden=hidden,
                                intermediate=intermediate, device=device)
        return cls(gate, bias, banks, top_k=top_k, routed_scaling_factor=routed_scaling_factor)

    def router_logits(self, flat: torch.Tensor) -> torch.Tensor:
        return router_logits(flat, self.gate_weight)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        if hidden_states.shape[-1] != self.hidden_size:
            raise ValueError(f"MoE input width {hidden_states.shape[-1]} does not match {self.hidden_size}")
        original_shape = hidden_states.shape
        flat = hidden_states.reshape(-1, self.hidden_size)
        if self._block is None:
            self._block = registry.resolve(W4A16_MOE_BLOCK)
        grouping = {} if self.num_expert_group == 1 else {
            "num_expert_group": self.num_expert_group, "topk_group": self.topk_group}
        y, _, _ = self._block(flat, self.router_logits(flat), self.e_score_correction_bias,
                              *self.banks.as_tuple(), self.top_k, self.routed_scaling_factor,
                              self.renormalize, **grouping)
        return y.reshape(original_shape)


class MoEDecodeGraph:
    """One MoE layer's decode step for ``tokens`` rows, captured in a HIP graph.

    Warm-up runs on a side stream (so capture sees initialised workspaces and
    resolved kernels), then one capture; ``__call__`` copies the input into the
    static buffer and replays. Nothing allocates or synchronises per replay.
    """

    def __init__(self, moe: KLinearMoE, tokens: int = 1, *, warmup: int = 2) -> None:
        device = moe.gate_weight.device
        self.moe = moe
        self.static_input = torch.zeros((tokens, moe.hidden_size), dtype=torch.bfloat16, device=device)
        side = torch.cuda.Stream(device=device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            for _ in range(warmup):
                moe(self.static_input)
        torch.cuda.current_stream(device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.static_output = moe(self.static_input)

    def __call__(self, hidden_states: torch.Tensor) -> torch.Tensor:
        self.static_input.copy_(hidden_states)
        self.graph.replay()
        return self.static_output


class MoELayerTail(nn.Module):
    """The post-attention half of a MoE decoder layer (engine/klinear/layer.py:155-170).

    ``forward(residual, attended)`` returns ``hidden = (residual + attended) +
    moe(post_attention_layernorm(residual + attended))``. With ``next_norm``
    (the following layer's input_layernorm) the final residual add runs fused
    with that norm and ``(hidden, next_norm(hidden))`` is returned.
    """

    def __init__(self, moe: KLinearMoE, post_attention_layernorm: RMSNorm) -> None:
        super().__init__()
        self.moe = moe
        self.post_attention_layernorm = post_attention_layernorm

    def forward(self, residual: torch.Tensor, attended: torch.Tensor,
                next_norm: RMSNorm | None = None):
        ln = self.post_attention_layernorm
        hidden, ff_in = add_rms_norm(residual, attended, ln.weight.detach(), ln.variance_epsilon)
        ff = self.moe(ff_in)
        if next_norm is None:
            return hidden + ff
        return add_rms_norm(hidden, ff, next_norm.weight.detach(), next_norm.variance_epsilon)
