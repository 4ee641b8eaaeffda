"""W4A16 / MXFP4 kernel ops for MI355X, registered behind the reference's registry.

Importing this package registers every op and selects the shipped default,
mirroring engine/kernels/__init__.py:19-223: op names ``w4a16_grouped``,
``w4a16_dense`` and ``w4a16_swiglu`` keep the reference signatures; new ops
(``w4a16_fused_qkv``, ``w4a16_w2_combine``, ``w4a16_moe_block``) follow the
same style. Every op has two HIP variants:

* ``reference`` -- one thread per output with the reference's rounding
  contract (weights decoded to ``bf16(q * s)`` before the multiply-add);
  simple and slow, used as the in-process equivalence baseline;
* ``hip`` -- the gfx950 kernels, the shipped default.

Both are ``requires_cuda=True``: on a machine without a GPU the registry
refuses them instead of running anything on the CPU, and a missing HIP library
raises on first call.
"""

from . import registry
from .kda import fused_kda_gates, fused_short_conv_triple, kda_decode_layer, kda_decode_step
from .norm import add_rms_norm, rms_gated_norm, rms_norm
from .moe import (moe_router, moe_schedule, router_logits, shape_stable_expert_indices, w4a16_moe_block,
                  w4a16_moe_block_reference, w4a16_moe_decode, w4a16_moe_forward,
                  w4a16_moe_gateup, w4a16_moe_routed)
from .mxfp4 import (grouped_mxfp4_gemm, grouped_mxfp4_reference, grouped_mxfp4_swiglu_gemm,
                    mxfp4_expert_mlp, mxfp4_gemm, mxfp4_gemm_reference, mxfp4_linear,
                    mxfp4_moe_block, mxfp4_moe_block_reference, split_activations_fp8)
from .w4a16 import (fused_qkv_w4a16, fused_qkv_w4a16_reference, fused_w2_combine,
                    fused_w2_combine_reference, grouped_w4a16_gemm, grouped_w4a16_gemv,
                    grouped_w4a16_reference, grouped_w4a16_swiglu_gemm,
                    grouped_w4a16_swiglu_gemv, route_combine, silu_mul, w4a16_dense,
                    w4a16_dense_gemm, w4a16_dense_reference)

W4A16_GROUPED = "w4a16_grouped"
W4A16_DENSE = "w4a16_dense"
W4A16_SWIGLU = "w4a16_swiglu"
W4A16_FUSED_QKV = "w4a16_fused_qkv"
W4A16_W2_COMBINE = "w4a16_w2_combine"
W4A16_MOE_BLOCK = "w4a16_moe_block"
MXFP4_GEMM = "mxfp4_gemm"
MXFP4_GROUPED = "mxfp4_grouped"
MXFP4_MOE_BLOCK = "mxfp4_moe_block"

HIP = "hip"
REFERENCE = "reference"


def _register_grouped() -> None:
    registry.register(W4A16_GROUPED, REFERENCE, reference=True, requires_cuda=True,
                      description="One thread per output, weights rounded to bf16(q*s).")(
        grouped_w4a16_reference)
    registry.register(W4A16_GROUPED, HIP, requires_cuda=True,
                      description="gfx950 grouped GEMV: 8 lanes per row, 16 B nibble loads, "
                      "bf16 dot2 with per-chunk scales, DPP row reduction.")(grouped_w4a16_gemv)
    registry.set_default(W4A16_GROUPED, HIP)


def _register_dense() -> None:
    registry.register(W4A16_DENSE, REFERENCE, reference=True, requires_cuda=True,
                      description="One thread per output, weights rounded to bf16(q*s).")(
        w4a16_dense_reference)
    registry.register(W4A16_DENSE, HIP, requires_cuda=True,
                      description="gfx950 dense GEMV with LDS-staged activations.")(w4a16_dense)
    registry.set_default(W4A16_DENSE, HIP)


def _register_swiglu() -> None:
    cache: dict[str, object] = {}

    def swiglu_reference(activations, expert_indices, w1_packed, w1_scales, w3_packed, w3_scales):
        """Two grouped calls through the active grouped variant, then silu * up
        (engine/kernels/__init__.py:182-197)."""
        name = registry.active(W4A16_GROUPED)
        kernel = cache.get(name)
        if kernel is None:
            kernel = registry.resolve(W4A16_GROUPED)
            cache[name] = kernel
        gate = kernel(activations, expert_indices, w1_packed, w1_scales)
        up = kernel(activations, expert_indices, w3_packed, w3_scales)
        return silu_mul(gate, up)

    registry.register(W4A16_SWIGLU, REFERENCE, reference=True, requires_cuda=True,
                      description="Two grouped calls plus silu and multiply.")(swiglu_reference)
    registry.register(W4A16_SWIGLU, HIP, requires_cuda=True,
                      description="One launch reading W1 and W3 together, writing only the "
                      "activated result.")(grouped_w4a16_swiglu_gemv)
    registry.set_default(W4A16_SWIGLU, HIP)


def _register_others() -> None:
    registry.register(W4A16_FUSED_QKV, REFERENCE, reference=True, requires_cuda=True,
                      description="Three reference dense calls.")(fused_qkv_w4a16_reference)
    registry.register(W4A16_FUSED_QKV, HIP, requires_cuda=True,
                      description="Q, K, V through the gfx950 dense path.")(fused_qkv_w4a16)
    registry.set_default(W4A16_FUSED_QKV, HIP)

    registry.register(W4A16_W2_COMBINE, REFERENCE, reference=True, requires_cuda=True,
                      description="Reference grouped W2 per route, then the combine kernel.")(
        fused_w2_combine_reference)
    registry.register(W4A16_W2_COMBINE, HIP, requires_cuda=True,
                      description="W2 for all routes plus weighted combine and shared expert "
                      "in one launch.")(fused_w2_combine)
    registry.set_default(W4A16_W2_COMBINE, HIP)

    registry.register(W4A16_MOE_BLOCK, REFERENCE, reference=True, requires_cuda=True,
                      description="Router, reference gate/up, silu*up, reference W2 + combine.")(
        w4a16_moe_block_reference)
    registry.register(W4A16_MOE_BLOCK, HIP, requires_cuda=True,
                      description="Router + gate/up + SwiGLU in one launch, W2 + combine in a "
                      "second.")(w4a16_moe_block)
    registry.set_default(W4A16_MOE_BLOCK, HIP)


def _register_mxfp4() -> None:
    registry.register(MXFP4_GEMM, REFERENCE, reference=True, requires_cuda=True,
                      description="Each weight decoded to the activation dtype, fp32 dot per "
                      "output.")(mxfp4_gemm_reference)
    registry.register(MXFP4_GEMM, HIP, requires_cuda=True,
                      description="Scaled fp4 decode into bf16/fp16 MFMA tiles.")(mxfp4_gemm)
    registry.set_default(MXFP4_GEMM, HIP)

    registry.register(MXFP4_GROUPED, REFERENCE, reference=True, requires_cuda=True,
                      description="Reference GEMM per expert over its gathered rows.")(
        grouped_mxfp4_reference)
    registry.register(MXFP4_GROUPED, HIP, requires_cuda=True,
                      description="Expert-sorted schedule + MFMA GEMM.")(grouped_mxfp4_gemm)
    registry.set_default(MXFP4_GROUPED, HIP)

    registry.register(MXFP4_MOE_BLOCK, REFERENCE, reference=True, requires_cuda=True,
                      description="Router, reference grouped GEMMs, silu*up, combine.")(
        mxfp4_moe_block_reference)
    registry.register(MXFP4_MOE_BLOCK, HIP, requires_cuda=True,
                      description="Router, schedule, gate/up + SwiGLU GEMM, down GEMM, "
                      "combine.")(mxfp4_moe_block)
    registry.set_default(MXFP4_MOE_BLOCK, HIP)


_register_grouped()
_register_dense()
_register_swiglu()
_register_others()
_register_mxfp4()

__all__ = [
    "registry", "kda_decode_step", "kda_decode_layer", "fused_short_conv_triple",
    "fused_kda_gates", "rms_norm", "add_rms_norm", "rms_gated_norm",
    "W4A16_GROUPED", "W4A16_DENSE", "W4A16_SWIGLU", "W4A16_FUSED_QKV",
    "W4A16_W2_COMBINE", "W4A16_MOE_BLOCK", "moe_router", "router_logits",
    "shape_stable_expert_indices",
    "w4a16_moe_block", "w4a16_moe_decode", "w4a16_moe_forward", "w4a16_moe_gateup",
    "w4a16_moe_routed",
    "moe_schedule", "w4a16_dense", "w4a16_dense_gemm", "grouped_w4a16_gemv",
    "grouped_w4a16_gemm", "grouped_w4a16_swiglu_gemv", "grouped_w4a16_swiglu_gemm",
    "fused_w2_combine", "fused_qkv_w4a16", "route_combine", "silu_mul",
    "MXFP4_GEMM", "MXFP4_GROUPED", "MXFP4_MOE_BLOCK", "mxfp4_gemm", "mxfp4_linear",
    "mxfp4_gemm_reference", "grouped_mxfp4_gemm", "grouped_mxfp4_swiglu_gemm",
    "grouped_mxfp4_reference", "mxfp4_moe_block", "mxfp4_moe_block_reference",
    "split_activations_fp8",
    "mxfp4_expert_mlp",
]
