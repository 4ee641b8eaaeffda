"""Registry semantics (mirrors the reference's tests/test_kernel_registry.py and
tests/test_kernel_defaults.py against this package's registry)."""

from __future__ import annotations

import pytest
import torch

from local_kimi_amd.kernels import (W4A16_DENSE, W4A16_GROUPED, W4A16_MOE_BLOCK, W4A16_SWIGLU,
                                    W4A16_W2_COMBINE, W4A16_FUSED_QKV, registry)
from local_kimi_amd.kernels.equivalence import assert_equivalent, check_equivalence
from local_kimi_amd.kernels.registry import active, register, resolve, use, using


def test_duplicate_reference_raises_and_names_both_variants():
    op = "test_duplicate_reference"

    @register(op, "baseline", reference=True)
    def baseline(v):
        return v

    with pytest.raises(ValueError) as error:
        @register(op, "replacement", reference=True)
        def replacement(v):
            return v

    assert "baseline" in str(error.value) and "replacement" in str(error.value)


def test_unknown_environment_variant_names_available_options(monkeypatch):
    op = "test_unknown_env_variant"
    register(op, "baseline", reference=True)(lambda v: v)
    register(op, "fast")(lambda v: v)
    monkeypatch.setenv("KIMI_KERNELS", f"{op}=typo")
    with pytest.raises(ValueError) as error:
        resolve(op)
    for word in (op, "typo", "baseline", "fast"):
        assert word in str(error.value)


def test_malformed_environment_entry_is_rejected(monkeypatch):
    monkeypatch.setenv("KIMI_KERNELS", "no_separator")
    with pytest.raises(ValueError, match="expected op=variant"):
        active(W4A16_DENSE)


def test_unknown_environment_operation_is_ignored(monkeypatch):
    op = "test_unknown_env_op"
    register(op, "baseline", reference=True)(lambda v: v + 1)
    monkeypatch.setenv("KIMI_KERNELS", "future_operation=future_variant")
    assert active(op) == "baseline"
    assert torch.equal(resolve(op)(torch.tensor([2.0])), torch.tensor([3.0]))


def test_using_restores_state_when_body_raises():
    op = "test_using_restores"
    register(op, "baseline", reference=True)(lambda v: v)
    register(op, "experimental")(lambda v: v + 1)
    with pytest.raises(RuntimeError, match="body failed"):
        with using(op, "experimental"):
            assert active(op) == "experimental"
            with using(op, "baseline"):
                assert active(op) == "baseline"
            assert active(op) == "experimental"
            raise RuntimeError("body failed")
    assert active(op) == "baseline"


def test_active_reports_environment_then_programmatic_override(monkeypatch):
    op = "test_active_order"
    register(op, "baseline", reference=True)(lambda v: v)
    register(op, "environment_choice")(lambda v: v)
    monkeypatch.setenv("KIMI_KERNELS", f" {op} = environment_choice ")
    assert active(op) == "environment_choice"
    use(op, "baseline")
    assert active(op) == "baseline"
    registry.clear_override(op)


def test_requires_cuda_variant_raises_instead_of_falling_back(monkeypatch):
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    for op in (W4A16_DENSE, W4A16_GROUPED, W4A16_SWIGLU, W4A16_W2_COMBINE, W4A16_MOE_BLOCK):
        for variant in registry.variants(op):
            with using(op, variant):
                with pytest.raises(RuntimeError) as error:
                    resolve(op)
                assert variant in str(error.value) and "CUDA" in str(error.value)


def test_equivalence_reports_known_bad_variant_as_failed():
    op = "test_equivalence_bad"
    register(op, "baseline", reference=True)(lambda v: v)
    register(op, "wrong")(lambda v: v * 1.01)
    reports = check_equivalence(op, lambda device: (torch.tensor([1.0, -4.0, 100.0], device=device),),
                                rtol=1e-6, atol=1e-6, device="cpu")
    assert len(reports) == 1 and not reports[0].passed and reports[0].max_abs_err > 0
    with pytest.raises(AssertionError, match="wrong | FAIL"):
        assert_equivalent(op, lambda device: (torch.tensor([1.0], device=device),), rtol=1e-6,
                          atol=1e-6, device="cpu")


def test_equivalence_skips_cuda_variant_when_cuda_is_unavailable(monkeypatch):
    op = "test_equivalence_skip"
    register(op, "baseline", reference=True)(lambda v: v)

    @register(op, "cuda_fast", requires_cuda=True)
    def cuda_fast(v):
        raise AssertionError("a skipped CUDA variant must not execute")

    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    reports = check_equivalence(op, lambda: (torch.ones(2),), rtol=0.0, atol=0.0, device="cpu")
    assert reports[0].skipped and "CUDA" in reports[0].skip_reason


def test_shipped_defaults_are_the_hip_kernels(monkeypatch):
    monkeypatch.delenv("KIMI_KERNELS", raising=False)
    for op in (W4A16_DENSE, W4A16_GROUPED, W4A16_SWIGLU, W4A16_FUSED_QKV, W4A16_W2_COMBINE,
               W4A16_MOE_BLOCK):
        assert registry.default_of(op) == "hip"
        assert registry.active(op) == "hip"
        assert registry.variants(op) == ("reference", "hip")


def test_environment_variable_still_overrides_the_shipped_default(monkeypatch):
    monkeypatch.setenv("KIMI_KERNELS", f"{W4A16_GROUPED}=reference")
    assert registry.active(W4A16_GROUPED) == "reference"
    with using(W4A16_GROUPED, "hip"):
        assert registry.active(W4A16_GROUPED) == "hip"
