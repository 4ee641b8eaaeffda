"""Compare every registered variant of an op with its reference variant.

Same interface as the reference harness (engine/kernels/equivalence.py:165-286):
``check_equivalence(op, make_inputs, rtol=, atol=, variants=, device=)`` runs
the reference variant once on cloned inputs, runs each other variant on its own
clone, and reports max abs / rel error and bit-exactness; ``assert_equivalent``
raises with a table when any non-skipped variant fails.
"""

from __future__ import annotations

import inspect
import math
from collections.abc import Callable, Sequence
from dataclasses import dataclass

import torch

from . import registry


@dataclass(frozen=True)
class EquivalenceReport:
    op: str
    variant: str
    passed: bool
    max_abs_err: float
    max_rel_err: float
    exact_match: bool
    skipped: bool
    skip_reason: str


def _call_factory(factory: Callable[..., object], device: torch.device) -> tuple:
    try:
        params = inspect.signature(factory).parameters
    except (TypeError, ValueError):
        params = None
    if params is None:
        produced = factory(device)
    elif len(params) == 0:
        produced = factory()
    elif "device" in params:
        produced = factory(device=device)
    else:
        produced = factory(device)
    return produced if isinstance(produced, tuple) else (produced,)


def _map(value, fn):
    if isinstance(value, torch.Tensor):
        return fn(value)
    if isinstance(value, tuple):
        return tuple(_map(v, fn) for v in value)
    if isinstance(value, list):
        return [_map(v, fn) for v in value]
    if isinstance(value, dict):
        return {k: _map(v, fn) for k, v in value.items()}
    return value


def _outputs(value) -> tuple[torch.Tensor, ...]:
    out = value if isinstance(value, tuple) else (value,)
    if not all(isinstance(t, torch.Tensor) for t in out):
        raise TypeError("kernel output must be a tensor or a tuple of tensors")
    return out


def _compare(actual: torch.Tensor, expected: torch.Tensor, rtol: float, atol: float):
    if actual.shape != expected.shape:
        return False, False, math.inf, math.inf
    exact = actual.dtype == expected.dtype and actual.device == expected.device and torch.equal(actual, expected)
    dtype = torch.complex128 if (actual.is_complex() or expected.is_complex()) else torch.float64
    a = actual.detach().to("cpu", dtype)
    e = expected.detach().to("cpu", dtype)
    diff = (a - e).abs()
    if diff.numel() == 0:
        return True, exact, 0.0, 0.0
    passed = bool(torch.all(diff <= atol + rtol * e.abs()).item())
    rel = torch.where(e.abs() == 0,
                      torch.where(diff == 0, torch.zeros_like(diff), torch.full_like(diff, math.inf)),
                      diff / e.abs())
    return passed, exact, float(diff.max().item()), float(rel.max().item())


def check_equivalence(op: str, make_inputs: Callable[..., object], *, rtol: float, atol: float,
                      variants: Sequence[str] | None = None,
                      device: str | torch.device | None = None) -> list[EquivalenceReport]:
    target = torch.device(device if device is not None else ("cuda" if torch.cuda.is_available() else "cpu"))
    inputs = _map(_call_factory(make_inputs, target), lambda t: t.to(target))
    reference = registry.reference_of(op)
    expected = reference.fn(*_map(inputs, lambda t: t.clone()))
    names = tuple(variants) if variants is not None else tuple(
        n for n in registry.variants(op) if n != reference.name)
    reports: list[EquivalenceReport] = []
    for name in names:
        cand = registry.get_variant(op, name)
        skip = ""
        if cand.requires_cuda and not torch.cuda.is_available():
            skip = "CUDA is not available"
        elif cand.requires_cuda and target.type != "cuda":
            skip = f"variant requires CUDA but device is {target.type}"
        if skip:
            reports.append(EquivalenceReport(op, name, False, math.nan, math.nan, False, True, skip))
            continue
        actual = cand.fn(*_map(inputs, lambda t: t.clone()))
        a_out, e_out = _outputs(actual), _outputs(expected)
        if len(a_out) != len(e_out):
            reports.append(EquivalenceReport(op, name, False, math.inf, math.inf, False, False, ""))
            continue
        passed, exact, mabs, mrel = True, True, 0.0, 0.0
        for a, e in zip(a_out, e_out):
            p, x, ab, re = _compare(a, e, rtol, atol)
            passed, exact = passed and p, exact and x
            mabs, mrel = max(mabs, ab), max(mrel, re)
        reports.append(EquivalenceReport(op, name, passed, mabs, mrel, exact, False, ""))
    return reports


def _fmt(v: float) -> str:
    return "n/a" if math.isnan(v) else "inf" if math.isinf(v) else f"{v:.6g}"


def assert_equivalent(op: str, make_inputs: Callable[..., object], *, rtol: float, atol: float,
                      variants: Sequence[str] | None = None,
                      device: str | torch.device | None = None) -> list[EquivalenceReport]:
    reports = check_equivalence(op, make_inputs, rtol=rtol, atol=atol, variants=variants, device=device)
    if any(not r.skipped and not r.passed for r in reports):
        lines = [f"kernel equivalence failed for operation {op!r}",
                 "variant | status | max_abs_err | max_rel_err | exact_match | reason",
                 "------- | ------ | ----------- | ----------- | ----------- | ------"]
        for r in reports:
            status = "SKIP" if r.skipped else "PASS" if r.passed else "FAIL"
            lines.append(f"{r.variant} | {status} | {_fmt(r.max_abs_err)} | {_fmt(r.max_rel_err)} | "
                         f"{r.exact_match} | {r.skip_reason}")
        raise AssertionError("\n".join(lines))
    return reports
