"""Check every registered variant of an op against its reference variant.

Public interface (kept so that callers of the reference harness,
engine/kernels/equivalence.py:165-286, run unchanged): ``check_equivalence``
and ``assert_equivalent`` with the keyword-only ``rtol``/``atol``/``variants``/
``device`` arguments, the :class:`EquivalenceReport` fields, and the failure
table that ``assert_equivalent`` raises.

Design. The factory's output is taken apart once into a flat list of tensors
on the target device plus a template of the surrounding containers
(:class:`_ArgumentSet`); every run gets the template filled with fresh copies,
so no variant can see another's in-place writes. Each output pair is reduced
to one :class:`_Gap` in float64 on the host, and a variant's gaps fold into
its report. The ops checked here produce real tensors only (bf16, fp16,
fp32, integer indices), so complex outputs are refused rather than compared.
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
    """The comparison result for one kernel variant."""

    op: str
    variant: str
    passed: bool
    max_abs_err: float
    max_rel_err: float
    exact_match: bool
    skipped: bool
    skip_reason: str


# ---------------------------------------------------------------------------
# inputs

class _Slot:
    """Placeholder for the n-th tensor of an argument template."""

    __slots__ = ("n",)

    def __init__(self, n: int) -> None:
        self.n = n


class _ArgumentSet:
    """The factory's arguments as (template, tensors); :meth:`fresh` rebuilds them."""

    def __init__(self, produced: object, device: torch.device) -> None:
        self.tensors: list[torch.Tensor] = []
        args = produced if isinstance(produced, tuple) else (produced,)
        self.template = tuple(self._strip(a, device) for a in args)

    def _strip(self, value: object, device: torch.device) -> object:
        if isinstance(value, torch.Tensor):
            self.tensors.append(value.to(device))
            return _Slot(len(self.tensors) - 1)
        if isinstance(value, (tuple, list)):
            inner = [self._strip(v, device) for v in value]
            return inner if isinstance(value, list) else tuple(inner)
        if isinstance(value, dict):
            return {key: self._strip(v, device) for key, v in value.items()}
        return value

    def fresh(self) -> tuple:
        copies = [t.clone() for t in self.tensors]

        def fill(node: object) -> object:
            if isinstance(node, _Slot):
                return copies[node.n]
            if isinstance(node, list):
                return [fill(v) for v in node]
            if isinstance(node, tuple):
                return tuple(fill(v) for v in node)
            if isinstance(node, dict):
                return {key: fill(v) for key, v in node.items()}
            return node

        return fill(self.template)


def _run_factory(factory: Callable[..., object], device: torch.device) -> object:
    """Call ``factory`` with the device positionally, by keyword, or not at all,
    whichever its signature accepts (in that order of preference)."""
    try:
        sig = inspect.signature(factory)
    except (TypeError, ValueError):  # builtins without introspection take the device
        return factory(device)
    for args, kwargs in (((device,), {}), ((), {"device": device}), ((), {})):
        try:
            sig.bind(*args, **kwargs)
        except TypeError:
            continue
        return factory(*args, **kwargs)
    return factory()  # raises the factory's own argument error


# ---------------------------------------------------------------------------
# comparison

@dataclass(frozen=True)
class _Gap:
    """How far one output lies from the reference output."""

    abs_err: float
    rel_err: float
    within: bool
    identical: bool

    @staticmethod
    def unmatched() -> "_Gap":
        return _Gap(math.inf, math.inf, False, False)

    def join(self, other: "_Gap") -> "_Gap":
        return _Gap(max(self.abs_err, other.abs_err), max(self.rel_err, other.rel_err),
                    self.within and other.within, self.identical and other.identical)


def _as_outputs(value: object) -> tuple[torch.Tensor, ...]:
    outs = value if isinstance(value, tuple) else (value,)
    if not all(isinstance(t, torch.Tensor) for t in outs):
        raise TypeError("kernel output must be a tensor or a tuple of tensors")
    return outs


def _gap(actual: torch.Tensor, expected: torch.Tensor, rtol: float, atol: float) -> _Gap:
    if actual.shape != expected.shape:
        return _Gap.unmatched()
    if actual.is_complex() or expected.is_complex():
        raise TypeError("complex kernel outputs are not supported by this harness")
    a = actual.detach().cpu()
    e = expected.detach().cpu()
    identical = a.dtype == e.dtype and torch.equal(a, e)
    if a.numel() == 0:
        return _Gap(0.0, 0.0, True, identical)
    a64, e64 = a.double(), e.double()
    both_nan = a64.isnan() & e64.isnan()
    diff = (a64 - e64).abs().masked_fill(both_nan, 0.0).nan_to_num(nan=math.inf, posinf=math.inf)
    bound = atol + rtol * e64.abs().nan_to_num(nan=0.0, posinf=math.inf)
    within = bool((diff <= bound).all())
    # relative error: 0 where both agree exactly, inf where the reference is 0 and the output not
    rel = (diff / e64.abs()).masked_fill(diff == 0, 0.0).nan_to_num(nan=math.inf, posinf=math.inf)
    return _Gap(float(diff.max()), float(rel.max()), within, identical)


def _skip_reason(variant: registry.KernelVariant, device: torch.device) -> str:
    if not variant.requires_cuda:
        return ""
    if not torch.cuda.is_available():
        return "CUDA is not available"
    if device.type != "cuda":
        return f"variant requires CUDA but device is {device.type}"
    return ""


# ---------------------------------------------------------------------------
# public entry points

def check_equivalence(op: str, make_inputs: Callable[..., object], *, rtol: float, atol: float,
                      variants: Sequence[str] | None = None,
                      device: str | torch.device | None = None) -> list[EquivalenceReport]:
    """Run the reference variant once and compare every selected variant with it."""
    if device is None:
        device = "cuda" if torch.cuda.is_available() else "cpu"
    device = torch.device(device)
    args = _ArgumentSet(_run_factory(make_inputs, device), device)
    ref = registry.reference_of(op)
    expected = _as_outputs(ref.fn(*args.fresh()))
    chosen = list(variants) if variants is not None else [
        name for name in registry.variants(op) if name != ref.name]

    reports: list[EquivalenceReport] = []
    for name in chosen:
        variant = registry.get_variant(op, name)
        reason = _skip_reason(variant, device)
        if reason:
            reports.append(EquivalenceReport(op, name, passed=False, max_abs_err=math.nan,
                                             max_rel_err=math.nan, exact_match=False,
                                             skipped=True, skip_reason=reason))
            continue
        got = _as_outputs(variant.fn(*args.fresh()))
        total = _Gap(0.0, 0.0, True, True)
        if len(got) != len(expected):
            total = _Gap.unmatched()
        else:
            for g, e in zip(got, expected):
                total = total.join(_gap(g, e, rtol, atol))
        reports.append(EquivalenceReport(op, name, passed=total.within, max_abs_err=total.abs_err,
                                         max_rel_err=total.rel_err, exact_match=total.identical,
                                         skipped=False, skip_reason=""))
    return reports


_TABLE_HEAD = ("variant | status | max_abs_err | max_rel_err | exact_match | reason",
               "------- | ------ | ----------- | ----------- | ----------- | ------")


def _number(v: float) -> str:
    if math.isnan(v):
        return "n/a"
    return "inf" if math.isinf(v) else f"{v:.6g}"


def _row(r: EquivalenceReport) -> str:
    status = "SKIP" if r.skipped else ("PASS" if r.passed else "FAIL")
    cells = (r.variant, status, _number(r.max_abs_err), _number(r.max_rel_err),
             str(r.exact_match), r.skip_reason)
    return " | ".join(cells)


def assert_equivalent(op: str, make_inputs: Callable[..., object], *, rtol: float, atol: float,
                      variants: Sequence[str] | None = None,
                      device: str | torch.device | None = None) -> list[EquivalenceReport]:
    """:func:`check_equivalence`, raising ``AssertionError`` with a table on any failure."""
    reports = check_equivalence(op, make_inputs, rtol=rtol, atol=atol, variants=variants,
                                device=device)
    if any(not (r.skipped or r.passed) for r in reports):
        text = [f"kernel equivalence failed for operation {op!r}", *_TABLE_HEAD,
                *(_row(r) for r in reports)]
        raise AssertionError("\n".join(text))
    return reports
