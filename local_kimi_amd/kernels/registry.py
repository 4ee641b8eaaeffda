"""Registration and selection of interchangeable kernel implementations.

Mirrors the reference's plugin interface (engine/kernels/registry.py:34-204):
same functions, same selection order and the same errors, so a caller written
against the reference registry selects these HIP variants unchanged.

Selection order: programmatic override (``use``/``using``), then the
``KIMI_KERNELS=op=variant,...`` environment variable, then the shipped default
(``set_default``), then the op's reference variant. A variant registered with
``requires_cuda=True`` is refused by :func:`resolve` when
``torch.cuda.is_available()`` is False (on ROCm this is the HIP device check).
"""

from __future__ import annotations

import os
from collections.abc import Callable, Iterator
from contextlib import contextmanager
from dataclasses import dataclass
from typing import TypeVar, cast

import torch

KernelFunction = Callable[..., object]
_Function = TypeVar("_Function", bound=KernelFunction)


@dataclass(frozen=True)
class KernelVariant:
    """One named implementation of a kernel operation."""

    name: str
    fn: KernelFunction
    is_reference: bool
    requires_cuda: bool
    description: str


_REGISTRY: dict[str, dict[str, KernelVariant]] = {}
_OVERRIDES: dict[str, str] = {}
_DEFAULTS: dict[str, str] = {}
_MISSING = object()


def register(op: str, variant: str, *, reference: bool = False, requires_cuda: bool = False,
             description: str = "") -> Callable[[_Function], _Function]:
    """Register a function as a named implementation of an operation (registry.py:34-69)."""

    def decorator(fn: _Function) -> _Function:
        registered = _REGISTRY.setdefault(op, {})
        if reference:
            existing = next((v for v in registered.values() if v.is_reference), None)
            if existing is not None:
                raise ValueError(
                    f"operation {op!r} already has reference variant {existing.name!r}; "
                    f"cannot register second reference variant {variant!r}"
                )
        if variant in registered:
            raise ValueError(f"variant {variant!r} is already registered for operation {op!r}")
        registered[variant] = KernelVariant(variant, fn, reference, requires_cuda, description)
        return fn

    return decorator


def reference_of(op: str) -> KernelVariant:
    for variant in _REGISTRY.get(op, {}).values():
        if variant.is_reference:
            return variant
    raise KeyError(f"operation {op!r} has no reference kernel variant")


def variants(op: str) -> tuple[str, ...]:
    """Registered names: the reference first, then the others sorted."""
    registered = _REGISTRY.get(op, {})
    refs = sorted(v.name for v in registered.values() if v.is_reference)
    others = sorted(v.name for v in registered.values() if not v.is_reference)
    return tuple(refs + others)


def operations() -> tuple[str, ...]:
    return tuple(sorted(_REGISTRY))


def _variant_of(op: str, variant: str) -> KernelVariant:
    registered = _REGISTRY.get(op)
    if registered is None:
        raise KeyError(f"operation {op!r} has no registered kernel variants")
    try:
        return registered[variant]
    except KeyError as error:
        available = ", ".join(variants(op)) or "none"
        raise ValueError(
            f"unknown variant {variant!r} for operation {op!r}; available variants: {available}"
        ) from error


def _environment_overrides() -> dict[str, str]:
    selected: dict[str, str] = {}
    for raw_entry in os.getenv("KIMI_KERNELS", "").split(","):
        entry = raw_entry.strip()
        if not entry:
            continue
        raw_op, separator, raw_variant = entry.partition("=")
        op = raw_op.strip()
        variant = raw_variant.strip()
        if not separator or not op:
            raise ValueError(f"invalid KIMI_KERNELS entry {entry!r}; expected op=variant")
        if op not in _REGISTRY:
            continue
        if not variant:
            available = ", ".join(variants(op)) or "none"
            raise ValueError(
                f"unknown variant {variant!r} for operation {op!r}; available variants: {available}"
            )
        _variant_of(op, variant)
        selected[op] = variant
    return selected


def set_default(op: str, variant: str) -> None:
    """Choose the shipped variant, used when no override or environment entry selects one."""
    _variant_of(op, variant)
    _DEFAULTS[op] = variant


def default_of(op: str) -> str:
    return _DEFAULTS.get(op, reference_of(op).name)


def _selected_variant(op: str) -> KernelVariant:
    if op not in _REGISTRY:
        raise KeyError(f"operation {op!r} has no registered kernel variants")
    override = _OVERRIDES.get(op)
    if override is not None:
        return _variant_of(op, override)
    env_variant = _environment_overrides().get(op)
    if env_variant is not None:
        return _variant_of(op, env_variant)
    shipped = _DEFAULTS.get(op)
    if shipped is not None:
        return _variant_of(op, shipped)
    return reference_of(op)


def resolve(op: str) -> KernelFunction:
    """Return the selected function; refuse a GPU variant on a machine without one."""
    selected = _selected_variant(op)
    if selected.requires_cuda and not torch.cuda.is_available():
        raise RuntimeError(
            f"kernel variant {selected.name!r} for operation {op!r} requires CUDA, "
            "but torch.cuda.is_available() is False"
        )
    return selected.fn


def use(op: str, variant: str) -> None:
    _variant_of(op, variant)
    _OVERRIDES[op] = variant


def clear_override(op: str) -> None:
    _OVERRIDES.pop(op, None)


@contextmanager
def using(op: str, variant: str) -> Iterator[None]:
    """Temporarily override an operation, restoring the previous selection."""
    previous = _OVERRIDES.get(op, _MISSING)
    use(op, variant)
    try:
        yield
    finally:
        if previous is _MISSING:
            _OVERRIDES.pop(op, None)
        else:
            _OVERRIDES[op] = cast(str, previous)


def active(op: str) -> str:
    return _selected_variant(op).name
