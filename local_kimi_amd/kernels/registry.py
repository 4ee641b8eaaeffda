"""Named, interchangeable implementations of each kernel operation.

The public functions, their exception types and their messages are the
reference's plugin contract (engine/kernels/registry.py:34-204), so a caller
written against that registry selects this package's HIP variants unchanged:
``register`` (decorator), ``set_default`` / ``default_of``, ``use`` /
``clear_override`` / ``using``, ``resolve`` and ``active``.

Design. Every operation is one :class:`_Operation` that owns its variants and
its two pieces of selection state (the programmatic override and the shipped
default). Selection walks a fixed chain of selectors, each of which either
names a variant or passes:

1. the programmatic override (``use`` / ``using``);
2. the ``KIMI_KERNELS="op=variant,..."`` environment entry for the op;
3. the shipped default (``set_default``);
4. the op's reference variant.

``KIMI_KERNELS`` is parsed on every selection (so a changed environment takes
effect at once) and every entry naming a registered op is validated, whichever
op is being selected; entries for unknown ops are ignored, so one setting can
serve several builds. A variant registered with ``requires_cuda=True`` is
refused by :func:`resolve` when ``torch.cuda.is_available()`` is False (on
ROCm that is the HIP device check) rather than silently replaced.
"""

from __future__ import annotations

import os
from collections.abc import Callable, Iterator
from contextlib import contextmanager
from dataclasses import dataclass, field
from typing import TypeVar

import torch

KernelFunction = Callable[..., object]
_F = TypeVar("_F", bound=KernelFunction)

ENV_VAR = "KIMI_KERNELS"


@dataclass(frozen=True)
class KernelVariant:
    """One named implementation of a kernel operation."""

    name: str
    fn: KernelFunction
    is_reference: bool
    requires_cuda: bool
    description: str


@dataclass
class _Operation:
    """The variants of one operation and its selection state."""

    name: str
    table: dict[str, KernelVariant] = field(default_factory=dict)
    override: str | None = None
    shipped: str | None = None

    def names(self) -> tuple[str, ...]:
        refs = [v.name for v in self.table.values() if v.is_reference]
        rest = [v.name for v in self.table.values() if not v.is_reference]
        return tuple(sorted(refs) + sorted(rest))

    def reference(self) -> KernelVariant | None:
        return next((v for v in self.table.values() if v.is_reference), None)

    def get(self, variant: str) -> KernelVariant:
        found = self.table.get(variant)
        if found is None:
            available = ", ".join(self.names()) or "none"
            raise ValueError(f"unknown variant {variant!r} for operation {self.name!r}; "
                             f"available variants: {available}")
        return found

    def add(self, entry: KernelVariant) -> None:
        if entry.is_reference:
            held = self.reference()
            if held is not None:
                raise ValueError(f"operation {self.name!r} already has reference variant "
                                 f"{held.name!r}; cannot register second reference variant "
                                 f"{entry.name!r}")
        if entry.name in self.table:
            raise ValueError(f"variant {entry.name!r} is already registered for operation "
                             f"{self.name!r}")
        self.table[entry.name] = entry


_operations: dict[str, _Operation] = {}


def _operation(op: str) -> _Operation:
    found = _operations.get(op)
    if found is None:
        raise KeyError(f"operation {op!r} has no registered kernel variants")
    return found


def register(op: str, variant: str, *, reference: bool = False, requires_cuda: bool = False,
             description: str = "") -> Callable[[_F], _F]:
    """Decorator registering ``fn`` as variant ``variant`` of operation ``op``.

    At most one variant per op may be the reference; names are unique per op.
    """

    def add(fn: _F) -> _F:
        entry = KernelVariant(variant, fn, reference, requires_cuda, description)
        _operations.setdefault(op, _Operation(op)).add(entry)
        return fn

    return add


def operations() -> tuple[str, ...]:
    return tuple(sorted(_operations))


def variants(op: str) -> tuple[str, ...]:
    """Registered names: the reference first, then the others sorted (empty
    for an unknown op)."""
    found = _operations.get(op)
    return found.names() if found is not None else ()


def reference_of(op: str) -> KernelVariant:
    found = _operations.get(op)
    ref = found.reference() if found is not None else None
    if ref is None:
        raise KeyError(f"operation {op!r} has no reference kernel variant")
    return ref


def get_variant(op: str, variant: str) -> KernelVariant:
    """The named variant; KeyError for an unknown op, ValueError for an unknown name."""
    return _operation(op).get(variant)


# ---------------------------------------------------------------------------
# the KIMI_KERNELS environment entry


def _parse_environment() -> dict[str, str]:
    """Validated ``op -> variant`` choices from KIMI_KERNELS (registered ops only)."""
    chosen: dict[str, str] = {}
    for piece in os.environ.get(ENV_VAR, "").split(","):
        text = piece.strip()
        if not text:
            continue
        op, has_sep, variant = (part.strip() for part in text.partition("="))
        if not has_sep or not op:
            raise ValueError(f"invalid {ENV_VAR} entry {text!r}; expected op=variant")
        target = _operations.get(op)
        if target is None:
            continue  # an op this build does not have
        chosen[op] = target.get(variant).name  # an empty or unknown name raises here
    return chosen


# ---------------------------------------------------------------------------
# selection


def _from_override(entry: _Operation) -> str | None:
    return entry.override


def _from_environment(entry: _Operation) -> str | None:
    return _parse_environment().get(entry.name)


def _from_shipped(entry: _Operation) -> str | None:
    return entry.shipped


def _from_reference(entry: _Operation) -> str | None:
    ref = entry.reference()
    if ref is None:
        raise KeyError(f"operation {entry.name!r} has no reference kernel variant")
    return ref.name


_SELECTORS = (_from_override, _from_environment, _from_shipped, _from_reference)


def _selected(op: str) -> KernelVariant:
    entry = _operation(op)
    for selector in _SELECTORS:
        name = selector(entry)
        if name is not None:
            return entry.get(name)
    raise AssertionError("the reference selector always decides")


def set_default(op: str, variant: str) -> None:
    """The shipped choice: used when neither an override nor KIMI_KERNELS picks one."""
    entry = _operation(op)
    entry.shipped = entry.get(variant).name


def default_of(op: str) -> str:
    found = _operations.get(op)
    if found is not None and found.shipped is not None:
        return found.shipped
    return reference_of(op).name


def use(op: str, variant: str) -> None:
    """Programmatic override, above KIMI_KERNELS and the shipped default."""
    entry = _operation(op)
    entry.override = entry.get(variant).name


def clear_override(op: str) -> None:
    found = _operations.get(op)
    if found is not None:
        found.override = None


@contextmanager
def using(op: str, variant: str) -> Iterator[None]:
    """Override ``op`` for the body, then restore whatever override was there."""
    entry = _operation(op)
    saved = entry.override
    use(op, variant)
    try:
        yield
    finally:
        entry.override = saved


def active(op: str) -> str:
    """Name of the variant :func:`resolve` would return."""
    return _selected(op).name


def resolve(op: str) -> KernelFunction:
    """The selected implementation; a CUDA-only variant is refused without a GPU."""
    chosen = _selected(op)
    if chosen.requires_cuda and not torch.cuda.is_available():
        raise RuntimeError(f"kernel variant {chosen.name!r} for operation {op!r} requires CUDA, "
                           "but torch.cuda.is_available() is False")
    return chosen.fn
