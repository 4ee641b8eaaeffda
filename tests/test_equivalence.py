"""The equivalence harness's own behaviour, on the CPU: every variant gets its
own copies of the inputs, nested containers keep their shape, the factory may
take the device in any of three ways, and the error figures follow their
definitions (max |a - e|; max |a - e| / |e| with 0/0 = 0 and x/0 = inf)."""

from __future__ import annotations

import itertools
import math

import pytest
import torch

from local_kimi_amd.kernels.equivalence import assert_equivalent, check_equivalence
from local_kimi_amd.kernels.registry import register

_ids = itertools.count()


def _op(reference, **variants):
    name = f"test_harness_{next(_ids)}"
    register(name, "baseline", reference=True)(reference)
    for variant, fn in variants.items():
        register(name, variant)(fn)
    return name


def test_in_place_writes_of_one_variant_do_not_reach_another():
    def clobber(v):
        out = v * 2
        v.fill_(1e6)
        return out

    op = _op(lambda v: v * 2, first=clobber, second=lambda v: v * 2)
    reports = check_equivalence(op, lambda: torch.arange(4.0), rtol=0.0, atol=0.0, device="cpu")
    assert [r.variant for r in reports] == ["first", "second"]
    assert all(r.passed and r.exact_match for r in reports)


def test_nested_containers_reach_the_variant_with_their_shape():
    def ref(pair, table, scale):
        assert isinstance(pair, list) and isinstance(table, dict) and scale == 3
        return pair[0] * scale + table["b"][1]

    op = _op(ref, same=ref)
    make = lambda device: ([torch.ones(2), None], {"b": (0, torch.full((2,), 5.0))}, 3)  # noqa: E731
    (report,) = check_equivalence(op, make, rtol=0.0, atol=0.0, device="cpu")
    assert report.passed and report.exact_match


@pytest.mark.parametrize("factory", [lambda d: torch.ones(3, device=d),
                                     lambda *, device: torch.ones(3, device=device),
                                     lambda: torch.ones(3)])
def test_factory_may_take_the_device_positionally_by_keyword_or_not_at_all(factory):
    op = _op(lambda v: v + 1, hip=lambda v: v + 1)
    (report,) = check_equivalence(op, factory, rtol=0.0, atol=0.0, device="cpu")
    assert report.passed


def test_error_figures_follow_their_definitions():
    expected = torch.tensor([0.0, 2.0, -4.0, 0.0])
    off = torch.tensor([0.0, 0.5, 1.0, 0.0])
    op = _op(lambda v: expected.clone(), off=lambda v: expected + off)
    (r,) = check_equivalence(op, lambda: torch.zeros(1), rtol=0.25, atol=0.0, device="cpu")
    assert r.max_abs_err == 1.0 and r.max_rel_err == 0.25 and r.passed and not r.exact_match

    op = _op(lambda v: expected.clone(), off=lambda v: expected + torch.tensor([1e-3, 0, 0, 0]))
    (r,) = check_equivalence(op, lambda: torch.zeros(1), rtol=0.0, atol=1e-2, device="cpu")
    assert r.passed and math.isinf(r.max_rel_err)


def test_shape_mismatch_and_nan_fail_with_infinite_error():
    op = _op(lambda v: torch.zeros(3), short=lambda v: torch.zeros(2),
             nan=lambda v: torch.tensor([0.0, math.nan, 0.0]))
    reports = {r.variant: r for r in check_equivalence(op, lambda: torch.zeros(1), rtol=1.0,
                                                       atol=1.0, device="cpu")}
    for name in ("short", "nan"):
        assert not reports[name].passed and math.isinf(reports[name].max_abs_err)


def test_nan_in_both_outputs_at_the_same_place_counts_as_equal():
    both = lambda v: torch.tensor([1.0, math.nan])  # noqa: E731
    op = _op(both, same=both)
    (r,) = check_equivalence(op, lambda: torch.zeros(1), rtol=0.0, atol=0.0, device="cpu")
    assert r.passed and r.max_abs_err == 0.0


def test_output_count_and_type_are_checked():
    op = _op(lambda v: (v, v), one=lambda v: v)
    (r,) = check_equivalence(op, lambda: torch.zeros(2), rtol=1.0, atol=1.0, device="cpu")
    assert not r.passed
    op = _op(lambda v: v, listy=lambda v: [v])
    with pytest.raises(TypeError, match="tensor or a tuple of tensors"):
        check_equivalence(op, lambda: torch.zeros(2), rtol=1.0, atol=1.0, device="cpu")


def test_failure_table_lists_every_variant():
    op = _op(lambda v: v, good=lambda v: v.clone(), bad=lambda v: v + 1)
    with pytest.raises(AssertionError) as error:
        assert_equivalent(op, lambda: torch.zeros(2), rtol=0.0, atol=0.0, device="cpu")
    lines = str(error.value).splitlines()
    assert lines[0] == f"kernel equivalence failed for operation {op!r}"
    assert lines[1] == "variant | status | max_abs_err | max_rel_err | exact_match | reason"
    assert lines[3].startswith("bad | FAIL | 1 | inf | False")
    assert lines[4].startswith("good | PASS | 0 | 0 | True")
