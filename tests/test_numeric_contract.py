"""The output contract (autotuner_runtime.numeric / exact) on CPU tensors.

The known-answer tables are the reference's (tests/test_numeric_contract.py:
10-135, for its autotuner_runtime/numeric.py:1-122): exact vs tolerance on
signed zeros, NaN, infinities and a small relative change; integer outputs
that no float tolerance may loosen; an overflowing subtraction that must not
pass; tolerance validation; per-dtype defaults; a NaN inside the comparison
failing closed. Plus the max-abs-normalised form the region checks use.
"""

from __future__ import annotations

import pytest
import torch

from autotuner_runtime import numeric
from autotuner_runtime.exact import bitwise_equal
from autotuner_runtime.numeric import (MAX_TOLERANCE, check, compare, max_abs_normalised,
                                       tolerance_for)


@pytest.mark.parametrize("dtype, value", [
    (torch.int32, 2**24),
    (torch.int64, 2**40),
    (torch.uint8, 7),
    (torch.bool, False),
])
def test_nonfloating_corruption_is_rejected_whatever_the_tolerance(dtype, value):
    reference = torch.tensor([value], dtype=dtype)
    corrupted = torch.tensor([not value if dtype == torch.bool else value + 1], dtype=dtype)
    result = compare(corrupted, reference, rtol=1.0, atol=100.0)
    assert not result.passed and result.max_excess == float("inf")
    assert not check(corrupted, reference).passed


def test_uint32_words_above_2_pow_24_stay_exact():
    reference = torch.tensor([2**24 + 1], dtype=torch.int64).to(torch.uint32)
    corrupted = torch.tensor([2**24], dtype=torch.int64).to(torch.uint32)
    # float32 cannot tell these apart; the contract must
    assert torch.tensor(2**24 + 1, dtype=torch.float32) == torch.tensor(2**24, dtype=torch.float32)
    assert not check(corrupted, reference).passed
    assert not compare(corrupted.view(torch.int32), reference.view(torch.int32), 1.0, 100.0).passed
    assert check(reference.clone(), reference).passed


@pytest.mark.parametrize("dtype, value", [(torch.int32, 2**24 + 1), (torch.bool, True)])
def test_matching_nonfloating_outputs_pass(dtype, value):
    reference = torch.tensor([value], dtype=dtype)
    same = reference.clone()
    assert compare(same, reference, rtol=0.0, atol=0.0).passed
    assert check(same, reference).passed


@pytest.mark.parametrize("reference,candidate,exact,passed", [
    ([0.0], [-0.0], True, False),
    ([0.0], [-0.0], False, True),
    ([1.0], [1.001], True, False),
    ([1.0], [1.001], False, True),
    ([float("nan")], [float("nan")], False, True),
    ([float("inf")], [-float("inf")], False, False),
    ([float("inf")], [float("inf")], False, True),
    ([1.0], [float("nan")], False, False),
])
def test_shared_policy_exact_and_tolerance(reference, candidate, exact, passed):
    result = check(torch.tensor(candidate), torch.tensor(reference), exact=exact,
                   rtol=0.01, atol=0.001)
    assert result.passed is passed


def test_tolerance_cannot_hide_extreme_subtraction_overflow():
    reference = torch.tensor([3e38], dtype=torch.float32)
    candidate = -reference
    assert not check(candidate, reference, exact=False, rtol=1.5, atol=0.0).passed
    assert check(candidate, reference, exact=False, rtol=2.5, atol=0.0).passed


def test_output_defaults_follow_each_dtype():
    assert tolerance_for(torch.float16) == (1e-2, 2e-2)
    assert tolerance_for(torch.float32) == (1e-5, 1e-6)
    assert tolerance_for(torch.bfloat16) == (2e-2, 4e-2)
    assert tolerance_for(torch.int32) == (0.0, 0.0)
    assert tolerance_for(torch.float16, (0.01, 0.0001)) == (0.01, 0.0001)


@pytest.mark.parametrize("values", [(float("nan"), 0), (-1, 0), (True, 0), (0, float("inf"))])
def test_shared_policy_rejects_invalid_tolerances(values):
    with pytest.raises(ValueError, match="finite non-negative"):
        check(torch.tensor([1.0]), torch.tensor([1.0]), exact=False, rtol=values[0], atol=values[1])


def test_exact_mismatch_has_no_fictitious_numeric_distance():
    result = check(torch.tensor([1.0]), torch.tensor([2.0]))
    assert not result.passed
    assert result.reason == "exact"
    assert result.max_excess is None


def test_shape_and_dtype_changes_fail_both_ways():
    a = torch.zeros(2, 3)
    assert check(a, torch.zeros(3, 2)).reason == "shape"
    assert check(a.half(), a).reason == "dtype"
    assert compare(a, torch.zeros(3, 2), 1.0, 1.0).reason == "shape"
    assert compare(a.bfloat16(), a, 1.0, 1.0).reason == "dtype"
    assert compare(torch.zeros(0), torch.zeros(0), 0.0, 0.0).passed


@pytest.mark.parametrize("candidate, reference, rtol, atol", [
    (1.0, 0.0, 1e300, 0.0),
    (3e38, -3e38, 0.0, 4e38),
])
def test_unrepresentable_tolerances_cannot_overflow_into_a_silent_pass(candidate, reference, rtol, atol):
    with pytest.raises(ValueError, match="fit in float32"):
        check(torch.tensor([candidate]), torch.tensor([reference]), exact=False, rtol=rtol, atol=atol)


def test_nan_comparison_error_is_never_an_acceptance(monkeypatch):
    monkeypatch.setattr(numeric, "_worst", lambda *_: float("nan"))
    result = check(torch.tensor([1.0]), torch.tensor([0.0]), exact=False, rtol=0.0, atol=0.0)
    assert not result.passed
    assert result.reason == "nonfinite_error"


def test_largest_finite_tolerance_still_obeys_zero_reference_rule():
    result = check(torch.tensor([1.0]), torch.tensor([0.0]), exact=False, rtol=MAX_TOLERANCE, atol=0.0)
    assert not result.passed


def test_worst_offender_is_reported():
    r = torch.tensor([[1.0, 2.0], [3.0, 4.0]])
    c = r.clone()
    c[1, 0] += 1.0
    c[0, 1] += 0.5
    result = compare(c, r, rtol=0.0, atol=0.1)
    assert not result.passed and result.index == (1, 0)
    assert result.max_excess == pytest.approx(0.9)


def test_bitwise_equal_sees_signed_zero_and_nan_payloads():
    assert bitwise_equal(torch.tensor([float("nan")]), torch.tensor([float("nan")]))
    assert not bitwise_equal(torch.tensor([0.0]), torch.tensor([-0.0]))
    b = torch.tensor([1.0], dtype=torch.bfloat16)
    assert bitwise_equal(b, b.clone()) and not bitwise_equal(b, b + 0.0078125)


# ------------------------------------------------------- max-abs-normalised


def test_max_abs_normalised_bar():
    r = torch.tensor([10.0, -20.0, 5.0])
    assert max_abs_normalised(r + 0.19, r, 1e-2).passed          # 0.19 <= 0.2
    res = max_abs_normalised(r + torch.tensor([0.0, 0.0, 0.21]), r, 1e-2)
    assert not res.passed and res.error == pytest.approx(0.0105)
    assert max_abs_normalised(r.bfloat16(), r.bfloat16()).tol == 1e-2
    assert max_abs_normalised(r, r).tol == 1e-5
    assert not max_abs_normalised(r.half(), r).passed              # dtype change
    nan = torch.tensor([float("nan"), 1.0])
    assert max_abs_normalised(nan, nan).passed
    assert not max_abs_normalised(torch.tensor([1.0, 1.0]), nan).passed
    assert max_abs_normalised(torch.zeros(3), torch.zeros(3)).passed
    assert not max_abs_normalised(torch.ones(3), torch.zeros(3)).passed


def test_compare_evaluates_the_allowance_in_float32_like_the_reference():
    """A value on the tolerance boundary: float32 arithmetic (the reference's
    numeric.py:83-96) accepts it while exact arithmetic would reject it, so
    the comparison must follow float32 here."""
    import numpy as np

    r, c, rtol = 0.612636387348175, 0.6144742965698242, 0.003
    r32, c32 = np.float32(r), np.float32(c)
    assert np.abs(c32 - r32) - np.float32(rtol) * np.abs(r32) <= 0       # float32: within
    assert abs(float(c32) - float(r32)) - rtol * abs(float(r32)) > 0     # exact: outside
    res = numeric.compare(torch.tensor([c32]), torch.tensor([r32]), rtol, 0.0)
    assert res.passed, res
