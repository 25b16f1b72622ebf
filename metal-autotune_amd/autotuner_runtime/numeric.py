"""Output contract shared by parity tests, region checks and whole-model checks.

Same policy as the reference's numeric.py:1-122, on torch tensors:

* ``check(c, r, exact=True)`` is bitwise (shape, dtype, bytes);
* ``check(c, r, exact=False, rtol, atol)`` -> ``compare``: shape and dtype
  first; non-float outputs (indices, packed words) must match exactly
  whatever the tolerance; then the non-finite pattern (finite where finite,
  NaN where NaN, same signed inf where inf); then elementwise
  ``|c - r| <= max(atol + rtol*|r|, wobble_floor)``, evaluated in float32
  as the reference does (numeric.py:83-96), an overflowing difference
  re-evaluated on both sides scaled by max(|c|, |r|, 1), failing closed on
  a NaN error;
* ``tolerance_for(dtype)`` gives the per-dtype defaults
  (fp32 (1e-5, 1e-6), fp16 (1e-2, 2e-2), bf16 (2e-2, 4e-2)).

``max_abs_normalised`` is the criterion the port's spec states for region
outputs: ``max|c - r| <= tol * max|r|`` with tol 1e-5 for fp32 and 1e-2 for
bf16/fp16 (BASELINE_TOLERANCES); the closest reference form is the
``atol + rtol * max|ref|`` allowance of artifact/validate.py:207-209.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from types import MappingProxyType

import torch

from .exact import bitwise_equal

FLOAT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
MAX_TOLERANCE = float.fromhex("0x1.fffffep+127")  # largest finite float32
DEFAULT_TOLERANCES = MappingProxyType({
    "float32": (1e-5, 1e-6),
    "float16": (1e-2, 2e-2),
    "bfloat16": (2e-2, 4e-2),
})
# max-abs-normalised tolerance per dtype (the port's region criterion)
BASELINE_TOLERANCES = MappingProxyType({"float32": 1e-5, "float16": 1e-2, "bfloat16": 1e-2})


def dtype_name(dtype) -> str:
    return str(dtype).replace("torch.", "")


def validate_tolerances(values) -> None:
    if len(values) != 2 or any(isinstance(v, bool) or not isinstance(v, (int, float))
                               or not math.isfinite(v) or v < 0 for v in values):
        raise ValueError("tolerances must be two finite non-negative numbers (rtol, atol)")
    if any(v > MAX_TOLERANCE for v in values):
        raise ValueError("tolerances must fit in float32, the comparison dtype")


def tolerance_for(dtype, override=None):
    if override is not None:
        validate_tolerances(override)
        return tuple(override)
    return DEFAULT_TOLERANCES.get(dtype_name(dtype), (0.0, 0.0))


@dataclass(frozen=True)
class CompareResult:
    passed: bool
    reason: str                    # "" | shape | dtype | exact | nonfinite_pattern | tolerance | nonfinite_error
    max_excess: float | None       # worst excess when meaningful; None for exact mismatches
    index: tuple | None            # the worst offender (or first pattern violation)
    detail: str = ""


def nonfinite_pattern_ok(c: torch.Tensor, r: torch.Tensor) -> torch.Tensor:
    """Per element: where the reference is finite the candidate must be
    finite, where it is NaN the candidate must be NaN, and where it is an
    infinity the candidate must be that same infinity."""
    return torch.where(torch.isfinite(r), torch.isfinite(c),
                       torch.where(torch.isnan(r), torch.isnan(c), c == r))


def _unravel(flat: int, shape: tuple) -> tuple:
    out = []
    for dim in reversed(shape):
        flat, rem = divmod(flat, dim)
        out.append(rem)
    return tuple(reversed(out))


def _first(mask: torch.Tensor) -> tuple:
    flat = mask.reshape(-1).nonzero()
    return _unravel(int(flat[0, 0]), tuple(mask.shape)) if flat.numel() else ()


def _worst(excess: torch.Tensor) -> float:
    """The largest excess (a separate function so a test can force a NaN here)."""
    return float(excess.max())


def _same_structure(candidate, reference, distance) -> CompareResult | None:
    """A failed result when shape or dtype differ, else None."""
    cs, rs = tuple(candidate.shape), tuple(reference.shape)
    if cs != rs:
        return CompareResult(False, "shape", distance, None, f"shape {cs} != {rs}")
    if candidate.dtype != reference.dtype:
        return CompareResult(False, "dtype", distance, None,
                             f"dtype {candidate.dtype} != {reference.dtype}")
    return None


def compare(candidate: torch.Tensor, reference: torch.Tensor, rtol: float, atol: float,
            wobble_floor: float = 0.0) -> CompareResult:
    """Tolerance comparison: per element |c - r| <= max(atol + rtol*|r|,
    wobble_floor) after the non-finite pattern rule.

    Both sides and the allowance are float32, so a value at the boundary
    passes or fails exactly as in the reference (numeric.py:83-96). Where the
    float32 excess is NaN (an overflowing difference against an infinite
    allowance) it is taken again with both sides divided by max(|c|, |r|, 1):
    3e38 against -3e38 stays a failure instead of an accidental pass. Integer
    and boolean outputs must be equal whatever the tolerance."""
    validate_tolerances((rtol, atol))
    bad = _same_structure(candidate, reference, float("inf"))
    if bad is not None:
        return bad
    if candidate.numel() == 0:
        return CompareResult(True, "", 0.0, None)
    cand = candidate.detach()
    ref = reference.detach().to(cand.device)
    if ref.dtype not in FLOAT_DTYPES:
        differs = cand != ref
        if bool(differs.any()):
            return CompareResult(False, "tolerance", float("inf"), _first(differs),
                                 "integer/boolean outputs must be equal; tolerances do not apply")
        return CompareResult(True, "", 0.0, None)
    c = cand.to(torch.float32)
    r = ref.to(torch.float32)
    broken = ~nonfinite_pattern_ok(c, r)
    if bool(broken.any()):
        return CompareResult(False, "nonfinite_pattern", float("inf"), _first(broken),
                             f"{int(broken.sum())} elements break the non-finite pattern")
    finite = torch.isfinite(r)

    def f32(v):
        return torch.tensor(v, dtype=torch.float32, device=r.device)

    budget = torch.maximum(f32(atol) + f32(rtol) * r.abs(), f32(wobble_floor))
    excess = torch.where(finite, (c - r).abs() - budget, torch.zeros_like(r))
    scale = torch.clamp(torch.maximum(c.abs(), r.abs()), min=1.0)
    scaled = (c / scale - r / scale).abs() - (f32(atol) / scale + f32(rtol) * (r / scale).abs())
    excess = torch.where(finite & torch.isnan(excess), scaled * scale, excess)
    worst = _worst(excess)
    if math.isnan(worst):
        return CompareResult(False, "nonfinite_error", None, None,
                             "the comparison itself produced a NaN")
    index = _unravel(int(excess.reshape(-1).argmax()), tuple(r.shape))
    if worst > 0:
        return CompareResult(False, "tolerance", worst, index,
                             f"{int((excess > 0).sum())} elements over tolerance")
    return CompareResult(True, "", worst, index)


def check(candidate, reference, *, exact=True, rtol=0.0, atol=0.0) -> CompareResult:
    """The verdict for one output: bit for bit unless ``exact=False``, which
    applies ``compare`` with (rtol, atol)."""
    if not exact:
        return compare(candidate, reference, rtol, atol)
    bad = _same_structure(candidate, reference, None)
    if bad is not None:
        return bad
    if bitwise_equal(candidate, reference.to(candidate.device)):
        return CompareResult(True, "", 0.0, None)
    return CompareResult(False, "exact", None, None, "bits differ from the original output")


@dataclass(frozen=True)
class NormalisedResult:
    passed: bool
    error: float        # max|c - r| / max|r|
    tol: float
    detail: str = ""


def max_abs_normalised(candidate: torch.Tensor, reference: torch.Tensor,
                       tol: float | None = None) -> NormalisedResult:
    """max|c - r| <= tol * max|r|, after the shape/dtype/non-finite rules."""
    tol = BASELINE_TOLERANCES.get(dtype_name(reference.dtype), 0.0) if tol is None else tol
    if tuple(candidate.shape) != tuple(reference.shape) or candidate.dtype != reference.dtype:
        return NormalisedResult(False, float("inf"), tol, "shape or dtype changed")
    if candidate.numel() == 0:
        return NormalisedResult(True, 0.0, tol)
    c = candidate.detach().float()
    r = reference.detach().to(c.device).float()
    if not bool(nonfinite_pattern_ok(c, r).all()):
        return NormalisedResult(False, float("inf"), tol, "non-finite pattern differs")
    f = torch.isfinite(r)
    denom = float(r[f].abs().max()) if bool(f.any()) else 0.0
    err = float((c[f] - r[f]).abs().max()) if bool(f.any()) else 0.0
    rel = err / denom if denom > 0 else (0.0 if err == 0 else float("inf"))
    return NormalisedResult(rel <= tol, rel, tol, f"max abs err {err:.3e}, max |ref| {denom:.3e}")
