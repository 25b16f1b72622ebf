"""Output contract shared by parity tests, region checks and whole-model checks.

Same policy as the reference's numeric.py:1-122, on torch tensors:

* ``check(c, r, exact=True)`` is bitwise (shape, dtype, bytes);
* ``check(c, r, exact=False, rtol, atol)`` -> ``compare``: shape and dtype
  first; non-float outputs (indices, packed words) must match exactly
  whatever the tolerance; then the non-finite pattern (finite where finite,
  NaN where NaN, same signed inf where inf); then elementwise
  ``|c - r| <= max(atol + rtol*|r|, wobble_floor)`` in float32 with an
  overflow-safe excess, failing closed on a NaN error;
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
    finite_ok = torch.isfinite(r) & torch.isfinite(c)
    nan_ok = torch.isnan(r) & torch.isnan(c)
    inf_ok = torch.isinf(r) & (c == r)
    return finite_ok | nan_ok | inf_ok


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


def compare(candidate: torch.Tensor, reference: torch.Tensor, rtol: float, atol: float,
            wobble_floor: float = 0.0) -> CompareResult:
    validate_tolerances((rtol, atol))
    if tuple(candidate.shape) != tuple(reference.shape):
        return CompareResult(False, "shape", float("inf"), None,
                             f"{tuple(candidate.shape)} != {tuple(reference.shape)}")
    if candidate.dtype != reference.dtype:
        return CompareResult(False, "dtype", float("inf"), None,
                             f"{candidate.dtype} != {reference.dtype}")
    if candidate.numel() == 0:
        return CompareResult(True, "", 0.0, None)
    candidate = candidate.detach()
    reference = reference.detach().to(candidate.device)
    if reference.dtype not in FLOAT_DTYPES:
        # exact values: a float32 conversion could hide a one-unit change above 2**24
        diff = candidate != reference
        if bool(diff.any()):
            return CompareResult(False, "tolerance", float("inf"), _first(diff),
                                 "non-floating outputs must match exactly")
        return CompareResult(True, "", 0.0, None)
    c = candidate.float()
    r = reference.float()
    ok = nonfinite_pattern_ok(c, r)
    if not bool(ok.all()):
        viol = ~ok
        return CompareResult(False, "nonfinite_pattern", float("inf"), _first(viol),
                             f"{int(viol.sum())} elements break the non-finite pattern")
    finite = torch.isfinite(r)
    allowed = torch.clamp(atol + rtol * r.abs(), min=wobble_floor)
    excess = torch.where(finite, (c - r).abs() - allowed, torch.zeros_like(r))
    # opposite extreme values overflow the subtraction: recompute scaled
    scale = torch.clamp(torch.maximum(c.abs(), r.abs()), min=1.0)
    scaled = ((c / scale - r / scale).abs() - (atol / scale + rtol * (r / scale).abs())) * scale
    bad = finite & (torch.isnan(excess) | torch.isinf(excess))
    excess = torch.where(bad, scaled, excess)
    worst = _worst(excess)
    if math.isnan(worst):
        return CompareResult(False, "nonfinite_error", None, None,
                             "comparison produced a NaN error")
    index = _unravel(int(excess.reshape(-1).argmax()), tuple(r.shape))
    if worst > 0:
        over = int((excess > 0).sum())
        return CompareResult(False, "tolerance", worst, index, f"{over} elements over tolerance")
    return CompareResult(True, "", worst, index)


def check(candidate, reference, *, exact=True, rtol=0.0, atol=0.0) -> CompareResult:
    """Exact by default; tolerance is opt-in for floating evaluation changes."""
    if not exact:
        return compare(candidate, reference, rtol, atol)
    if tuple(candidate.shape) != tuple(reference.shape):
        return CompareResult(False, "shape", None, None, "output shape changed")
    if candidate.dtype != reference.dtype:
        return CompareResult(False, "dtype", None, None, "output dtype changed")
    if not bitwise_equal(candidate, reference.to(candidate.device)):
        return CompareResult(False, "exact", None, None,
                             "output must match the original bit-for-bit")
    return CompareResult(True, "", 0.0, None)


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
