"""Size-generic serving: which prompt lengths each region kernel is served at.

The reference's job records a scope at a few sizes, generalises the replay
over the size (bind/sized.py:1-20) and then serves each shipped kernel only
over the contiguous range of sizes where it was checked against its original
operations and timed against them (autotuner/serve.py:1-24, served_range at
serve.py:264-291).

Here the region wrappers already read the size from their input (they are
written against x.shape, not recorded at one size), so what remains is the
check and the range:

- ``check_sizes`` runs one region kernel (the others left on their original
  ops) against the unpatched layer at every requested size: outputs must be
  equal bit for bit, and both are timed with HIP events;
- ``served_range`` is the reference's rule for the served run around the
  primary size: contiguous correct sizes, extended on each side to the
  furthest size the kernel wins at, stopping at a grid size it does not win
  at and never past one it loses at;
- ``SizedRegions`` is the wrapper base: ``RANGES`` (kernel id -> runs of
  [lo, hi]) gates every ``try_sized`` call, outside the ranges the original
  ops run. ``None`` serves every size the spec's fallback predicate accepts.
"""

from __future__ import annotations

import itertools
import statistics

import torch

from . import kernels as _kernels
from .swap import ReplayWrapper

SIZE_NAME = "_n"


def runs(sizes) -> list[list[int]]:
    """Distinct sizes grouped into consecutive [first, last] runs, ascending.
    (Consecutive integers share n - rank, which is what groups them.)"""
    ordered = sorted({int(s) for s in sizes})
    return [[grp[0][1], grp[-1][1]]
            for _, grp in ((k, list(g)) for k, g in
                           itertools.groupby(enumerate(ordered), key=lambda t: t[1] - t[0]))]


def size_test(sizes, name: str = SIZE_NAME) -> str:
    """A Python expression over ``name`` that holds exactly for ``sizes``:
    an equality or a chained comparison for one run, else a membership test."""
    spans = runs(sizes)
    if not spans:
        return "False"
    if len(spans) > 1:
        members = tuple(n for lo, hi in spans for n in range(lo, hi + 1))
        return f"{name} in {members!r}"
    lo, hi = spans[0]
    return f"{name} == {lo}" if lo == hi else f"{lo} <= {name} <= {hi}"


def in_runs(n: int, ranges) -> bool:
    return any(lo <= n <= hi for lo, hi in ranges)


def served_range(correct, clock: dict, primary: int, grid=None):
    """The (lo, hi) of sizes a kernel is served at around ``primary``, or
    None when ``primary`` is itself not servable.

    Servable sizes are the correct ones that were not timed as a loss. From
    the contiguous servable run around the primary, each side keeps the
    sizes out to its furthest timed win that lies before the first ``grid``
    size on that side it does not win at. ``clock`` maps timed sizes to
    {"win": bool, "loss": bool}; ``grid`` defaults to every timed size, and a
    timed size outside it that does not win is ignored. The primary counts as
    a win."""
    grid = set(clock) if grid is None else set(grid)
    lost = {n for n, t in clock.items() if t.get("loss")}
    servable = set(correct) - lost
    if primary not in servable:
        return None
    lo = hi = primary
    while lo - 1 in servable:
        lo -= 1
    while hi + 1 in servable:
        hi += 1
    won = {n for n, t in clock.items() if t.get("win")}
    blocked = {n for n in clock if n in grid and n not in won}

    def reach(side: int) -> int:
        inside = (lambda n: primary < n <= hi) if side > 0 else (lambda n: lo <= n < primary)
        dist = lambda n: (n - primary) * side  # noqa: E731
        stop = min((dist(n) for n in blocked if inside(n)), default=None)
        ok = [n for n in won if inside(n) and (stop is None or dist(n) < stop)]
        return max(ok, key=dist, default=primary)

    return reach(-1), reach(+1)


class SizedRegions(ReplayWrapper):
    """Region-wrapper base: ``self._try(role, inputs, n)`` launches the role's
    spec through ``try_sized`` when its kernel serves size ``n`` (the
    ``RANGES`` table, class- or instance-level), else returns None so the
    caller runs the original ops."""

    RANGES: dict | None = None

    def _try(self, role: str, inputs, n: int):
        spec = self._specs.get(role)
        if spec is None:
            return None
        return self._try_spec(spec, inputs, n)

    def _try_spec(self, spec, inputs, n: int):
        ranges = self.__dict__.get("_ranges", type(self).RANGES)
        if ranges is not None and not in_runs(n, ranges.get(spec.kernel_id, ())):
            return None
        return _kernels.try_sized(spec, inputs)

    def _serves(self, role: str, inputs, n: int) -> bool:
        """Whether ``self._try(role, inputs, n)`` would launch the role's kernel
        (for a caller that runs a fused form of the same cut in its place)."""
        spec = self._specs.get(role)
        if spec is None:
            return False
        ranges = self.__dict__.get("_ranges", type(self).RANGES)
        if ranges is not None and not in_runs(n, ranges.get(spec.kernel_id, ())):
            return False
        return _kernels.covers_sized(spec, inputs)

    def set_ranges(self, ranges: dict | None) -> None:
        object.__setattr__(self, "_ranges", ranges)


# ---------------------------------------------------------------------------
# checking and timing one kernel at many sizes


def _time_ms(fn, reps: int) -> float:
    times = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1))
    return statistics.median(times)


def check_sizes(original, make_wrapper, role_specs: dict, sizes, make_call, *, timed=None,
                reps: int = 5, margin: float = 0.03) -> dict:
    """For each kernel (role -> spec): the wrapper built with only that role's
    spec (``make_wrapper(specs)``) against ``original``, both called as
    ``make_call(module, n)`` (which builds fresh inputs/state for size n and
    returns the outputs). Every size of ``sizes`` is checked bit for bit (a
    served range is a run of consecutive checked sizes); the sizes of
    ``timed`` (default: all) are also timed. Returns kernel id ->
    {"correct": [n...], "clock": {n: {"win", "loss", "ms_kernel",
    "ms_original"}}}. A win is at least ``margin`` faster, a loss at least
    ``margin`` slower."""
    timed = list(sizes) if timed is None else list(timed)
    out = {}
    for role, spec in role_specs.items():
        wrapper = make_wrapper({role: spec})
        correct, clock = [], {}
        for n in sorted(set(sizes) | set(timed)):
            want = make_call(original, n)
            got = make_call(wrapper, n)
            torch.cuda.synchronize()
            same = all(torch.equal(a, b) for a, b in zip(_flat(want), _flat(got)))
            if same:
                correct.append(n)
            if n not in timed:
                continue
            t_o = _time_ms(lambda: make_call(original, n), reps)
            t_k = _time_ms(lambda: make_call(wrapper, n), reps)
            clock[n] = {"win": t_k <= t_o * (1 - margin), "loss": t_k >= t_o * (1 + margin),
                        "ms_kernel": t_k, "ms_original": t_o}
        out[spec.kernel_id] = {"correct": correct, "clock": clock}
    return out


def _flat(tree):
    if isinstance(tree, torch.Tensor):
        return [tree]
    if isinstance(tree, (list, tuple)):
        return [t for item in tree for t in _flat(item)]
    return []


def plan_ranges(results: dict, primary: int, grid=None) -> dict:
    """kernel id -> [[lo, hi]] from check_sizes results (kernels whose
    primary size fails are served nowhere: an empty list)."""
    out = {}
    for kid, r in results.items():
        rng = served_range(r["correct"], r["clock"], primary, grid)
        out[kid] = [] if rng is None else [list(rng)]
    return out
