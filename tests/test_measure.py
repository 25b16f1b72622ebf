"""The benchmark's clock statistics (metal-autotune_amd/measure.py), on the CPU:
the median/spread summary and the paired ABBA/BAAB reduction follow the
reference's clocks (autotuner/measure/clocks.py:217-287) and stats
(autotuner_runtime/stats.py:12, 91-130)."""

from __future__ import annotations

import math
import statistics
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "metal-autotune_amd"))

import measure  # noqa: E402


def test_summary_is_the_median_with_the_median_standard_error():
    xs = [10.0, 12.0, 11.0, 30.0, 9.0, 10.5, 11.5, 10.0, 12.5]  # one outlier
    s = measure.summarize(xs, per=2)
    assert s["median"] == pytest.approx(statistics.median(xs) / 2)
    assert s["min"] == 4.5 and s["max"] == 15.0 and s["n"] == 9
    sd = statistics.stdev([x / 2 for x in xs])
    assert s["se"] == pytest.approx(1.2533 * sd / 3.0)


def test_compare_pairs_abba_blocks_and_reports_the_median_ratio(monkeypatch):
    """An arm twice as fast under a linear drift: the block pairing cancels the
    drift, so every observation's ratio is the same and the agreement is 1."""
    t = {"now": 0.0}

    def fake_time(fn, reps):
        t["now"] += 1.0
        return reps * fn(t["now"])  # ms for reps calls

    drift = lambda now: 1.0 + 0.01 * now
    base = lambda now=0.0: 2.0 * drift(now)
    cand = lambda now=0.0: 1.0 * drift(now)
    monkeypatch.setattr(measure, "_time", lambda fn, reps: fake_time(fn, reps))
    monkeypatch.setattr(measure, "reps_for", lambda fn, target_ms=20.0: 3)
    r = measure.compare(base, cand, pairs=8)
    assert r["observations"] == 4
    # ABBA: a at t, t+3; b at t+1, t+2 -> equal midpoints, ratio exactly 1/2
    assert r["median_ratio"] == pytest.approx(0.5)
    assert r["median_delta_ms"] > 0
    assert r["stability"] == pytest.approx(1.0)
    with pytest.raises(ValueError):
        measure.compare(base, cand, pairs=3)
