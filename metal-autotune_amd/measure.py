"""Clocks and peaks for the MI355X benchmark figures.

The reference never reports one timed window or a spec-sheet peak:

- a figure is the median of >= 9 samples, each a loop holding >= 20 ms of
  work so the fixed submit-and-sync cost is a rounding error
  (autotuner/measure/clocks.py:30 CLOCK_TARGET_MS, :217-231 step_clock);
- two arms are compared in alternating ABBA / BAAB blocks, each block's two
  samples of an arm averaged into one observation, and the comparison is the
  median ratio with its standard error and a 0..1 agreement score
  (clocks.py:234-287, autotuner_runtime/stats.py:1-20, 91-130);
- peaks are microbenchmarked on the device, and the best reading is the peak,
  since throttling and contention only push readings down
  (autotuner/measure/peaks.py:1-7, 34-42).

This module does the same on HIP: every sample is timed with HIP events on
the stream the work runs on, around graph replays or launches that are
already enqueued-ready (nothing is allocated or compiled inside a sample).
The peak kernels are the library's mi_peak_* entries (include/mi_peaks.h).
"""

from __future__ import annotations

import ctypes
import math
import statistics
from typing import Callable

import torch

from autotuner_runtime import hip

CLOCK_TARGET_MS = 20.0   # work per sample (clocks.py:30)
SAMPLES = 9              # samples per figure (clocks.py:217 reps=9)
MEDIAN_SE_FACTOR = 1.2533  # SE(median) ~ 1.2533 sigma / sqrt(n) for normal noise (stats.py:12)
MAX_REPS = 20000


def _events():
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def _time(once: Callable[[], object], reps: int) -> float:
    """ms for `reps` back-to-back calls of once(), HIP events on the current stream."""
    e0, e1 = _events()
    e0.record()
    for _ in range(reps):
        once()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1)


def reps_for(once: Callable[[], object], target_ms: float = CLOCK_TARGET_MS) -> int:
    """How many calls one sample needs to hold target_ms of work (sized from a
    10-call estimate after a warm call)."""
    once()
    torch.cuda.synchronize()
    est = _time(once, 10) / 10
    return max(1, min(MAX_REPS, math.ceil(target_ms / max(est, 1e-6))))


def summarize(samples_ms: list[float], per: int = 1) -> dict:
    """Median and spread of per-call times (each sample divided by `per`)."""
    xs = [s / per for s in samples_ms]
    med = statistics.median(xs)
    sd = statistics.stdev(xs) if len(xs) > 1 else 0.0
    q = statistics.quantiles(xs, n=4) if len(xs) >= 4 else [med, med, med]
    return {"median": med, "min": min(xs), "max": max(xs), "n": len(xs),
            "se": MEDIAN_SE_FACTOR * sd / math.sqrt(len(xs)),
            "iqr_rel": (q[2] - q[0]) / med if med > 0 else 0.0}


def clock(once: Callable[[], object], per_call: int = 1, samples: int = SAMPLES,
          target_ms: float = CLOCK_TARGET_MS) -> dict:
    """The per-unit time of once() (which runs `per_call` units): median of
    `samples` samples of >= target_ms each, in ms, with the spread."""
    reps = reps_for(once, target_ms)
    for _ in range(2):  # warm until the clock holds
        _time(once, reps)
    raw = [_time(once, reps) for _ in range(samples)]
    out = summarize(raw, per=reps * per_call)
    out["calls_per_sample"] = reps
    out["sample_ms"] = round(statistics.median(raw), 3)
    return out


def compare(base: Callable[[], object], cand: Callable[[], object], pairs: int = 16,
            target_ms: float = CLOCK_TARGET_MS) -> dict:
    """Paired interleaved A/B: ABBA then BAAB blocks (clocks.py:234-287). Each
    block's two samples of an arm average into one observation; the result is
    the median per-observation ratio cand/base (< 1: the candidate is faster),
    the median delta base - cand (> 0: faster) with its standard error, and
    the agreement score median / (median + IQR) of the ratios (stats.py:91-110)."""
    if pairs < 2 or pairs % 2:
        raise ValueError("pairs must be even and >= 2")
    reps = max(reps_for(base, target_ms), reps_for(cand, target_ms))
    _time(base, reps)
    _time(cand, reps)
    a, b = [], []
    for block in range(pairs // 2):
        order = "abba" if block % 2 == 0 else "baab"
        for arm in order:
            (a if arm == "a" else b).append(_time(base if arm == "a" else cand, reps) / reps)
    pa = [(a[i] + a[i + 1]) / 2 for i in range(0, len(a), 2)]
    pb = [(b[i] + b[i + 1]) / 2 for i in range(0, len(b), 2)]
    deltas = [x - y for x, y in zip(pa, pb)]
    ratios = [y / x for x, y in zip(pa, pb)]
    mr = statistics.median(ratios)
    q = statistics.quantiles(ratios, n=4) if len(ratios) >= 4 else [mr, mr, mr]
    sd = statistics.stdev(deltas) if len(deltas) > 1 else float("inf")
    return {"median_base_ms": statistics.median(pa), "median_cand_ms": statistics.median(pb),
            "median_ratio": mr, "median_delta_ms": statistics.median(deltas),
            "se_delta_ms": MEDIAN_SE_FACTOR * sd / math.sqrt(len(deltas)),
            "stability": mr / (mr + (q[2] - q[0])) if mr > 0 else 0.0,
            "observations": len(deltas), "calls_per_sample": reps}


# ---------------------------------------------------------------------------
# peaks

_peak_lib = None


def peak_lib():
    """libmiqmm.so with the mi_peak_* argument types set."""
    global _peak_lib
    if _peak_lib is None:
        L = hip.lib()
        P, I, I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        L.mi_peak_mfma_bf16.argtypes = [I, I, P, P, P]
        L.mi_peak_read.argtypes = [P, I64, I, P, P]
        L.mi_peak_empty.argtypes = [P]
        for f in (L.mi_peak_mfma_bf16, L.mi_peak_read, L.mi_peak_empty):
            f.restype = ctypes.c_int
        _peak_lib = L
    return _peak_lib


PEAK_SYMBOLS = ("mi_peak_mfma_bf16", "mi_peak_read", "mi_peak_empty")


def _ok(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what}: {hip.lib().mi_last_error().decode(errors='replace')}")


def cus() -> int:
    return torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count


def peak_mfma(samples: int = 5) -> dict:
    """Dense bf16 MFMA rate, best over 1-3 workgroups (4-12 waves) per CU, and
    the shader clock the one-wave-per-SIMD run held (s_memtime over the
    100 MHz s_memrealtime)."""
    L = peak_lib()
    n = cus()
    stream = torch.cuda.current_stream().cuda_stream
    best, per_cfg, ghz = 0.0, {}, None
    for w in (1, 2, 3):
        blocks = n * w
        sink = torch.empty(blocks * 4, dtype=torch.float32, device="cuda")
        clk = torch.zeros(blocks * 8, dtype=torch.int64, device="cuda")
        iters = 64
        run = lambda: _ok(L.mi_peak_mfma_bf16(blocks, iters, sink.data_ptr(), clk.data_ptr(), stream),
                          "peak_mfma")
        # size iters so one launch is ~20 ms
        t = _time(run, 1)
        iters = max(64, int(iters * CLOCK_TARGET_MS / max(_time(run, 1), 1e-3)))
        ms = min(_time(run, 1) for _ in range(samples))
        fl = blocks * 4 * iters * 16 * 32768.0
        tf = fl / (ms * 1e-3) / 1e12
        per_cfg[f"{4 * w}_waves_per_cu"] = round(tf, 1)
        best = max(best, tf)
        if w == 1:
            c = clk.view(-1, 2).double()
            ghz = float((c[:, 0].sum() / c[:, 1].sum()) * 0.1)  # ticks per 10 ns -> GHz
        del t
    return {"TF_s": round(best, 1), "by_occupancy": per_cfg,
            "shader_clock_GHz_one_wave_per_simd": round(ghz, 3) if ghz else None,
            "method": "v_mfma_f32_32x32x16_bf16 x 16 per iteration over 4 independent "
                      "accumulators, every CU, one launch of ~20 ms, best of "
                      f"{samples}"}


def peak_read(gib: float = 2.0, samples: int = 5) -> dict:
    """HBM read rate over a buffer far larger than the 256 MB Infinity Cache."""
    L = peak_lib()
    nbytes = int(gib * (1 << 30))
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    src.fill_(1)
    blocks = cus() * 32
    sink = torch.empty(blocks, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    run = lambda: _ok(L.mi_peak_read(src.data_ptr(), nbytes, blocks, sink.data_ptr(), stream),
                      "peak_read")
    reps = reps_for(run)
    ms = min(_time(run, reps) / reps for _ in range(samples))
    # a device-to-device copy of the same buffer (read + write bytes)
    dst = torch.empty_like(src)
    cp = lambda: dst.copy_(src)
    creps = reps_for(cp)
    cms = min(_time(cp, creps) / creps for _ in range(samples))
    del src, dst
    torch.cuda.empty_cache()
    return {"read_GB_s": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "copy_GB_s": round(2 * nbytes / (cms * 1e-3) / 1e9, 1),
            "method": f"{gib:g} GiB read by mi_peak_read ({blocks} workgroups) and copied by "
                      f"torch, loops of >= {CLOCK_TARGET_MS:g} ms, best of {samples}"}


def launch_floor(chain: int = 256, samples: int = 9) -> dict:
    """Per-launch cost of an empty kernel inside a HIP graph of `chain`
    launches (peaks.py LAUNCH_CHAIN), the floor every kernel of a graph pays."""
    L = peak_lib()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        _ok(L.mi_peak_empty(s.cuda_stream), "peak_empty")
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        st = torch.cuda.current_stream().cuda_stream
        for _ in range(chain):
            _ok(L.mi_peak_empty(st), "peak_empty")
    torch.cuda.synchronize()
    c = clock(g.replay, per_call=chain, samples=samples)
    return {"us": round(c["median"] * 1000.0, 3), "min_us": round(c["min"] * 1000.0, 3),
            "method": f"median of {samples} samples of graph replays of {chain} empty launches"}


def peaks() -> dict:
    """Every on-box peak the benchmark reports."""
    out = {"mfma_bf16": peak_mfma(), "hbm": peak_read(), "graph_launch": launch_floor()}
    torch.cuda.synchronize()
    return out
