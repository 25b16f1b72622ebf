"""The on-box peak kernels (include/mi_peaks.h) behind bench.py's `peaks`:
each runs, returns a checksum that depends on every value it touched, and the
measured rates are physically plausible for an MI355X (the reference keeps
the same kind of floor on its own readings, autotuner/measure/peaks.py:45-49)."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "metal-autotune_amd"))

pytestmark = pytest.mark.gpu


def test_read_kernel_folds_every_word():
    import measure

    L = measure.peak_lib()
    r = np.random.Generator(np.random.PCG64(41))
    host = r.integers(0, 2**32, size=(1 << 20) // 4 + 16, dtype=np.uint64).astype(np.uint32)
    src = torch.from_numpy(host.view(np.int32)).cuda()
    blocks = 37
    sink = torch.zeros(blocks, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    assert L.mi_peak_read(src.data_ptr(), host.nbytes, blocks, sink.data_ptr(), st) == 0
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(host)
    assert L.mi_peak_read(src.data_ptr(), 100, blocks, sink.data_ptr(), st) == 1  # not a multiple of 64


def test_mfma_kernel_sums_are_finite_and_deterministic():
    import measure

    L = measure.peak_lib()
    blocks = 8
    st = torch.cuda.current_stream().cuda_stream
    outs = []
    for _ in range(2):
        sink = torch.empty(blocks * 4, dtype=torch.float32, device="cuda")
        clk = torch.zeros(blocks * 8, dtype=torch.int64, device="cuda")
        assert L.mi_peak_mfma_bf16(blocks, 50, sink.data_ptr(), clk.data_ptr(), st) == 0
        torch.cuda.synchronize()
        assert torch.isfinite(sink).all()
        c = clk.view(-1, 2)
        assert (c > 0).all()
        outs.append(sink)
    assert torch.equal(outs[0], outs[1])


def test_measured_peaks_are_plausible():
    import measure

    p = measure.peaks()
    print("\npeaks:", p)
    assert 1500 < p["mfma_bf16"]["TF_s"] < 3000  # dense bf16, spec 2,500 TFLOP/s
    assert 0.8 < p["mfma_bf16"]["shader_clock_GHz_one_wave_per_simd"] < 3.0
    assert 3000 < p["hbm"]["read_GB_s"] < 9000  # spec 8,000 GB/s
    assert 0.1 < p["graph_launch"]["us"] < 20
