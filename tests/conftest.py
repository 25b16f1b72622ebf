"""Shared test setup: import paths, the `gpu` marker, tensor helpers.

Tests marked ``gpu`` need an MI355X and the built HIP library; they call the
kernels through the C ABI (autotuner_runtime.hip) and compare with the CPU
oracle (oracle/). Everything else runs on the CPU.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "metal-autotune_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def oracle_lib():
    """The C oracle, built on demand (test infrastructure)."""
    import oracle

    so = ROOT / "oracle" / "liboracle.so"
    if not so.exists():
        import subprocess
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    return oracle.lib()


def to_torch(a: np.ndarray, dtype: str, device: str = "cuda"):
    """float32 values representable in `dtype` -> torch tensor of that dtype."""
    import torch

    tdt = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}[dtype]
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device=device, dtype=tdt)


def to_np(t) -> np.ndarray:
    import torch

    return t.detach().to(device="cpu", dtype=torch.float32).numpy()


def packed_to_torch(wq: np.ndarray, device: str = "cuda"):
    import torch

    return torch.from_numpy(np.ascontiguousarray(wq, dtype=np.uint32)).to(device)


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))
