"""The allocation-free argmax (mi_argmax_noalloc) against mi_argmax through
the C ABI: equal indices on back-to-back calls (the second smaller, so stale
partials of the first would show), over bf16 / fp32, vectorised and scalar
rows, ties and NaN; an over-size request is refused before any launch."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import rng

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from autotuner_runtime import hip  # noqa: E402


def _with_workspace(x: torch.Tensor) -> torch.Tensor:
    L = hip.lib()
    V = x.shape[-1]
    rows = x.numel() // V
    out = torch.full((rows,), -7, dtype=torch.int32, device=x.device)
    nbytes = int(L.mi_argmax_workspace_bytes(rows, V))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    st = torch.cuda.current_stream().cuda_stream
    assert L.mi_argmax(x.data_ptr(), out.data_ptr(), rows, V, hip._dt(x), ws.data_ptr(), nbytes,
                       st) == 0
    return out


def _no_alloc(x: torch.Tensor) -> torch.Tensor:
    L = hip.lib()
    V = x.shape[-1]
    rows = x.numel() // V
    out = torch.full((rows,), -7, dtype=torch.int32, device=x.device)
    st = torch.cuda.current_stream().cuda_stream
    status = L.mi_argmax_noalloc(x.data_ptr(), out.data_ptr(), rows, V, hip._dt(x), st)
    assert status == 0, L.mi_last_error()
    return out


def _logits(seed, rows, V, dtype):
    x = oracle.round_to(rng(seed).normal(0, 1, (rows, V)), dtype)
    x[0, V // 3] = x[0, V - 1] = 40.0          # a tie across spans: the lower index wins
    if rows > 1:
        x[1, : min(V, 4096)] = np.nan          # NaN never wins
    tdt = torch.bfloat16 if dtype == "bfloat16" else torch.float32
    return torch.from_numpy(x).to(device="cuda", dtype=tdt)


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_noalloc_equals_workspace_argmax_on_back_to_back_calls(dtype):
    cases = [(1, 200, 151936), (2, 3, 2049)]     # the second call smaller than the first
    if dtype == "float32":
        cases = [(3, 100, 151936), (4, 2, 4097)]
    for seed, rows, V in cases:
        x = _logits(seed, rows, V, dtype)
        got = _no_alloc(x)
        want = _with_workspace(x)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (dtype, rows, V)
        assert int(got[0]) == V // 3
        ref = np.nanargmax(np.where(np.isnan(x.float().cpu().numpy()), -np.inf,
                                    x.float().cpu().numpy()), axis=1)
        assert np.array_equal(got.cpu().numpy(), ref), (dtype, rows, V)


def test_noalloc_scalar_rows_and_repeat():
    """Rows one element off 16-byte alignment take the scalar span path."""
    base = _logits(5, 8, 3001, "bfloat16")
    flat = torch.cat([torch.zeros(1, dtype=base.dtype, device="cuda"), base.reshape(-1)])
    x = flat[1:].reshape(8, 3001)
    for _ in range(2):
        got = _no_alloc(x)
        torch.cuda.synchronize()
        assert torch.equal(got, _with_workspace(x))


def test_noalloc_refuses_more_partials_than_its_scratch():
    L = hip.lib()
    x = torch.zeros((216, 151936), dtype=torch.bfloat16, device="cuda")
    out = torch.zeros(216, dtype=torch.int32, device="cuda")
    status = L.mi_argmax_noalloc(x.data_ptr(), out.data_ptr(), 216, 151936, hip.MI_BF16,
                                 torch.cuda.current_stream().cuda_stream)
    assert status == hip.MI_ERR_ARG
    assert b"scratch" in L.mi_last_error()
    # 215 rows fit
    assert _no_alloc(x[:215]).shape == (215,)
