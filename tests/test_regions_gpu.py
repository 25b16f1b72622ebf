"""The reference's verification gates on every region spec, on the GPU.

The reference's correctness child launches each candidate with NaN-poisoned
outputs (autotuner/ladder/child.py:10-13,174) and requires three re-poisoned
runs to be bitwise identical (child.py:419-428). Here every region spec of
autotuner_runtime.regions runs through ``kernels.call(spec, inputs,
init_value=nan)`` three times at a ragged shape (N = 200, rows that do not
fill a tile) and at the model shapes that take the mixed tile grids (the
M = 100 / 128 dual at N = 9728, q/k/v at 4096 + 1024 + 1024, a single qmm at
N = 5120): no NaN may survive (a skipped tile would leave one), the three runs
must be equal bit for bit, and the result must match the oracle composition of
the region (max-abs-normalised 1e-2 for bf16, 1e-5 for fp32; dequant exact).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import packed_to_torch, rng, to_np, to_torch

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from autotuner_runtime import kernels, regions  # noqa: E402

BF = "bfloat16"


def _quant(seed, N, K, bits=4, gs=64):
    r = rng(seed)
    return oracle.quantize_affine(r.normal(0, 0.02, (N, K)).astype(np.float32), gs, bits, BF)


def _dev(q):
    wq, s, b = q
    return [packed_to_torch(wq), to_torch(s, BF), to_torch(b, BF)]


def _x(seed, shape, scale=1.0):
    return oracle.round_to(rng(seed).normal(0, scale, shape), BF)


def _qmm(x, q, bits=4):
    return oracle.qmm_factored(x, *q, 64, bits, BF)


def _gates(spec, ins, wants, tol=1e-2):
    """Three NaN-poisoned runs: no NaN left, bitwise identical, close to the
    oracle (tol None: exact). A want may be a (array, tol) pair of its own."""
    runs = [kernels.call(spec, ins, init_value=float("nan")) for _ in range(3)]
    torch.cuda.synchronize()
    assert len(runs[0]) == len(wants)
    for j, want in enumerate(wants):
        want, bar = want if isinstance(want, tuple) else (want, tol)
        first = runs[0][j]
        assert not torch.isnan(first).any(), f"{spec.kernel_id} output {j}: unwritten elements"
        for r in runs[1:]:
            assert torch.equal(first, r[j]), f"{spec.kernel_id} output {j}: runs differ"
        got = to_np(first).astype(np.float64)
        if bar is None:
            assert np.array_equal(got, want), f"{spec.kernel_id} output {j}: not exact"
        else:
            err = np.abs(got - want).max() / max(np.abs(want).max(), 1e-30)
            assert err <= bar, f"{spec.kernel_id} output {j}: error {err:.3e} > {bar}"


# (M, N, K): ragged N = 200 at GEMV, generic and MFMA row counts; the mixed
# 64/32-token grid of a single part (N = 5120, M = 100 and 128)
QMM_SHAPES = [(1, 200, 512), (7, 200, 512), (100, 200, 512), (100, 5120, 2560),
              (128, 5120, 2560)]


@pytest.mark.parametrize("M,N,K", QMM_SHAPES)
def test_qmm_region(M, N, K):
    q = _quant(2000 + N, N, K)
    x = _x(2001 + M, (1, M, K))
    ins = [to_torch(x, BF)] + _dev(q)
    _gates(regions.qmm(), ins, [_qmm(x, q)])


@pytest.mark.parametrize("M,N,K", [(100, 200, 512), (100, 9728, 2560), (128, 9728, 2560)])
def test_dual_regions(M, N, K):
    """[qmm(w1), qmm(w3)] and its SwiGLU-fused form; N = 9728 at M = 100/128
    takes the mixed 128/64-token grid."""
    q1, q3 = _quant(2010, N, K), _quant(2011, N, K)
    x = _x(2012 + M, (1, M, K))
    ins = [to_torch(x, BF)] + _dev(q1) + _dev(q3)
    g, u = _qmm(x, q1), _qmm(x, q3)
    _gates(regions.dual(), ins, [g, u])
    _gates(regions.dual_swiglu(), ins, [oracle.swiglu(g, u, BF)])


@pytest.mark.parametrize("M,Ns,K", [(100, (224, 96, 32), 512), (100, (4096, 1024, 1024), 2560),
                                    (128, (4096, 1024, 1024), 2560)])
def test_grouped3_region(M, Ns, K):
    qs = [_quant(2020 + i, n, K) for i, n in enumerate(Ns)]
    x = _x(2023 + M, (1, M, K))
    ins = [to_torch(x, BF)] + [t for q in qs for t in _dev(q)]
    _gates(regions.grouped3(), ins, [_qmm(x, q) for q in qs])


@pytest.mark.parametrize("M,D,K", [(100, 200, 512), (128, 2048, 2048)])
def test_split_gate_region(M, D, K):
    """(C, B*x). B*x is the product of two rounded projections, so a one-ulp
    rounding difference in each operand can add up to about three ulps of the
    product: it is checked as the exact T(B * x) of the GPU's own unfused
    projection, whose three parts are each held to the 1e-2 bar."""
    q = _quant(2030, 3 * D, K)
    x = _x(2031 + M, (1, M, K))
    (y3,) = kernels.call(regions.qmm(), [to_torch(x, BF)] + _dev(q))
    y3 = to_np(y3).astype(np.float64)
    want = _qmm(x, q)
    err = np.abs(y3 - want).max() / np.abs(want).max()
    assert err <= 1e-2, f"unfused in_proj error {err:.3e}"
    c, bx = oracle.split_gate(y3, BF)
    c_o, _ = oracle.split_gate(want, BF)
    _gates(regions.split_gate(), [to_torch(x, BF)] + _dev(q), [(c, None), (bx, None)])
    _gates(regions.split_gate(), [to_torch(x, BF)] + _dev(q), [c_o, (bx, None)])


@pytest.mark.parametrize("M,N,K", [(100, 200, 512), (128, 2560, 4096), (128, 2560, 9728),
                                   (7, 200, 512)])
def test_residual_regions(M, N, K):
    """[qmm, add] and [qmm, add, rms_norm] (o_proj / down_proj shapes: K parts
    run as workgroups of their own, then a kernel adds them)."""
    q = _quant(2040, N, K)
    x = _x(2041 + M, (1, M, K))
    res = _x(2042 + M, (1, M, N))
    nw = oracle.round_to(rng(2043).normal(1, 0.1, N), BF)
    h = oracle.round_to(res.astype(np.float64) + _qmm(x, q), BF)
    ins = [to_torch(x, BF)] + _dev(q) + [to_torch(res, BF)]
    _gates(regions.residual(), ins, [h])
    _gates(regions.residual_rmsnorm(eps=1e-6), ins + [to_torch(nw, BF)],
           [h, oracle.rms_norm(h, nw, 1e-6, BF)])


def test_dequant_region():
    q = _quant(2050, 200, 512)
    _gates(regions.dequant(), _dev(q), [oracle.dequantize(*q, 64, 4, BF)], tol=None)


def test_elementwise_and_attention_regions():
    x = _x(2060, (1, 100, 2560))
    w = oracle.round_to(rng(2061).normal(1, 0.1, 2560), BF)
    _gates(regions.rms_norm(), [to_torch(x, BF), to_torch(w, BF)],
           [oracle.rms_norm(x, w, 1e-6, BF)])
    g, u = _x(2062, (1, 100, 200)), _x(2063, (1, 100, 200))
    _gates(regions.swiglu(), [to_torch(g, BF), to_torch(u, BF)], [oracle.swiglu(g, u, BF)])
    qx = _x(2064, (1, 100, 32 * 128))
    qn = oracle.round_to(rng(2065).normal(1, 0.1, 128), BF)
    _gates(regions.norm_rope(), [to_torch(qx, BF), to_torch(qn, BF)],
           [oracle.norm_rope(qx, qn, 1e-6, 32, 128, 1e6, 0, BF)])
    q, k, v = _x(2066, (1, 32, 100, 128)), _x(2067, (1, 8, 100, 128)), _x(2068, (1, 8, 100, 128))
    _gates(regions.sdpa(), [to_torch(q, BF), to_torch(k, BF), to_torch(v, BF)],
           [oracle.sdpa(q, k, v, 128 ** -0.5, True, BF)])


def test_tiny_mlp_region_gates():
    r = rng(2070)
    x = r.normal(0, 1, (32, 256)).astype(np.float32)
    w1 = r.normal(0, 0.02, (1024, 256)).astype(np.float32)
    w2 = r.normal(0, 0.02, (256, 1024)).astype(np.float32)
    b1 = np.zeros(1024, np.float32)
    b2 = np.zeros(256, np.float32)
    ins = [to_torch(a, "float32") for a in (x, w1, b1, w2, b2)]
    want = oracle.tiny_mlp(x, w1, b1, w2, b2).astype(np.float64)
    _gates(regions.tiny_mlp(), ins, [want], tol=1e-5)
    _gates(regions.tiny_mlp_two_stage(), ins, [want], tol=1e-5)
