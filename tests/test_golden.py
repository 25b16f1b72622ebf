"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from the CPU oracle).

CPU: the oracle recomputes every fixture bit for bit, so a change that moves
any oracle output is caught against data fixed in the repository.

GPU: the HIP entry points, called through the C ABI on the fixture inputs,
match the fixture outputs -- dequant and argmax bit-exact, everything else
within the max-abs-normalised tolerance written beside each call (1e-2 for
bf16/fp16 outputs, 1e-5 for fp32).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

import oracle
from conftest import to_np, to_torch

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_golden  # noqa: E402

NAMES = sorted(make_golden.CASES)


def test_every_case_has_a_committed_fixture():
    on_disk = sorted(p.stem for p in make_golden.HERE.glob("*.npz"))
    assert on_disk == NAMES


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_fixture_bit_for_bit(name, oracle_lib):
    meta, arrays = make_golden.load(name)
    meta2, arrays2 = make_golden.build(name)
    assert meta == meta2
    assert sorted(arrays) == sorted(arrays2)
    for key in arrays:
        a, b = np.asarray(arrays[key]), np.asarray(arrays2[key])
        assert a.shape == b.shape and a.dtype == b.dtype, key
        assert a.tobytes() == b.tobytes(), f"{name}:{key} changed"


def _close(got, want, tol):
    want = np.asarray(want, np.float64)
    err = np.abs(np.asarray(got, np.float64) - want).max() / max(np.abs(want).max(), 1e-30)
    assert err <= tol, f"max-abs-normalised error {err:.3e} > {tol}"


def _tol(dtype):
    return 1e-5 if dtype == "float32" else 1e-2


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_hip_matches_fixture(name):
    import torch

    from autotuner_runtime import kernels, ops, regions

    meta, a = make_golden.load(name)
    dt = meta["dtype"]
    op = meta["op"]

    def T(key):
        return to_torch(a[f"in_{key}"], dt)

    def W():
        return (torch.from_numpy(a["in_w"]).cuda(), T("scales"), T("biases"))

    if op == "dequant":
        got = ops.dequantize(*W(), meta["group_size"], meta["bits"])
        want = a["out_out"]
        assert np.array_equal(to_np(got).view(np.uint32), want.view(np.uint32)), "not bit-exact"
    elif op == "qmm":
        got = ops.quantized_matmul(T("x"), *W(), group_size=meta["group_size"], bits=meta["bits"])
        _close(to_np(got), a["out_y"], _tol(dt))
    elif op == "rms_norm":
        _close(to_np(ops.rms_norm(T("x"), T("weight"), meta["eps"])), a["out_y"], _tol(dt))
    elif op == "norm_rope":
        got = ops.norm_rope(T("x"), T("weight"), meta["heads"], meta["eps"], meta["dims"],
                            meta["base"], meta["offset"])
        _close(to_np(got), a["out_y"], _tol(dt))
    elif op == "sdpa":
        got = ops.scaled_dot_product_attention(T("q"), T("k"), T("v"), meta["scale"], "causal")
        _close(to_np(got), a["out_o"], _tol(dt))
    elif op == "swiglu":
        _close(to_np(ops.swiglu(T("g"), T("u"))), a["out_y"], _tol(dt))
    elif op == "shortconv":
        state = T("state") if "in_state" in a else None
        out, st = ops.shortconv(T("bx"), T("c"), T("w"), state)
        _close(to_np(out), a["out_out"], _tol(dt))
        assert np.array_equal(to_np(st), a["out_state_out"])  # a copy of the last two rows
    elif op == "tiny_mlp":
        ins = [T("x"), T("w1"), T("b1"), T("w2"), T("b2")]
        h = ops.linear_f32(ins[0], ins[1], ins[2], gelu=True)
        _close(to_np(ops.linear_f32(h, ins[3], ins[4])), a["out_y"], 1e-5)   # two launches
        (got,) = kernels.call(regions.tiny_mlp(), ins, init_value=float("nan"))  # one launch
        _close(to_np(got), a["out_y"], 1e-5)
    elif op == "argmax":
        got = ops.argmax(T("x")).cpu().numpy()
        assert np.array_equal(got, a["out_idx"])
    else:
        raise AssertionError(f"unknown op {op}")
    torch.cuda.synchronize()


def test_fixtures_hold_no_pickles():
    for p in make_golden.HERE.glob("*.npz"):
        with np.load(p, allow_pickle=False) as z:
            for k in z.files:
                assert z[k].dtype != object, f"{p.name}:{k}"


def test_tie_breaking_fixture_has_a_tie():
    _, a = make_golden.load("argmax_bf16")
    x = a["in_x"][1]
    assert (x == x.max()).sum() == 2 and a["out_idx"][1] == int(np.flatnonzero(x == x.max())[0])
    assert oracle.round_to(x, "bfloat16").tobytes() == x.tobytes()
