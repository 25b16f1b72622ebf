"""Size-generic serving on the CPU: the served-range rule (the reference's
autotuner/serve.py:264-291 restated), the size tests written into generated
wrappers, and SizedRegions gating try_sized by the served ranges."""

from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")


def test_runs_and_size_test():
    from autotuner_runtime.serve import runs, size_test

    assert runs([5, 3, 4, 9, 10, 3]) == [[3, 5], [9, 10]]
    assert runs([]) == []
    assert size_test([7]) == "_n == 7"
    assert size_test(range(2, 2049)) == "2 <= _n <= 2048"
    assert size_test([1, 3]) == "_n in (1, 3)"
    assert size_test([]) == "False"
    _n = 2048
    assert eval(size_test(range(2, 2049)))


def _clock(wins=(), losses=(), ties=()):
    c = {n: {"win": True, "loss": False} for n in wins}
    c.update({n: {"win": False, "loss": True} for n in losses})
    c.update({n: {"win": False, "loss": False} for n in ties})
    return c


def test_served_range_rule():
    from autotuner_runtime.serve import served_range

    correct = list(range(1, 101))
    # wins on both sides out to the grid ends
    assert served_range(correct, _clock(wins=(10, 50, 90, 100)), 50) == (10, 100)
    # a grid point it does not win at stops that side; the furthest win before it bounds it
    assert served_range(correct, _clock(wins=(10, 50, 90), ties=(30,)), 50) == (50, 90)
    # a loss removes the size from the correct run: the range never passes it
    assert served_range(correct, _clock(wins=(10, 50, 90), losses=(70,)), 50) == (10, 50)
    # a sample outside the grid that only ties neither extends nor stops
    assert served_range(correct, _clock(wins=(10, 50, 90), ties=(30,)), 50, grid={10, 50, 90}) \
        == (10, 90)
    # an incorrect size breaks the contiguous run
    assert served_range([n for n in correct if n != 20], _clock(wins=(10, 50)), 50) == (50, 50)
    # the primary itself incorrect or losing -> not served
    assert served_range([1, 2], _clock(wins=(1,)), 3) is None
    assert served_range(correct, _clock(losses=(50,)), 50) is None


def test_sized_regions_gate_try_sized(monkeypatch):
    from autotuner_runtime import kernels, serve
    from autotuner_runtime.kernels import KernelSpec

    calls = []
    monkeypatch.setattr(kernels, "try_sized", lambda spec, ins, init_value=None:
                        calls.append(spec.kernel_id) or ["kernel"])
    spec = KernelSpec(kernel_id="k1", name="mi_qmm_affine", input_names=("in0",),
                      output_names=("out0",), source="mi_qmm_affine",
                      output_shapes=(("in0.shape[0]",),), output_dtypes=("bfloat16",))

    class W(serve.SizedRegions):
        def forward(self, x, n):
            out = self._try("role", [x], n)
            return "original" if out is None else out[0]

    w = W(torch.nn.Identity(), {"role": spec})
    assert w(torch.zeros(1), 5) == "kernel"               # RANGES None: every size
    W.RANGES = {"k1": [[2, 4], [8, 8]]}
    assert [w(torch.zeros(1), n) for n in (1, 2, 4, 5, 8, 9)] == \
        ["original", "kernel", "kernel", "original", "kernel", "original"]
    w.set_ranges({"k1": []})                               # instance override: served nowhere
    assert w(torch.zeros(1), 3) == "original"
    assert W(torch.nn.Identity(), {})(torch.zeros(1), 3) == "original"  # no spec for the role
    assert calls == ["k1", "k1", "k1", "k1"]


def test_sized_regions_serves_agrees_with_try():
    """``_serves`` (a caller about to run a fused form of a cut) says yes
    exactly where ``_try`` would launch: spec present, size served, fallback
    predicate quiet."""
    from autotuner_runtime import serve
    from autotuner_runtime.kernels import KernelSpec

    spec = KernelSpec(kernel_id="k2", name="mi_qmm_affine", input_names=("in0",),
                      output_names=("out0",), source="mi_qmm_affine",
                      output_shapes=(("in0.shape[0]",),), output_dtypes=("bfloat16",),
                      fallback_predicate="in0.shape[0] > 4")

    class W(serve.SizedRegions):
        def forward(self, x, n):
            return self._serves("role", [x], n)

    w = W(torch.nn.Identity(), {"role": spec})
    assert w(torch.zeros(3), 7) is True
    assert w(torch.zeros(5), 7) is False                  # the predicate declines
    w.set_ranges({"k2": [[1, 4]]})
    assert w(torch.zeros(3), 7) is False and w(torch.zeros(3), 2) is True
    assert W(torch.nn.Identity(), {})(torch.zeros(3), 2) is False  # no spec for the role
