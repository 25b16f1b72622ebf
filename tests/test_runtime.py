"""The region runtime on the CPU: launch grammar, spec JSON, launch
resolution and fallback, poison, stage wiring, module swap and apply().

The grammar, fallback and cache expectations are the reference's own
known-answer cases (tests/test_runtime.py:10-136) restated on torch; kernel
bodies are replaced by host stubs registered under a spec's ``source`` name so
the runtime's host logic is exercised without a GPU. The GPU tests call the
real entry points through the same runtime.
"""

from __future__ import annotations

import json

import pytest
import torch
from torch import nn

from autotuner_runtime import hip, kernels, stages, swap
from autotuner_runtime.apply import apply, load_specs
from autotuner_runtime.grammar import Expr, GrammarError
from autotuner_runtime.kernels import KernelSpec, KernelStage, LoadedKernel


# ------------------------------------------------------------------ grammar


def test_grammar_evaluates():
    assert Expr("in0.shape[0] * in0.shape[1]").evaluate([(4, 8)]) == 32
    assert Expr("ceil_div(in0.shape[0], 32) * 32").evaluate([(50,)]) == 64
    assert Expr("in0.ndim == 2 and in0.shape[1] % 4 == 0").evaluate([(3, 8)]) is True
    assert Expr("in1.shape[0] - in0.shape[0]").evaluate([(3,), (10,)]) == 7
    assert Expr("-in0.shape[0] + 5").evaluate([(2,)]) == 3
    assert Expr("max(in0.shape[0] // 3, 2)").evaluate([(10,)]) == 3
    assert Expr("min(in0.shape[-1], 4)").evaluate([(2, 9)]) == 4
    assert Expr("not in0.shape[0] > 3 or in0.ndim != 1").evaluate([(5,)]) is False


@pytest.mark.parametrize("bad", [
    "__import__('os')", "in0.shape[0] ** 2", "lambda: 1", "x", "min(1,2,3)",
    "1.5", "in0.dtype", "f(1,2)", "in0.shape", "[1,2]", "'s'",
])
def test_grammar_rejects_everything_outside(bad):
    with pytest.raises(GrammarError):
        Expr(bad)


def test_grammar_error_is_a_value_error():
    assert issubclass(GrammarError, ValueError)


def test_grammar_runtime_bounds():
    with pytest.raises(GrammarError, match="out of range"):
        Expr("in2.shape[0]").evaluate([(4,)])
    with pytest.raises(GrammarError, match="axis"):
        Expr("in0.shape[5]").evaluate([(4,)])


# ------------------------------------------------------------ spec and JSON


def _double_spec():
    return KernelSpec(
        kernel_id="t_double", name="rt_test_double",
        input_names=("inp",), output_names=("out",),
        source="rt_test_double",
        grid=("in0.shape[0] * in0.shape[1]", "1", "1"),
        threadgroup=("min(in0.shape[0] * in0.shape[1], 256)", "1", "1"),
        output_shapes=(("in0.shape[0]", "in0.shape[1]"),),
        output_dtypes=("float32",),
        template=(("T", "in0"),),
    )


@pytest.fixture
def stubs(monkeypatch):
    """Host stand-ins for entry points, registered by name like the real ones."""
    table = dict(hip.BINDINGS)

    def double(ins, outs, p):
        assert p["T"] == ins[0].dtype
        outs[0].copy_(ins[0] * 2)

    def half_write(ins, outs, p):
        outs[0][:16] = ins[0][:16]

    def copy(ins, outs, p):
        outs[0].copy_(ins[0])

    def add(ins, outs, p):
        outs[0].copy_(ins[0] + ins[1])

    table.update({"rt_test_double": double, "rt_test_half_write": half_write,
                  "rt_copy": copy, "rt_add": add})
    monkeypatch.setattr(hip, "BINDINGS", table)
    kernels._cache.clear()
    yield table
    kernels._cache.clear()


def test_kernel_call_site_and_shape_generality(stubs):
    spec = _double_spec()
    for shape in [(4, 8), (7, 13), (64, 32)]:
        x = torch.randn(shape, generator=torch.Generator().manual_seed(0))
        out = kernels.call(spec, [x])[0]
        assert torch.equal(out, x * 2)


def test_kernel_spec_round_trips():
    spec = _double_spec()
    assert KernelSpec.from_json(spec.to_json()) == spec
    staged = KernelSpec(
        kernel_id="t_staged", name="t_staged", input_names=("in0", "in1"),
        output_names=("out0",), source="",
        output_shapes=(("in0.shape[0]",),), output_dtypes=("float32",),
        stages=(KernelStage(("in0", "in1"), ("tmp0",), _stage("rt_add", 2)),
                KernelStage(("tmp0",), ("out0",), _stage("rt_copy", 1))))
    assert KernelSpec.from_json(staged.to_json()) == staged


def test_load_spec_reads_launch_json_and_entry_name(tmp_path):
    spec = _double_spec()
    d = json.loads(spec.to_json())
    del d["source"]
    (tmp_path / "t_double.launch.json").write_text(json.dumps(d))
    (tmp_path / "t_double.hip").write_text("rt_test_double\n")
    assert kernels.load_spec(tmp_path / "t_double.launch.json") == spec


def test_unknown_entry_point_is_a_build_error():
    spec = KernelSpec(kernel_id="t_nope", name="t_nope", input_names=("in0",),
                      output_names=("out0",), source="mi_no_such_entry",
                      output_shapes=(("1",),), output_dtypes=("float32",))
    with pytest.raises(RuntimeError, match="Unable to bind"):
        LoadedKernel(spec)


@pytest.mark.parametrize("field,value", [("native_call", {"abi": 1}), ("atomic_outputs", True)])
def test_metal_only_fields_are_rejected(stubs, field, value):
    spec = KernelSpec(**{**_double_spec().__dict__, field: value})
    with pytest.raises(ValueError):
        LoadedKernel(spec)


# ------------------------------------------------------ fallback and poison


def test_fallback_predicate_and_poison(stubs):
    spec = KernelSpec(
        kernel_id="t_half", name="rt_test_half_write",
        input_names=("inp",), output_names=("out",), source="rt_test_half_write",
        grid=("32", "1", "1"), threadgroup=("32", "1", "1"),
        output_shapes=(("32",),), output_dtypes=("float32",),
        fallback_predicate="in0.shape[0] != 32",
    )
    lk = LoadedKernel(spec)
    assert lk.fallback_fires([torch.zeros(7)])
    assert not lk.fallback_fires([torch.zeros(32)])
    y = kernels.call(spec, [torch.ones(32)], init_value=float("nan"))[0]
    assert torch.isnan(y[16:]).all()
    assert torch.equal(y[:16], torch.ones(16))


def test_the_fallback_decides_before_the_launch_is_evaluated(stubs):
    spec = KernelSpec(kernel_id="guarded", name="rt_guarded_copy", input_names=("in0",),
                      output_names=("out0",), source="rt_copy",
                      grid=("in0.shape[0]", "1", "1"),
                      threadgroup=("in0.shape[0] // (in0.shape[0] // 8)", "1", "1"),
                      output_shapes=(("in0.shape[0]",),), output_dtypes=("float32",),
                      fallback_predicate="in0.shape[0] < 8")
    lk = LoadedKernel(spec)
    assert lk.fallback_fires([torch.zeros(3)])          # no ZeroDivisionError
    assert kernels.try_call(spec, [torch.zeros(3)]) is None
    assert kernels.try_sized(spec, [torch.zeros(3)]) is None
    x = torch.arange(16, dtype=torch.float32)
    assert kernels.try_call(spec, [x])[0].tolist() == x.tolist()
    with pytest.raises(ValueError, match="fallback"):
        lk([torch.zeros(3)])
    for n in range(kernels.LAUNCH_CACHE_MAX + 5):
        lk.fallback_fires([torch.zeros(8 + n)])
    assert len(lk._launches) <= kernels.LAUNCH_CACHE_MAX


def test_launch_is_evaluated_once_per_call_signature(stubs, monkeypatch):
    from autotuner_runtime import grammar

    calls = []
    real = grammar.Expr.evaluate

    def counting(self, shapes):
        calls.append(self.text)
        return real(self, shapes)

    monkeypatch.setattr(grammar.Expr, "evaluate", counting)
    spec = KernelSpec(kernel_id="once", name="once_copy", input_names=("in0",),
                      output_names=("out0",), source="rt_copy",
                      grid=("in0.shape[0]", "1", "1"), threadgroup=("min(in0.shape[0], 256)", "1", "1"),
                      output_shapes=(("in0.shape[0]",),), output_dtypes=("float32",),
                      fallback_predicate="in0.shape[0] > 64")
    lk = LoadedKernel(spec)
    x = torch.arange(8, dtype=torch.float32)
    assert lk([x])[0].tolist() == x.tolist()
    first = len(calls)
    assert first > 0
    lk([x + 1])
    assert not lk.fallback_fires([x])
    assert len(calls) == first                       # same signature: nothing re-evaluated
    assert lk.fallback_fires([torch.zeros(128)])     # a new shape is evaluated afresh
    assert len(calls) > first


def test_recorded_signatures_bound_try_call_but_not_try_sized(stubs):
    spec = KernelSpec(kernel_id="t_sig", name="t_sig", input_names=("in0",),
                      output_names=("out0",), source="rt_copy",
                      output_shapes=(("in0.shape[0]",),), output_dtypes=("float32",),
                      input_signature=[[[8], "float32"]], fallback_predicate="in0.shape[0] > 32")
    assert kernels.try_call(spec, [torch.zeros(8)]) is not None
    assert kernels.try_call(spec, [torch.zeros(9)]) is None        # not a recorded signature
    assert kernels.try_sized(spec, [torch.zeros(9)]) is not None   # size-generic caller
    assert kernels.try_sized(spec, [torch.zeros(33)]) is None      # the predicate still holds
    assert kernels.try_call(spec, [torch.zeros(8, dtype=torch.float16)]) is None


def test_non_positive_launch_is_an_error(stubs):
    spec = KernelSpec(kernel_id="t_zero", name="t_zero", input_names=("in0",),
                      output_names=("out0",), source="rt_copy",
                      grid=("in0.shape[0] - 8", "1", "1"),
                      output_shapes=(("in0.shape[0]",),), output_dtypes=("float32",))
    with pytest.raises(ValueError, match="non-positive"):
        kernels.call(spec, [torch.zeros(8)])


def test_inputs_are_made_row_contiguous(stubs):
    seen = []

    def probe(ins, outs, p):
        seen.append(ins[0].is_contiguous())
        outs[0].copy_(ins[0])

    stubs["rt_probe"] = probe
    spec = KernelSpec(kernel_id="t_contig", name="t_contig", input_names=("in0",),
                      output_names=("out0",), source="rt_probe",
                      output_shapes=(("in0.shape[0]", "in0.shape[1]"),), output_dtypes=("float32",))
    x = torch.arange(12, dtype=torch.float32).reshape(3, 4).t()
    y = kernels.call(spec, [x])[0]
    assert seen == [True] and torch.equal(y, x)


# --------------------------------------------------------------- stages


def _stage(source, n_in, n_out=1):
    return KernelSpec(kernel_id=f"st_{source}_{n_in}", name=source,
                      input_names=tuple(f"in{i}" for i in range(n_in)),
                      output_names=tuple(f"out{i}" for i in range(n_out)), source=source,
                      output_shapes=(("in0.shape[0]",),) * n_out,
                      output_dtypes=("float32",) * n_out)


def _staged(stage_list, outputs=("out0",)):
    return KernelSpec(kernel_id="t_stg", name="t_stg", input_names=("in0", "in1"),
                      output_names=outputs, source="",
                      output_shapes=(("in0.shape[0]",),) * len(outputs),
                      output_dtypes=("float32",) * len(outputs), stages=tuple(stage_list))


def test_stages_run_as_a_buffer_table(stubs):
    spec = _staged([KernelStage(("in0", "in1"), ("tmp0",), _stage("rt_add", 2)),
                    KernelStage(("tmp0", "in0"), ("out0",), _stage("rt_add", 2))])
    a, b = torch.arange(5.0), torch.ones(5)
    (y,) = kernels.call(spec, [a, b])
    assert torch.equal(y, 2 * a + 1)


@pytest.mark.parametrize("stage_list,match", [
    ([KernelStage(("in0", "in1"), ("in0",), _stage("rt_add", 2))], "new tmpN"),
    ([KernelStage(("in0", "zz"), ("out0",), _stage("rt_add", 2))], "unknown"),
    ([KernelStage(("in0", "in1"), ("tmp0",), _stage("rt_add", 2))], "every region output"),
    ([KernelStage(("in0", "in1"), ("tmp0",), _stage("rt_add", 2)),
      KernelStage(("in0", "in1"), ("out0",), _stage("rt_add", 2))], "unused"),
])
def test_stage_wiring_rules(stage_list, match):
    with pytest.raises(ValueError, match=match):
        stages.wiring(_staged(stage_list))


def test_stage_policies_belong_to_the_region():
    inner = KernelSpec(**{**_stage("rt_add", 2).__dict__, "fallback_predicate": "1 == 1"})
    with pytest.raises(ValueError, match="whole candidate"):
        stages.wiring(_staged([KernelStage(("in0", "in1"), ("out0",), inner)]))


# ------------------------------------------------------------ swap / apply


class _Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.lin = nn.Linear(4, 4)
        self.scale = 3.0

    def forward(self, x):
        return self.lin(x)


class _Model(nn.Module):
    def __init__(self):
        super().__init__()
        self.layers = nn.ModuleList([_Block(), _Block()])

    def forward(self, x):
        for layer in self.layers:
            x = layer(x)
        return x


class _Doubler(swap.ReplayWrapper):
    def forward(self, x):
        return 2 * self.wrapped(x)


def test_install_resolve_uninstall_and_delegation():
    model = _Model()
    x = torch.randn(2, 4)
    base = model(x)
    occupant = swap.install(model, "layers.1", _Doubler(model.layers[1]))
    assert isinstance(model.layers[1], _Doubler)
    assert model.layers[1].scale == 3.0                 # attribute falls through
    assert any(n.endswith("wrapped.lin.weight") for n, _ in model.named_parameters())
    torch.testing.assert_close(model(x), 2 * base)
    swap.uninstall(model, "layers.1", occupant)
    assert model.layers[1] is occupant
    torch.testing.assert_close(model(x), base)
    with pytest.raises(KeyError, match="cannot resolve"):
        swap.resolve(model, "layers.7")
    with pytest.raises(ValueError):
        swap.resolve(model, "")


def test_require_independent_models():
    a = _Model()
    swap.require_independent_models(a, _Model())
    b = _Model()
    b.layers[0] = a.layers[0]
    with pytest.raises(ValueError, match="reused"):
        swap.require_independent_models(a, b)


def test_flatten_arrays_walks_nested_results_in_order():
    a, b, c = torch.zeros(2, 3), torch.zeros(1), torch.zeros(4)
    got = swap.flatten_arrays([a, (b, 7, None), {"k": c, "n": "x"}])
    assert [t.shape for t in got] == [(2, 3), (1,), (4,)]
    assert got[0] is a and got[2] is c
    assert swap.flatten_arrays(5) == []


def test_install_into_dict_and_tuple_children():
    holder = nn.Module()
    holder.blocks = nn.ModuleDict({"a": _Block()})
    old = swap.install(holder, "blocks.a", _Doubler(holder.blocks["a"]))
    assert isinstance(holder.blocks["a"], _Doubler) and holder.blocks["a"].wrapped is old
    swap.uninstall(holder, "blocks.a", old)
    assert holder.blocks["a"] is old
    frozen = {"t": (_Block(),)}
    with pytest.raises(TypeError, match="tuple"):
        swap.install(frozen, "t.0", _Doubler(frozen["t"][0]))


def test_apply_installs_an_artifact(tmp_path, stubs):
    (tmp_path / "kernels").mkdir()
    (tmp_path / "patch").mkdir()
    spec = _double_spec()
    (tmp_path / "kernels" / "t_double.launch.json").write_text(spec.to_json())
    (tmp_path / "swap_table.json").write_text(json.dumps([
        {"scope_path": "layers.0", "wrapper_class": "Twice", "kernel_ids": ["t_double"]}]))
    (tmp_path / "patch" / "wrappers.py").write_text(
        "from autotuner_runtime import kernels\n"
        "from autotuner_runtime.swap import ReplayWrapper\n"
        "class Twice(ReplayWrapper):\n"
        "    def forward(self, x):\n"
        "        y = self.wrapped(x)\n"
        "        out = kernels.try_sized(self._specs['t_double'], [y])\n"
        "        return y * 2 if out is None else out[0]\n")
    assert sorted(load_specs(tmp_path)) == ["t_double"]
    model = _Model()
    x = torch.randn(3, 4)
    want = model.layers[1](2 * model.layers[0](x))
    patched = apply(model, tmp_path)
    assert patched is model and type(model.layers[0]).__name__ == "Twice"
    torch.testing.assert_close(model(x), want)
