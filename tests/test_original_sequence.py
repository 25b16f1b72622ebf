"""Replay of recorded original op sequences (``KernelSpec.reference_sequence``).

The record format is the reference's (autotuner/trace/serialize.py:16-30,
57-71; autotuner/scaffold/native.py:61-118): op names, each node's input and
output array ids, and scalar arguments with tagged containers. These run on
CPU tensors through the torch half of the op table; the library ops of the
table (quantized matmul, norms, RoPE, attention) run in
tests/test_kernels_gpu.py::test_reference_sequence_replays_library_ops.
"""

import pytest
import torch

from autotuner_runtime import kernels
from autotuner_runtime.kernels import KernelSpec, LoadedKernel
from autotuner_runtime.original_sequence import prepare_sequence, resolve


def ref(i):
    return {"$": "ref", "i": i}


def tup(*items):
    return {"$": "tuple", "items": list(items)}


def node(op, ins, outs, *args, **kwargs):
    return {"seq": 0, "op": op, "in_arrays": list(ins), "out_arrays": list(outs),
            "args": tup(*args), "kwargs": kwargs, "kernel_definition": None}


# silu(gate) * up with gate, up = split(x, 2, axis=-1): the LFM2 MLP's shape
SWIGLU = {
    "nodes": [
        node("mx.split", [0], [1, 2], ref(0), 2, axis=-1),
        node("mx.sigmoid", [1], [3], ref(0)),
        node("array.__mul__", [1, 3], [4], ref(0), ref(1)),
        node("array.__mul__", [4, 2], [5], ref(0), ref(1)),
    ],
    "input_ids": [0],
    "output_ids": [5],
}


def test_replay_follows_the_wiring():
    x = torch.randn(3, 8, generator=torch.Generator().manual_seed(1))
    (y,) = prepare_sequence(SWIGLU)([x])
    g, u = x[:, :4], x[:, 4:]
    assert torch.equal(y, (g * torch.sigmoid(g)) * u)


def test_tagged_arguments_decode():
    """Tuples, lists, dicts, slices, dtypes and Ellipsis as the recorder
    writes them; a reference inside a list; keyword arguments."""
    seq = {
        "nodes": [
            node("mx.reshape", [0], [1], ref(0), tup(2, 3, 4)),
            node("mx.transpose", [1], [2], ref(0), {"$": "list", "items": [0, 2, 1]}),
            node("array.__getitem__", [2], [3], ref(0),
                 tup({"$": "ellipsis"}, {"$": "slice", "parts": [1, None, None]})),
            node("array.astype", [3], [4], ref(0), {"$": "dtype", "name": "float16"}),
            node("mx.concatenate", [4, 4], [5], {"$": "list", "items": [ref(0), ref(1)]}, axis=1),
            node("mx.mean", [5], [6], ref(0), axis=-1, keepdims=True),
        ],
        "input_ids": [0],
        "output_ids": [5, 6],
    }
    x = torch.arange(24, dtype=torch.float32)
    cat, mean = prepare_sequence(seq)([x])
    t = x.reshape(2, 3, 4).permute(0, 2, 1)[..., 1:].to(torch.float16)
    want = torch.cat([t, t], dim=1)
    assert torch.equal(cat, want)
    assert torch.equal(mean, want.mean(dim=-1, keepdim=True))


def test_variants_pick_the_recorded_signature():
    double = {"nodes": [node("array.__add__", [0, 0], [1], ref(0), ref(1))],
              "input_ids": [0], "output_ids": [1]}
    square = {"nodes": [node("mx.square", [0], [1], ref(0))], "input_ids": [0], "output_ids": [1]}
    run = prepare_sequence({"variants": [
        {"signature": [[[2], "float32"]], "sequence": double},
        {"signature": [[[3], "float32"]], "sequence": square}]})
    assert torch.equal(run([torch.tensor([1.0, 3.0])])[0], torch.tensor([2.0, 6.0]))
    assert torch.equal(run([torch.tensor([1.0, 2.0, 3.0])])[0], torch.tensor([1.0, 4.0, 9.0]))
    with pytest.raises(ValueError, match="no recorded variant"):
        run([torch.zeros(4)])


def test_resolver_distinguishes_invert_from_mutation():
    """A pure operator whose name starts with __i resolves; an in-place one
    is not a fusion starter (the reference's
    tests/test_native_fusion.py:183-190)."""
    assert resolve("array.__invert__") is not None
    assert resolve("array.__getitem__") is not None
    with pytest.raises(ValueError, match="mutating operation"):
        resolve("array.__iadd__")
    with pytest.raises(ValueError, match="mutating operation"):
        resolve("array.__setitem__")


@pytest.mark.parametrize("bad,match", [
    ({"nodes": [{**node("mx.sigmoid", [0], [1], ref(0)), "kernel_definition": {"source": "x"}}],
      "input_ids": [0], "output_ids": [1]}, "captured Metal kernel"),
    ({"nodes": [node("mx.conv_general", [0], [1], ref(0))], "input_ids": [0],
      "output_ids": [1]}, "cannot be replayed"),
    ({"nodes": [node("mx.sigmoid", [0], [1], ref(1))], "input_ids": [0],
      "output_ids": [1]}, "refers to input 1"),
    ({"nodes": [node("mx.sigmoid", [7], [1], ref(0))], "input_ids": [0],
      "output_ids": [1]}, "no earlier node"),
    ({"nodes": [node("mx.sigmoid", [0], [1], ref(0))], "input_ids": [0],
      "output_ids": [9]}, "not all produced"),
    ({"ops": []}, "needs"),
])
def test_unreplayable_records_are_refused_at_load(bad, match):
    with pytest.raises(ValueError, match=match):
        prepare_sequence(bad)


def test_output_count_must_match_the_record():
    seq = {"nodes": [node("mx.split", [0], [1], ref(0), 2)], "input_ids": [0], "output_ids": [1]}
    with pytest.raises(ValueError, match="2 output arrays"):
        prepare_sequence(seq)([torch.zeros(4)])


def test_loaded_kernel_runs_a_sequence_spec():
    """A starter spec (the reference's sequence_seed: a comment for source,
    unit launch) runs its replay through kernels.call, no entry point bound;
    the fallback predicate still routes uncovered shapes to the original ops."""
    spec = KernelSpec(
        kernel_id="sequence_seed", name="at_sequence_seed", input_names=("in0",),
        output_names=("out0",), source="// original sequence starter",
        output_shapes=(("in0.shape[0]", "in0.shape[1] / 2"),), output_dtypes=("float32",),
        fallback_predicate="in0.shape[1] % 2", reference_sequence=SWIGLU)
    x = torch.randn(2, 6, generator=torch.Generator().manual_seed(2))
    (y,) = kernels.call(spec, [x])
    assert torch.equal(y, prepare_sequence(SWIGLU)([x])[0])
    assert kernels.try_call(spec, [torch.zeros(2, 5)]) is None
    staged = KernelSpec(**{**spec.__dict__, "stages": (None,)})
    with pytest.raises(ValueError, match="staged region"):
        LoadedKernel(staged)
