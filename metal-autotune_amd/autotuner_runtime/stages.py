"""Dataflow of a staged region: several launches run as one region call.

A staged ``KernelSpec`` lists ``KernelStage(inputs, outputs, kernel)``
entries (the reference's stage contract, autotuner_runtime/stages.py:7-39 and
kernels.py:201-205). Every array of the call lives in one buffer table:
first the region inputs, then each stage's results in stage order. A stage
names what it reads (region inputs or earlier results) and what it creates:
fresh ``tmpN`` intermediates or region outputs.

``wiring`` validates a spec once, when it is loaded, and returns the table
positions each stage reads plus the positions of the region outputs. It
rejects, with a ``ValueError`` naming the stage:

* stages that are themselves staged or carry their own fallback predicate,
  recorded signatures or atomic outputs (those are properties of the whole
  region);
* stage kernels whose local names are not ``in0..`` / ``out0..``;
* reads of names not yet in the table;
* results that reuse a name (stages never overwrite an array, inputs least
  of all) or are neither ``tmpN`` nor a region output;
* regions whose outputs are not all produced, or that create intermediates
  nothing reads (dead launches would still be timed as the region's cost).

``shapes`` evaluates each stage's output shapes in the stage's own
``inN`` environment, for the launch resolver.
"""

from __future__ import annotations

import re
from dataclasses import dataclass, field

from .grammar import Expr

_INTERMEDIATE = re.compile(r"tmp[0-9]+")


@dataclass
class _Table:
    """Name -> buffer position, growing as stages produce results."""
    pos: dict = field(default_factory=dict)
    made: list = field(default_factory=list)   # names produced by stages
    read: set = field(default_factory=set)     # names some stage reads

    def add(self, name: str) -> int:
        self.pos[name] = len(self.pos)
        return self.pos[name]


def _check_plain(i: int, kernel, n_in: int, n_out: int) -> None:
    problems = []
    if kernel.stages:
        problems.append("is itself staged")
    if kernel.reference_sequence is not None or kernel.native_call is not None:
        problems.append("is not a plain dispatch")
    if (kernel.fallback_predicate is not None or kernel.input_signature is not None
            or kernel.input_signatures is not None or kernel.atomic_outputs):
        problems.append("sets a fallback/signature/atomic policy, which belongs to the "
                        "whole candidate")
    if tuple(kernel.input_names) != tuple(f"in{j}" for j in range(n_in)):
        problems.append(f"must name its inputs in0..in{n_in - 1} (local inN ABI)")
    if n_out == 0 or tuple(kernel.output_names) != tuple(f"out{j}" for j in range(n_out)):
        problems.append(f"must name its outputs out0..out{max(n_out - 1, 0)} (local outN ABI)")
    if len(kernel.output_shapes) != n_out or len(kernel.output_dtypes) != n_out:
        problems.append("needs one shape and one dtype per output")
    if problems:
        raise ValueError(f"stage {i} kernel {kernel.kernel_id!r}: " + "; ".join(problems))


def wiring(spec) -> tuple[list[tuple[int, ...]], tuple[int, ...]]:
    """(per-stage read positions, region-output positions) of a staged spec."""
    if spec.reference_sequence is not None:
        raise ValueError("a staged region cannot also replay an original sequence")
    table = _Table()
    for name in spec.input_names:
        table.add(name)
    outputs = set(spec.output_names)
    reads: list[tuple[int, ...]] = []
    for i, stage in enumerate(spec.stages):
        _check_plain(i, stage.kernel, len(stage.inputs), len(stage.outputs))
        unknown = [n for n in stage.inputs if n not in table.pos]
        if unknown:
            raise ValueError(f"stage {i} reads unknown array(s) {unknown}: a stage reads "
                             "region inputs or results of earlier stages")
        reads.append(tuple(table.pos[n] for n in stage.inputs))
        table.read.update(stage.inputs)
        for name in stage.outputs:
            if name in table.pos:
                raise ValueError(f"stage {i} writes {name!r}, which already exists; results "
                                 "must be a new tmpN or region output")
            if name not in outputs and not _INTERMEDIATE.fullmatch(name):
                raise ValueError(f"stage {i} result {name!r} must be a new tmpN or region output")
            table.add(name)
            table.made.append(name)
    missing = [n for n in spec.output_names if n not in table.made]
    if missing:
        raise ValueError(f"no stage produces {missing}: stages must produce every region output")
    dead = [n for n in table.made if n not in outputs and n not in table.read]
    if dead:
        raise ValueError(f"intermediate(s) {dead} are never read: unused stage outputs would "
                         "hide work from timing")
    return reads, tuple(table.pos[n] for n in spec.output_names)


def shapes(spec, input_shapes, input_dtypes):
    """Evaluate every stage's output shapes in order.

    Returns ``(walk, results)``: ``walk`` holds, per stage, (its kernel, the
    (shape, dtype) pairs it reads, the shapes it produces); ``results`` the
    (shape, dtype) of each region output."""
    reads, out_pos = wiring(spec)
    buffers = [(tuple(s), d) for s, d in zip(input_shapes, input_dtypes)]
    walk = []
    for stage, pos in zip(spec.stages, reads):
        seen = [buffers[j] for j in pos]
        env = [s for s, _ in seen]
        made = [tuple(Expr(e).evaluate(env) for e in shape) for shape in stage.kernel.output_shapes]
        walk.append((stage.kernel, seen, made))
        buffers += list(zip(made, stage.kernel.output_dtypes))
    return walk, [buffers[j] for j in out_pos]
