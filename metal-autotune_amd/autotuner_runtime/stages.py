"""Explicit multi-dispatch dataflow of a region (the reference's stages.py:1-53).

A staged spec is a list of KernelStage(inputs, outputs, kernel): each stage
reads region inputs or earlier stage results by name and produces new
``tmpN`` scratch arrays or region outputs. The rules are the reference's:
no stage writes an input, stages are plain (non-nested) dispatches with
local ``inN``/``outN`` names, policies (fallback, signatures) belong to the
whole region, every region output is produced, and no intermediate result
is left unused (dead work would hide from timing).
"""

from __future__ import annotations

import re

from .grammar import Expr

_TMP = re.compile(r"tmp\d+")


def wiring(spec):
    """Return (per-stage input indices into the buffer table, output indices)."""
    if spec.reference_sequence is not None:
        raise ValueError("stages cannot also be an original reference sequence")
    table = {name: pos for pos, name in enumerate(spec.input_names)}
    produced: set[str] = set()
    consumed: set[str] = set()
    per_stage = []
    for i, stage in enumerate(spec.stages):
        k = stage.kernel
        if k.stages or k.reference_sequence is not None or k.native_call is not None:
            raise ValueError(f"stage {i}: must be a plain, non-nested dispatch")
        if (k.fallback_predicate is not None or k.input_signature is not None
                or k.input_signatures is not None or k.atomic_outputs):
            raise ValueError(f"stage {i}: fallback and compiler policies belong to the whole candidate")
        missing = [n for n in stage.inputs if n not in table]
        if missing:
            raise ValueError(f"stage {i}: inputs must name region inputs or earlier results "
                             f"(unknown {missing})")
        if tuple(k.input_names) != tuple(f"in{j}" for j in range(len(stage.inputs))):
            raise ValueError(f"stage {i}: kernel input names must use the local inN ABI")
        if not stage.outputs or tuple(k.output_names) != tuple(
                f"out{j}" for j in range(len(stage.outputs))):
            raise ValueError(f"stage {i}: kernel output names must use the local outN ABI")
        if len(k.output_shapes) != len(stage.outputs) or len(k.output_dtypes) != len(stage.outputs):
            raise ValueError(f"stage {i}: each output needs a shape and dtype")
        per_stage.append(tuple(table[n] for n in stage.inputs))
        consumed.update(stage.inputs)
        for name in stage.outputs:
            if name in table or not (name in spec.output_names or _TMP.fullmatch(name)):
                raise ValueError(f"stage {i}: output {name!r} must be a new tmpN or region output")
            table[name] = len(table)
            produced.add(name)
    if not set(spec.output_names) <= produced:
        raise ValueError("stages must produce every region output")
    if produced - consumed - set(spec.output_names):
        raise ValueError("unused stage outputs would hide work from timing; remove them")
    return per_stage, tuple(table[n] for n in spec.output_names)


def shapes(spec, input_shapes, input_dtypes):
    """Walk the stages in order, evaluating each stage's output shapes in its own
    local inN environment. Returns ([(kernel, [(shape, dtype)...], [shape...])...],
    [(shape, dtype) of each region output])."""
    per_stage, outs = wiring(spec)
    buffers = list(zip(input_shapes, input_dtypes))
    walked = []
    for stage, idx in zip(spec.stages, per_stage):
        ins = [buffers[j] for j in idx]
        env = [shape for shape, _ in ins]
        out_shapes = [tuple(Expr(e).evaluate(env) for e in shape)
                      for shape in stage.kernel.output_shapes]
        walked.append((stage.kernel, ins, out_shapes))
        buffers.extend(zip(out_shapes, stage.kernel.output_dtypes))
    return walked, [buffers[j] for j in outs]
