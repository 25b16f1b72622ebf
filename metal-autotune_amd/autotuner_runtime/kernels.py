"""Kernel specs and the one call site, on torch tensors and the gfx950 HIP library.

The same API as the reference's autotuner_runtime/kernels.py: ``KernelSpec``
(:35-72) and ``KernelStage`` (:76-79) with the same fields and JSON form,
``load_spec`` (:82-90), ``LoadedKernel.launch`` / ``__call__`` (:145-220) and
the module-level ``fallback_fires`` / ``call`` / ``try_call`` / ``try_sized``
(:241-268), with the same semantics:

* the launch is a function of the inputs' shapes and dtypes, resolved once
  per call signature (at most LAUNCH_CACHE_MAX kept); the fallback predicate
  and the recorded ``input_signature(s)`` are read before any other launch
  expression is evaluated, so a shape the kernel does not cover never
  evaluates (possibly undefined) grid arithmetic;
* ``try_call`` / ``try_sized`` return None on a fallback shape so the caller
  runs its original ops; calling a kernel on such a shape raises ValueError;
* outputs are allocated by the runtime from ``output_shapes`` /
  ``output_dtypes`` and pre-filled with ``init_value`` when given (NaN poison);
  inputs are made row-contiguous when ``ensure_row_contiguous``;
* stages run as a buffer table: region inputs, then every stage's outputs.

What differs is the backend. ``source`` names a C-ABI entry point of the
gfx950 library (include/mi_qmm.h) instead of carrying a Metal body; ``name``
stays a C identifier for the record. ``template`` entries are (name, value)
with value a dtype name, ``"inK"`` (input K's dtype), or a numeric literal --
the entry point's scalar arguments (group_size, bits, eps, ...). The HIP entry
points own their launch geometry (tiles are chosen per shape inside the
library), so ``grid`` / ``threadgroup`` are evaluated and validated like any
launch expression but not passed on; specs generated for this backend leave
them at ("1", "1", "1"), as the reference's staged specs do.
``reference_sequence`` (an MLX op replay) and ``native_call`` (a captured
Metal ABI) have no meaning here and are rejected at load.

Calls are stream-ordered on ``torch.cuda.current_stream()`` and never
synchronize the host.
"""

from __future__ import annotations

import importlib
import json
from dataclasses import asdict, dataclass
from pathlib import Path
from typing import NamedTuple

import torch

from .grammar import Expr

_DTYPES = {
    "bool": torch.bool, "uint8": torch.uint8, "uint16": torch.uint16, "uint32": torch.uint32,
    "uint64": torch.uint64, "int8": torch.int8, "int16": torch.int16, "int32": torch.int32,
    "int64": torch.int64, "float16": torch.float16, "bfloat16": torch.bfloat16,
    "float32": torch.float32, "complex64": torch.complex64,
}
_NAMES = {v: k for k, v in _DTYPES.items()}


def dtype_name(dtype: torch.dtype) -> str:
    return _NAMES[dtype]


@dataclass(frozen=True)
class KernelSpec:
    kernel_id: str
    name: str                                  # a valid C identifier
    input_names: tuple[str, ...]
    output_names: tuple[str, ...]
    source: str                                # C-ABI entry point of the HIP library
    header: str = ""
    grid: tuple[str, str, str] = ("1", "1", "1")         # launch grammar, TOTAL threads
    threadgroup: tuple[str, str, str] = ("1", "1", "1")
    output_shapes: tuple[tuple[str, ...], ...] = ()      # one expr tuple per output
    output_dtypes: tuple[str, ...] = ()
    template: tuple[tuple[str, str], ...] = ()           # (name, dtype | "inK" | literal)
    fallback_predicate: str | None = None                # true -> use the original ops
    ensure_row_contiguous: bool = True
    atomic_outputs: bool = False
    native_call: dict | None = None
    input_signature: list | None = None
    input_signatures: list | None = None
    reference_sequence: dict | None = None
    stages: tuple["KernelStage", ...] = ()
    reassociates: bool = False

    def to_json(self) -> str:
        d = {k: getattr(self, k) for k in self.__dataclass_fields__}
        d["stages"] = [asdict(stage) for stage in self.stages]
        return json.dumps(d, indent=1)

    @staticmethod
    def from_json(text: str) -> "KernelSpec":
        d = json.loads(text)
        for key in ("input_names", "output_names", "grid", "threadgroup", "output_dtypes"):
            d[key] = tuple(d[key])
        d["output_shapes"] = tuple(tuple(s) for s in d["output_shapes"])
        d["template"] = tuple(tuple(t) for t in d.get("template", ()))
        d["stages"] = tuple(
            KernelStage(tuple(s["inputs"]), tuple(s["outputs"]),
                        KernelSpec.from_json(json.dumps(s["kernel"])))
            for s in d.get("stages", ()))
        return KernelSpec(**d)


@dataclass(frozen=True)
class KernelStage:
    inputs: tuple[str, ...]   # region inN or an earlier tmpN/outN
    outputs: tuple[str, ...]  # new tmpN/outN names; never overwrite an array
    kernel: KernelSpec        # local ABI: in0.. and out0..


def load_spec(path: str | Path) -> KernelSpec:
    """Rebuild a spec from ``<id>.launch.json`` (+ ``<id>.hip`` holding the entry
    point name when the JSON has no ``source``) -- the reference's
    ``<id>.metal`` + ``<id>.launch.json`` pair (kernels.py:82-90)."""
    path = Path(path)
    stem = path.name
    for suffix in (".launch.json", ".hip", ".json"):
        if stem.endswith(suffix):
            stem = stem[: -len(suffix)]
            break
    base = path.with_name(stem)
    launch = json.loads(base.with_name(stem + ".launch.json").read_text())
    if "source" not in launch:
        launch["source"] = base.with_name(stem + ".hip").read_text().strip()
    for i, stage in enumerate(launch.get("stages", ())):
        if "source" not in stage["kernel"]:
            stage["kernel"]["source"] = (base.with_name(stem + ".stages") / f"{i}.hip").read_text().strip()
    return KernelSpec.from_json(json.dumps(launch))


class Launch(NamedTuple):
    """One call signature's launch, or the fact that the fallback covers it."""
    fallback: bool
    output_shapes: list | None = None
    grid: tuple | None = None
    threadgroup: tuple | None = None
    template: list | None = None


LAUNCH_CACHE_MAX = 64  # signatures kept per kernel; a shape sweep needs a handful


def _template_value(value: str, inputs):
    if value.startswith("in") and value[2:].isdigit():
        return inputs[int(value[2:])].dtype
    if value in _DTYPES:
        return _DTYPES[value]
    try:
        return int(value)
    except ValueError:
        pass
    try:
        return float(value)
    except ValueError:
        raise ValueError(f"template value {value!r} is not a dtype, inK or a number") from None


class LoadedKernel:
    """A spec bound to its HIP entry point plus its parsed launch expressions."""

    def __init__(self, spec: KernelSpec):
        from . import hip  # the backend; imported lazily so grammar-only use needs no GPU

        self.spec = spec
        if spec.reference_sequence is not None:
            raise ValueError(f"kernel {spec.kernel_id}: reference sequences replay MLX ops; "
                             "the HIP backend runs kernels only")
        if spec.native_call is not None:
            raise ValueError(f"kernel {spec.kernel_id}: native_call binds a captured Metal ABI")
        if spec.atomic_outputs:
            raise ValueError(f"kernel {spec.kernel_id}: atomic outputs are not part of this ABI")
        self._stages = None
        if spec.stages:
            from .stages import wiring
            indices, self._stage_outputs = wiring(spec)
            self._stages = [(LoadedKernel(stage.kernel), idx)
                            for stage, idx in zip(spec.stages, indices)]
            self._entry = None
        else:
            self._entry = hip.binding(spec.source)  # unknown entry -> RuntimeError (a build error)
        self._grid = tuple(Expr(e) for e in spec.grid)
        self._tg = tuple(Expr(e) for e in spec.threadgroup)
        self._out_shapes = tuple(tuple(Expr(e) for e in s) for s in spec.output_shapes)
        self._out_dtypes = [_DTYPES[d] for d in spec.output_dtypes]
        self._fallback = Expr(spec.fallback_predicate) if spec.fallback_predicate else None
        self._launches: dict[tuple, Launch] = {}

    def launch(self, inputs: list[torch.Tensor], checked_elsewhere: bool = False) -> Launch:
        """checked_elsewhere: the caller serves only sizes it checked this kernel
        at, so recorded signatures do not bound the call; the fallback
        predicate still does."""
        key = (checked_elsewhere, *((tuple(a.shape), a.dtype) for a in inputs))
        launch = self._launches.get(key)
        if launch is not None:
            return launch
        shapes = [shape for shape, _ in key[1:]]
        spec = self.spec
        signature = [[list(a.shape), dtype_name(a.dtype)] for a in inputs]
        if ((not checked_elsewhere and (
                (spec.input_signature is not None and signature != spec.input_signature)
                or (spec.input_signatures is not None and signature not in spec.input_signatures)))
                or (self._fallback is not None and self._fallback.evaluate(shapes))):
            launch = Launch(fallback=True)
        else:
            template = [(name, _template_value(v, inputs)) for name, v in spec.template]
            launch = Launch(
                fallback=False,
                output_shapes=[tuple(int(e.evaluate(shapes)) for e in s) for s in self._out_shapes],
                grid=tuple(int(e.evaluate(shapes)) for e in self._grid),
                threadgroup=tuple(int(e.evaluate(shapes)) for e in self._tg),
                template=template,
            )
            if any(g <= 0 for g in launch.grid + launch.threadgroup):
                raise ValueError(f"kernel {spec.kernel_id}: non-positive launch {launch.grid} "
                                 f"{launch.threadgroup}")
            if self._stages is not None:
                from .stages import shapes as stage_shapes
                _, outs = stage_shapes(spec, shapes, [dtype_name(d) for _, d in key[1:]])
                if outs != list(zip(launch.output_shapes, spec.output_dtypes)):
                    raise ValueError("stage results do not match the candidate's output shapes/dtypes")
        if len(self._launches) >= LAUNCH_CACHE_MAX:
            self._launches.clear()
        self._launches[key] = launch
        return launch

    def fallback_fires(self, inputs: list[torch.Tensor]) -> bool:
        return self.launch(inputs).fallback

    def __call__(self, inputs: list[torch.Tensor], init_value: float | None = None,
                 launch: Launch | None = None) -> list[torch.Tensor]:
        launch = launch or self.launch(inputs)
        if launch.fallback:
            raise ValueError(f"kernel {self.spec.kernel_id}: these shapes are the fallback's; "
                             "the original ops take them")
        if self.spec.ensure_row_contiguous:
            inputs = [a.contiguous() for a in inputs]
        if self._stages is not None:
            buffers = list(inputs)
            for kernel, idx in self._stages:
                buffers.extend(kernel([buffers[i] for i in idx], init_value=init_value))
            return [buffers[i] for i in self._stage_outputs]
        device = inputs[0].device
        outputs = []
        for shape, dtype in zip(launch.output_shapes, self._out_dtypes):
            if init_value is None:
                outputs.append(torch.empty(shape, dtype=dtype, device=device))
            else:
                outputs.append(torch.full(shape, init_value, dtype=dtype, device=device))
        self._entry(inputs, outputs, dict(launch.template))
        return outputs


def imported(path: str):
    """A callable found by its import path (the reference's kernels.imported)."""
    module, _, name = path.rpartition(".")
    return getattr(importlib.import_module(module), name)


_cache: dict[str, LoadedKernel] = {}


def _loaded(spec: KernelSpec) -> LoadedKernel:
    loaded = _cache.get(spec.kernel_id)
    if loaded is None or loaded.spec is not spec:
        loaded = LoadedKernel(spec)
        _cache[spec.kernel_id] = loaded
    return loaded


def fallback_fires(spec: KernelSpec, inputs: list[torch.Tensor]) -> bool:
    """True when this call's shapes are not covered and the wrapper must take
    the original op sequence instead."""
    return _loaded(spec).fallback_fires(inputs)


def call(spec: KernelSpec, inputs: list[torch.Tensor], init_value: float | None = None,
         launch: Launch | None = None) -> list[torch.Tensor]:
    """The replacement call site: every dispatch of the region, in order."""
    return _loaded(spec)(inputs, init_value=init_value, launch=launch)


def try_call(spec: KernelSpec, inputs: list[torch.Tensor]) -> list[torch.Tensor] | None:
    """The kernel's outputs, or None when the fallback covers these shapes."""
    launch = _loaded(spec).launch(inputs)
    return None if launch.fallback else call(spec, inputs, launch=launch)


def try_sized(spec: KernelSpec, inputs: list[torch.Tensor],
              init_value: float | None = None) -> list[torch.Tensor] | None:
    """try_call for a size-generic wrapper: recorded signatures do not bound the
    call, the fallback predicate still does."""
    launch = _loaded(spec).launch(inputs, checked_elsewhere=True)
    return None if launch.fallback else call(spec, inputs, init_value=init_value, launch=launch)
