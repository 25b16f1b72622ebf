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
A spec with a ``reference_sequence`` (the region's recorded original MLX
calls, a starter when no single kernel exists) replays those calls through
the library's ops and torch (``original_sequence.prepare_sequence``), as the
reference's LoadedKernel does (kernels.py:125-127,199-200). ``native_call``
(a captured Metal ABI) has no meaning here and is rejected at load.

Calls are stream-ordered on ``torch.cuda.current_stream()`` and never
synchronize the host.
"""

from __future__ import annotations

import json
from collections import OrderedDict
from dataclasses import asdict, dataclass
from pathlib import Path

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


@dataclass(frozen=True)
class Launch:
    """The resolved launch of one call signature.

    ``fallback`` true: the spec does not cover these shapes and the caller's
    original ops run. Otherwise the evaluated output shapes, the (validated,
    unused) grid / threadgroup, and the entry point's scalar arguments."""
    fallback: bool
    output_shapes: tuple = ()
    grid: tuple = ()
    threadgroup: tuple = ()
    template: tuple = ()


# Resolved signatures kept per kernel, least recently used dropped first. A
# wrapper serving a range of prompt lengths sees one signature per length.
LAUNCH_CACHE_MAX = 64


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


def _signature(inputs) -> list:
    """The recorded-signature form of a call: [[shape list, dtype name], ...]."""
    return [[list(a.shape), dtype_name(a.dtype)] for a in inputs]


class LoadedKernel:
    """A spec bound to its HIP entry point (or its stages), with the launch
    expressions parsed once."""

    def __init__(self, spec: KernelSpec):
        from . import hip  # the backend; imported lazily so grammar-only use needs no GPU

        self.spec = spec
        for field_name, what in (("native_call", "binds a captured Metal ABI"),
                                 ("atomic_outputs", "asks for Metal atomic outputs")):
            if getattr(spec, field_name) not in (None, False):
                raise ValueError(f"kernel {spec.kernel_id}: {field_name} {what}; the HIP "
                                 "backend runs its own entry points only")
        self._stages = None
        self._entry = None
        self._sequence = None
        if spec.reference_sequence is not None:
            if spec.stages:
                raise ValueError(f"kernel {spec.kernel_id}: a staged region cannot also "
                                 "replay an original sequence")
            from .original_sequence import prepare_sequence
            self._sequence = prepare_sequence(spec.reference_sequence)
        elif spec.stages:
            from .stages import wiring
            reads, self._stage_outputs = wiring(spec)
            self._stages = [(LoadedKernel(st.kernel), pos) for st, pos in zip(spec.stages, reads)]
        else:
            self._entry = hip.binding(spec.source)  # unknown entry -> RuntimeError (a build error)
        self._fallback = Expr(spec.fallback_predicate) if spec.fallback_predicate else None
        self._grid = [Expr(e) for e in spec.grid]
        self._tg = [Expr(e) for e in spec.threadgroup]
        self._out_shapes = [[Expr(e) for e in shape] for shape in spec.output_shapes]
        self._out_dtypes = [_DTYPES[d] for d in spec.output_dtypes]
        self._launches: OrderedDict[tuple, Launch] = OrderedDict()

    def _uncovered(self, inputs, shapes, checked_elsewhere: bool) -> bool:
        """True when the original ops must take this call. Decided before any
        launch expression is evaluated: grid arithmetic may be undefined on
        the shapes the predicate excludes."""
        spec = self.spec
        if not checked_elsewhere and (spec.input_signature is not None
                                      or spec.input_signatures is not None):
            sig = _signature(inputs)
            if spec.input_signature is not None and sig != spec.input_signature:
                return True
            if spec.input_signatures is not None and sig not in spec.input_signatures:
                return True
        return self._fallback is not None and bool(self._fallback.evaluate(shapes))

    def _resolve(self, inputs, shapes, checked_elsewhere: bool) -> Launch:
        if self._uncovered(inputs, shapes, checked_elsewhere):
            return Launch(fallback=True)
        ev = lambda exprs: tuple(int(e.evaluate(shapes)) for e in exprs)  # noqa: E731
        grid, tg = ev(self._grid), ev(self._tg)
        if min(grid + tg) <= 0:
            raise ValueError(f"kernel {self.spec.kernel_id}: non-positive launch {grid} {tg}")
        out_shapes = tuple(ev(s) for s in self._out_shapes)
        if self._stages is not None:
            from .stages import shapes as stage_shapes
            _, results = stage_shapes(self.spec, shapes, [dtype_name(a.dtype) for a in inputs])
            if results != list(zip(out_shapes, self.spec.output_dtypes)):
                raise ValueError(f"kernel {self.spec.kernel_id}: the stages produce {results}, "
                                 "not the region's declared output shapes/dtypes")
        scalars = tuple((name, _template_value(v, inputs)) for name, v in self.spec.template)
        return Launch(False, out_shapes, grid, tg, scalars)

    def launch(self, inputs: list[torch.Tensor], checked_elsewhere: bool = False) -> Launch:
        """The launch for these inputs' shapes and dtypes, resolved once per
        signature. ``checked_elsewhere``: a size-generic caller that serves
        only sizes this kernel was checked at; recorded signatures then do not
        restrict the call (the fallback predicate still does)."""
        key = (checked_elsewhere,) + tuple((tuple(a.shape), a.dtype) for a in inputs)
        hit = self._launches.get(key)
        if hit is not None:
            self._launches.move_to_end(key)
            return hit
        resolved = self._resolve(inputs, [tuple(a.shape) for a in inputs], checked_elsewhere)
        self._launches[key] = resolved
        while len(self._launches) > LAUNCH_CACHE_MAX:
            self._launches.popitem(last=False)
        return resolved

    def fallback_fires(self, inputs: list[torch.Tensor]) -> bool:
        return self.launch(inputs).fallback

    def _allocate(self, launch: Launch, device, init_value):
        if init_value is None:
            return [torch.empty(s, dtype=d, device=device)
                    for s, d in zip(launch.output_shapes, self._out_dtypes)]
        return [torch.full(s, init_value, dtype=d, device=device)
                for s, d in zip(launch.output_shapes, self._out_dtypes)]

    def __call__(self, inputs: list[torch.Tensor], init_value: float | None = None,
                 launch: Launch | None = None) -> list[torch.Tensor]:
        launch = launch if launch is not None else self.launch(inputs)
        if launch.fallback:
            raise ValueError(f"kernel {self.spec.kernel_id}: the fallback predicate covers "
                             "these shapes; the original ops must run them")
        if self._sequence is not None:
            return self._sequence(inputs)
        if self.spec.ensure_row_contiguous:
            inputs = [a.contiguous() for a in inputs]
        if self._stages is not None:
            table = list(inputs)
            for kernel, pos in self._stages:
                table += kernel([table[j] for j in pos], init_value=init_value)
            return [table[j] for j in self._stage_outputs]
        outputs = self._allocate(launch, inputs[0].device, init_value)
        self._entry(inputs, outputs, dict(launch.template))
        return outputs


_cache: dict[str, LoadedKernel] = {}


def _kernel_for(spec: KernelSpec) -> LoadedKernel:
    """The loaded kernel of ``spec``, rebuilt when a different spec object
    arrives under a known id."""
    lk = _cache.get(spec.kernel_id)
    if lk is None or lk.spec is not spec:
        lk = _cache[spec.kernel_id] = LoadedKernel(spec)
    return lk


def _covered_call(spec, inputs, sized: bool, init_value):
    lk = _kernel_for(spec)
    plan = lk.launch(inputs, checked_elsewhere=sized)
    if plan.fallback:
        return None
    return lk(inputs, init_value=init_value, launch=plan)


def covers_sized(spec: KernelSpec, inputs: list[torch.Tensor]) -> bool:
    """Whether ``try_sized(spec, inputs)`` would launch the region (not decline
    it to the original ops)."""
    return not _kernel_for(spec).launch(inputs, checked_elsewhere=True).fallback


def fallback_fires(spec: KernelSpec, inputs: list[torch.Tensor]) -> bool:
    """Whether the region's original ops must run these inputs."""
    return _kernel_for(spec).fallback_fires(inputs)


def call(spec: KernelSpec, inputs: list[torch.Tensor], init_value: float | None = None,
         launch: Launch | None = None) -> list[torch.Tensor]:
    """Run the region (all its launches) and return its outputs; ValueError on
    shapes the fallback covers."""
    return _kernel_for(spec)(inputs, init_value=init_value, launch=launch)


def try_call(spec: KernelSpec, inputs: list[torch.Tensor]) -> list[torch.Tensor] | None:
    """The region's outputs, or None for shapes (or unrecorded signatures) the
    original ops take."""
    return _covered_call(spec, inputs, False, None)


def try_sized(spec: KernelSpec, inputs: list[torch.Tensor],
              init_value: float | None = None) -> list[torch.Tensor] | None:
    """As ``try_call`` for callers that gate sizes themselves: only the fallback
    predicate can decline the call."""
    return _covered_call(spec, inputs, True, init_value)
