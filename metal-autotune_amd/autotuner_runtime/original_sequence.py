"""Replay of a region's recorded original op sequence (``reference_sequence``).

When no single kernel exists for a region, the reference keeps its original
calls as a correctness-preserving starter: the spec carries the recorded
nodes (op name, argument wiring, scalar arguments) instead of a kernel body
(autotuner/scaffold/native.py:61-118), and ``LoadedKernel`` replays them
(autotuner_runtime/kernels.py:53,125-127,199-200;
autotuner_runtime/original_sequence.py:1-7). The record is MLX's: op names
are ``mx.*`` functions or ``array.*`` methods, array arguments are
``{"$": "ref", "i": k}`` (the node's k-th input array) and the containers,
slices, dtypes and ``Ellipsis`` of the arguments are tagged dicts
(autotuner/trace/serialize.py:16-30,57-71).

On this backend each op name maps to the library op with MLX's meaning
(``autotuner_runtime.ops``: quantized matmul, dequantize, the fast norms,
RoPE and attention) or to the torch function that computes it (elementwise,
shape, reduction ops). The wiring is resolved once into a list of steps; no
code is generated. Refused at load, with ``ValueError``:

* nodes that call a captured Metal kernel (``kernel_definition``);
* mutating methods (``array.__iadd__`` and the like, ``__setitem__``);
* op names outside the table below.

A ``{"variants": [{"signature", "sequence"}, ...]}`` record holds one
sequence per recorded input signature (shapes and dtype names); a call picks
the variant of its inputs' signature.
"""

from __future__ import annotations

import operator
from typing import Any, Callable

import torch

from . import ops
from .swap import flatten_arrays

# -- the op table -------------------------------------------------------------

_TORCH_DTYPES = {
    "bool": torch.bool, "uint8": torch.uint8, "uint16": torch.uint16, "uint32": torch.uint32,
    "uint64": torch.uint64, "int8": torch.int8, "int16": torch.int16, "int32": torch.int32,
    "int64": torch.int64, "float16": torch.float16, "bfloat16": torch.bfloat16,
    "float32": torch.float32,
}


def _axes(*axes):
    """MLX methods take axes as varargs or as one sequence."""
    if len(axes) == 1 and isinstance(axes[0], (list, tuple)):
        return tuple(axes[0])
    return tuple(axes)


def _transpose(a, axes=None):
    return a.permute(tuple(reversed(range(a.dim()))) if axes is None else tuple(axes))


def _split(a, indices_or_sections, axis=0):
    if isinstance(indices_or_sections, int):
        if a.shape[axis] % indices_or_sections:
            raise ValueError(f"split: axis of size {a.shape[axis]} is not divisible into "
                             f"{indices_or_sections} equal sections")
    return tuple(torch.tensor_split(a, indices_or_sections, dim=axis))


def _expand_dims(a, axis):
    for ax in sorted(axis if isinstance(axis, (list, tuple)) else [axis]):
        a = a.unsqueeze(ax)
    return a


def _squeeze(a, axis=None):
    if axis is None:
        return a.squeeze()
    for ax in sorted(axis if isinstance(axis, (list, tuple)) else [axis], reverse=True):
        a = a.squeeze(ax)
    return a


def _reduction(fn: Callable) -> Callable:
    def reduce(a, axis=None, keepdims=False):
        if axis is None:
            axis = tuple(range(a.dim()))
        return fn(a, dim=axis, keepdim=keepdims)
    return reduce


def _argmax(a, axis=None, keepdims=False):
    if axis is None:
        return torch.argmax(a.reshape(-1)).to(torch.uint32)
    return torch.argmax(a, dim=axis, keepdim=keepdims).to(torch.uint32)


def _softmax(a, axis=None, precise=False):
    if axis is None:
        return torch.softmax(a.reshape(-1), dim=0).reshape(a.shape)
    if isinstance(axis, (list, tuple)):
        if len(axis) != 1:
            raise ValueError("softmax over several axes is not replayed")
        axis = axis[0]
    return torch.softmax(a.float() if precise else a, dim=axis).to(a.dtype)


def _matmul(a, b):
    # a transposed right operand goes through a copy: batched bf16 products
    # on a transposed view are avoided on this platform
    return torch.matmul(a, b.contiguous())


def _rms_norm(x, weight, eps):
    return ops.rms_norm(x, weight, eps)


def _rope(x, dims, *, traditional=False, base=10000.0, scale=1.0, offset=0, freqs=None):
    if freqs is not None:
        raise ValueError("mx.fast.rope with explicit freqs is not replayed")
    return ops.rope(x, dims, traditional, base, scale, int(offset))


def _sdpa(q, k, v, *, scale, mask=None, sinks=None):
    if sinks is not None or not (mask is None or isinstance(mask, str)):
        raise ValueError("sdpa with an array mask or sinks is not replayed")
    return ops.scaled_dot_product_attention(q, k, v, scale, mask)


def _qmm(x, w, scales, biases=None, transpose=True, group_size=64, bits=4, mode="affine"):
    if mode != "affine" or biases is None:
        raise ValueError(f"quantized_matmul mode {mode!r} is not replayed (affine only)")
    return ops.quantized_matmul(x, w, scales, biases, transpose, group_size, bits)


def _dequantize(w, scales, biases=None, group_size=64, bits=4, mode="affine"):
    if mode != "affine" or biases is None:
        raise ValueError(f"dequantize mode {mode!r} is not replayed (affine only)")
    return ops.dequantize(w, scales, biases, group_size, bits)


def _rsub(a, b):
    return b - a


def _rdiv(a, b):
    return b / a


def _rpow(a, b):
    return b ** a


_OPS: dict[str, Callable] = {
    # library ops with MLX's argument meaning
    "mx.quantized_matmul": _qmm,
    "mx.dequantize": _dequantize,
    "mx.fast.rms_norm": _rms_norm,
    "mx.fast.rope": _rope,
    "mx.fast.scaled_dot_product_attention": _sdpa,
    # elementwise
    "mx.add": torch.add, "mx.subtract": torch.sub, "mx.multiply": torch.mul,
    "mx.divide": torch.div, "mx.maximum": torch.maximum, "mx.minimum": torch.minimum,
    "mx.power": torch.pow, "mx.where": torch.where,
    "mx.negative": torch.neg, "mx.abs": torch.abs, "mx.exp": torch.exp, "mx.log": torch.log,
    "mx.sqrt": torch.sqrt, "mx.rsqrt": torch.rsqrt, "mx.square": torch.square,
    "mx.sigmoid": torch.sigmoid, "mx.tanh": torch.tanh, "mx.erf": torch.erf,
    "mx.sin": torch.sin, "mx.cos": torch.cos,
    "array.__add__": operator.add, "array.__radd__": operator.add,
    "array.__sub__": operator.sub, "array.__rsub__": _rsub,
    "array.__mul__": operator.mul, "array.__rmul__": operator.mul,
    "array.__truediv__": operator.truediv, "array.__rtruediv__": _rdiv,
    "array.__pow__": operator.pow, "array.__rpow__": _rpow,
    "array.__neg__": operator.neg, "array.__abs__": operator.abs,
    "array.__invert__": operator.invert,
    "array.__lt__": operator.lt, "array.__le__": operator.le, "array.__gt__": operator.gt,
    "array.__ge__": operator.ge, "array.__eq__": operator.eq, "array.__ne__": operator.ne,
    # products
    "mx.matmul": _matmul, "array.__matmul__": _matmul,
    # shapes
    "mx.reshape": lambda a, shape: a.reshape(tuple(shape)),
    "array.reshape": lambda a, *shape: a.reshape(_axes(*shape)),
    "mx.transpose": _transpose,
    "array.transpose": lambda a, *axes: _transpose(a, _axes(*axes) if axes else None),
    "array.T": lambda a: _transpose(a),
    "mx.swapaxes": lambda a, axis1, axis2: a.transpose(axis1, axis2),
    "array.swapaxes": lambda a, axis1, axis2: a.transpose(axis1, axis2),
    "mx.split": _split, "array.split": _split,
    "mx.concatenate": lambda arrays, axis=0: torch.cat(list(arrays), dim=axis),
    "mx.stack": lambda arrays, axis=0: torch.stack(list(arrays), dim=axis),
    "mx.expand_dims": _expand_dims, "mx.squeeze": _squeeze, "array.squeeze": _squeeze,
    "mx.flatten": lambda a, start_axis=0, end_axis=-1: a.flatten(start_axis, end_axis),
    "mx.contiguous": lambda a, allow_col_major=False: a.contiguous(),
    "array.__getitem__": operator.getitem,
    "mx.astype": lambda a, dtype: a.to(dtype), "array.astype": lambda a, dtype: a.to(dtype),
    # reductions
    "mx.sum": _reduction(torch.sum), "array.sum": _reduction(torch.sum),
    "mx.mean": _reduction(torch.mean), "array.mean": _reduction(torch.mean),
    "mx.max": _reduction(torch.amax), "array.max": _reduction(torch.amax),
    "mx.min": _reduction(torch.amin), "array.min": _reduction(torch.amin),
    "mx.argmax": _argmax, "array.argmax": _argmax,
    "mx.softmax": _softmax,
}

# array methods that write into their receiver: never a fusion starter
_MUTATING = frozenset({
    "__setitem__", "__iadd__", "__isub__", "__imul__", "__itruediv__", "__ifloordiv__",
    "__imod__", "__ipow__", "__imatmul__", "__iand__", "__ior__", "__ixor__", "__ilshift__",
    "__irshift__",
})


def resolve(op: str) -> Callable:
    """The callable replaying MLX op ``op``; ValueError when it cannot be."""
    if op.startswith("array.") and op.removeprefix("array.") in _MUTATING:
        raise ValueError(f"mutating operation {op} is not a fusion starter")
    fn = _OPS.get(op)
    if fn is None:
        raise ValueError(f"operation {op} cannot be replayed on the HIP backend")
    return fn


# -- argument wiring ----------------------------------------------------------

class _Input:
    """Placeholder for a node's k-th input array inside its arguments."""

    __slots__ = ("k",)

    def __init__(self, k: int):
        self.k = k


def _decode(value: Any, n_in: int) -> tuple[Any, bool]:
    """(decoded value, whether it holds input placeholders)."""
    if not (isinstance(value, dict) and "$" in value):
        return value, False
    tag = value["$"]
    if tag == "ref":
        k = value["i"]
        if not 0 <= k < n_in:
            raise ValueError(f"argument refers to input {k} of a node with {n_in}")
        return _Input(k), True
    if tag in ("tuple", "list"):
        items = [_decode(v, n_in) for v in value["items"]]
        seq = [v for v, _ in items]
        return (tuple(seq) if tag == "tuple" else seq), any(r for _, r in items)
    if tag == "dict":
        items = {k: _decode(v, n_in) for k, v in value["items"].items()}
        return {k: v for k, (v, _) in items.items()}, any(r for _, r in items.values())
    if tag == "slice":
        parts = [_decode(v, n_in) for v in value["parts"]]
        if any(r for _, r in parts):
            raise ValueError("a slice bound that is an array is not replayed")
        return slice(*(v for v, _ in parts)), False
    if tag == "dtype":
        name = value["name"]
        if name not in _TORCH_DTYPES:
            raise ValueError(f"dtype {name!r} has no torch counterpart here")
        return _TORCH_DTYPES[name], False
    if tag == "ellipsis":
        return Ellipsis, False
    raise ValueError(f"unsupported recorded argument {tag!r}")


def _bind(value: Any, arrays: list[torch.Tensor]) -> Any:
    if isinstance(value, _Input):
        return arrays[value.k]
    if isinstance(value, tuple):
        return tuple(_bind(v, arrays) for v in value)
    if isinstance(value, list):
        return [_bind(v, arrays) for v in value]
    if isinstance(value, dict):
        return {k: _bind(v, arrays) for k, v in value.items()}
    return value


class _Step:
    """One recorded call: its function, argument templates and wiring."""

    __slots__ = ("op", "fn", "args", "kwargs", "live", "reads", "writes")

    def __init__(self, node: dict):
        self.op = node["op"]
        if node.get("kernel_definition") is not None:
            raise ValueError(f"node {self.op}: a captured Metal kernel cannot run on the HIP "
                             "backend")
        self.fn = resolve(self.op)
        self.reads = list(node["in_arrays"])
        self.writes = list(node["out_arrays"])
        n_in = len(self.reads)
        raw = node["args"]  # an encoded tuple (or a plain list of encoded values)
        if isinstance(raw, list):
            raw = {"$": "tuple", "items": raw}
        self.args, ra = _decode(raw, n_in)
        if not isinstance(self.args, tuple):
            raise ValueError(f"node {self.op}: positional arguments must be a tuple")
        self.kwargs, rk = _decode({"$": "dict", "items": node.get("kwargs", {})}, n_in)
        self.live = ra or rk

    def run(self, values: dict) -> None:
        arrays = [values[a] for a in self.reads]
        args = _bind(self.args, arrays) if self.live else self.args
        kwargs = _bind(self.kwargs, arrays) if self.live else self.kwargs
        result = self.fn(*args, **kwargs)
        got = flatten_arrays(result)
        if len(got) != len(self.writes):
            raise ValueError(f"node {self.op}: {len(got)} output arrays where the record has "
                             f"{len(self.writes)}")
        values.update(zip(self.writes, got))


def _signature(inputs: list[torch.Tensor]) -> tuple:
    names = {v: k for k, v in _TORCH_DTYPES.items()}
    return tuple((tuple(a.shape), names.get(a.dtype, str(a.dtype))) for a in inputs)


def prepare_sequence(sequence: dict) -> Callable[[list[torch.Tensor]], list[torch.Tensor]]:
    """A function replaying the record on torch tensors: inputs in the
    record's ``input_ids`` order, outputs in its ``output_ids`` order."""
    if "variants" in sequence:
        table = {}
        for variant in sequence["variants"]:
            key = tuple((tuple(shape), dtype) for shape, dtype in variant["signature"])
            table[key] = prepare_sequence(variant["sequence"])

        def run_variant(inputs: list[torch.Tensor]) -> list[torch.Tensor]:
            fn = table.get(_signature(inputs))
            if fn is None:
                raise ValueError(f"no recorded variant for input signature {_signature(inputs)}")
            return fn(inputs)

        return run_variant

    missing = [k for k in ("nodes", "input_ids", "output_ids") if k not in sequence]
    if missing:
        raise ValueError(f"a recorded sequence needs {missing}")
    input_ids = list(sequence["input_ids"])
    output_ids = list(sequence["output_ids"])
    steps = [_Step(node) for node in sequence["nodes"]]
    known = set(input_ids)
    for step in steps:
        missing = [a for a in step.reads if a not in known]
        if missing:
            raise ValueError(f"node {step.op} reads arrays {missing} that no earlier node or "
                             "input provides")
        known.update(step.writes)
    if any(a not in known for a in output_ids):
        raise ValueError("the record's outputs are not all produced")

    def run(inputs: list[torch.Tensor]) -> list[torch.Tensor]:
        if len(inputs) != len(input_ids):
            raise ValueError(f"the sequence takes {len(input_ids)} inputs, got {len(inputs)}")
        values = dict(zip(input_ids, inputs))
        for step in steps:
            step.run(values)
        return [values[a] for a in output_ids]

    return run
