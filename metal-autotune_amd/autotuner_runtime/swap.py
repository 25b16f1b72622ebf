"""Installing region wrappers into live torch models.

The drop-in interface of the reference's autotuner_runtime/swap.py (install,
uninstall, resolve, ReplayWrapper; swap.py:67-152): an artifact's swap table
names each wrapped scope by a dot path (``model.layers.3.mlp``), and apply()
puts a wrapper instance in that place. The walk here is this build's own:

* a path is split once into steps; each step is an attribute name, a
  ``nn.ModuleList`` / list position, or a ``nn.ModuleDict`` / dict key,
  decided by the container's type (``_Step``);
* ``install`` returns what was there, and ``uninstall`` puts it back, so a
  caller can roll a swap back;
* wrappers are ``nn.Module`` subclasses holding the original as ``wrapped``,
  so ``parameters()`` still reaches the original weights, and attribute
  reads the wrapper does not answer go to the original.
"""

from __future__ import annotations

from typing import Any, Iterator

import torch
from torch import nn

_INDEXED = (list, tuple, nn.ModuleList, nn.Sequential)
_KEYED = (dict, nn.ModuleDict)


class _Step:
    """One component of a scope path, bound to the object it is taken from."""

    __slots__ = ("owner", "name")

    def __init__(self, owner: Any, name: str):
        self.owner, self.name = owner, name

    def get(self) -> Any:
        o = self.owner
        if isinstance(o, _INDEXED):
            return o[int(self.name)]
        if isinstance(o, _KEYED):
            return o[self.name]
        return getattr(o, self.name)

    def put(self, value: Any) -> None:
        o = self.owner
        if isinstance(o, tuple):
            raise TypeError(f"scope step {self.name!r} lives in a tuple, which cannot be "
                            "assigned; hold swappable children in a list or ModuleList")
        if isinstance(o, _INDEXED):
            o[int(self.name)] = value
        elif isinstance(o, _KEYED):
            o[self.name] = value
        else:
            setattr(o, self.name, value)


def _walk(model: Any, path: str) -> _Step:
    """The last step of ``path`` under ``model``; every step before it resolved."""
    if not path:
        raise ValueError("an empty scope path is the model itself; there is no parent "
                         "to install a wrapper under")
    names = path.split(".")
    node = model
    for depth, name in enumerate(names):
        step = _Step(node, name)
        try:
            child = step.get()
        except (AttributeError, KeyError, IndexError, ValueError, TypeError) as err:
            where = ".".join(names[:depth]) or "<model>"
            raise KeyError(f"cannot resolve scope {path!r}: {type(node).__name__} at {where} "
                           f"has no child {name!r} ({err})") from None
        if depth == len(names) - 1:
            return step
        node = child
    raise AssertionError("unreachable")


def resolve(model: Any, path: str) -> tuple[Any, str, Any]:
    """(parent container, last path component, current occupant) of ``path``."""
    step = _walk(model, path)
    return step.owner, step.name, step.get()


def install(model: Any, path: str, wrapper: nn.Module) -> Any:
    """Put ``wrapper`` at ``path``; returns the previous occupant."""
    step = _walk(model, path)
    previous = step.get()
    step.put(wrapper)
    return previous


def uninstall(model: Any, path: str, occupant: Any) -> None:
    """Undo ``install``: ``occupant`` (what install returned) goes back."""
    _walk(model, path).put(occupant)


def _iter_tensors(tree: Any) -> Iterator[torch.Tensor]:
    if isinstance(tree, torch.Tensor):
        yield tree
    elif isinstance(tree, dict):
        for v in tree.values():
            yield from _iter_tensors(v)
    elif isinstance(tree, (list, tuple)):
        for v in tree:
            yield from _iter_tensors(v)


def flatten_arrays(tree: Any) -> list[torch.Tensor]:
    """The tensors of a (nested) list / tuple / dict result, depth first in
    container order; anything else in the tree is skipped."""
    return list(_iter_tensors(tree))


def require_independent_models(first: Any, second: Any) -> None:
    """Two arms of a comparison may share weight tensors but not modules: a
    wrapper installed into one arm must leave the other untouched."""
    if not (isinstance(first, nn.Module) and isinstance(second, nn.Module)):
        return
    owned = {id(m): name for name, m in first.named_modules()}
    shared = [(name or "<root>") for name, m in second.named_modules() if id(m) in owned]
    if shared:
        raise ValueError(f"the model builder reused module instance(s) {shared[:3]} across "
                         "both arms; build fresh modules per arm (weight tensors may be shared)")


class ReplayWrapper(nn.Module):
    """Base class of region wrappers. A subclass's ``forward`` is the scope's
    op sequence with region kernels called through ``kernels.try_sized`` and
    the original ops kept for shapes a kernel does not cover. ``_specs`` maps
    kernel ids to their specs."""

    def __init__(self, wrapped: nn.Module, specs: dict | None = None):
        super().__init__()
        self.wrapped = wrapped
        # a plain attribute, kept out of nn.Module's registries
        self.__dict__["_specs"] = dict(specs or {})

    def __getattr__(self, name: str):
        try:
            return super().__getattr__(name)
        except AttributeError:
            inner = self.__dict__.get("_modules", {}).get("wrapped")
            if inner is None:
                raise
            return getattr(inner, name)
