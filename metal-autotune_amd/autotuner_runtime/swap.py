"""Module swap on live torch models (the reference's swap.py:1-152).

Scope addresses are dot paths, used for serialization only: the swap always
happens on live instances by parent attribute assignment, or index/key
assignment for children in ``nn.ModuleList`` / lists / dicts. Wrappers are
``nn.Module`` subclasses so the wrapped subtree stays visible to
``parameters()`` and ``named_modules()``; attribute lookups a wrapper does not
define fall through to the wrapped module.
"""

from __future__ import annotations

import torch
from torch import nn


def flatten_arrays(tree: object) -> list[torch.Tensor]:
    """Every tensor of a nested list/tuple/dict tree, in order (iterative walk)."""
    out: list[torch.Tensor] = []
    stack = [tree]
    while stack:
        obj = stack.pop()
        if isinstance(obj, torch.Tensor):
            out.append(obj)
        elif isinstance(obj, (list, tuple)):
            stack.extend(reversed(obj))
        elif isinstance(obj, dict):
            stack.extend(reversed(list(obj.values())))
    return out


def state_signature(value):
    """Structure, scalar settings and tensor shapes of a state object, never its
    data: guards replays whose control flow depended on a cache's layout."""
    seen: dict[int, int] = {}

    def visit(obj):
        if isinstance(obj, torch.Tensor):
            return ("array", tuple(obj.shape), str(obj.dtype).replace("torch.", ""))
        if obj is None or isinstance(obj, (str, int, float, bool)):
            return obj
        if id(obj) in seen:
            return ("alias", seen[id(obj)])
        seen[id(obj)] = len(seen)
        if isinstance(obj, dict):
            return ("dict", tuple((k, visit(v)) for k, v in sorted(obj.items())))
        if isinstance(obj, (tuple, list)):
            return (type(obj).__name__, tuple(visit(v) for v in obj))
        if hasattr(obj, "__dict__"):
            return (type(obj).__name__, visit(vars(obj)))
        raise TypeError(f"cannot describe state field of type {type(obj).__name__}")

    return visit(value)


class ReplayWrapper(nn.Module):
    """Base for region wrappers: subclasses implement forward as the scope's
    op stream with the shipped regions spliced in via kernels.try_sized."""

    def __init__(self, wrapped: nn.Module, specs: dict | None = None):
        super().__init__()
        self.wrapped = wrapped
        object.__setattr__(self, "_specs", dict(specs or {}))

    def __getattr__(self, name):
        try:
            return super().__getattr__(name)
        except AttributeError:
            modules = self.__dict__.get("_modules", {})
            if "wrapped" not in modules:
                raise
            return getattr(modules["wrapped"], name)


def require_independent_models(first, second) -> None:
    """Weight tensors may be shared; mutable modules must belong to one arm."""
    if not isinstance(first, nn.Module) or not isinstance(second, nn.Module):
        return
    originals = {id(m) for m in first.modules()}
    for path, module in second.named_modules():
        if id(module) in originals:
            raise ValueError(
                f"build() reused a model module at {path or '<root>'}; return fresh model "
                "and layer instances on every call so installing a kernel cannot modify "
                "the untouched baseline. Weight arrays may be shared.")


def _child(obj: object, key: str, full_path: str):
    try:
        if isinstance(obj, (list, tuple, nn.ModuleList, nn.Sequential)):
            return obj[int(key)]
        if isinstance(obj, nn.ModuleDict):
            return obj[key]
        if isinstance(obj, dict):
            return obj[key]
        return getattr(obj, key)
    except (AttributeError, KeyError, IndexError, ValueError, TypeError) as e:
        raise KeyError(
            f"cannot resolve scope address {full_path!r}: no child {key!r} on "
            f"{type(obj).__name__} ({e}); the model tree changed since the trace") from None


def resolve(model: object, path: str):
    """path -> (container, key, child). The empty path (the model itself) has no
    parent; installing there is the caller's special case."""
    if path == "":
        raise ValueError("the root scope has no parent to swap under")
    parts = path.split(".")
    obj = model
    for part in parts[:-1]:
        obj = _child(obj, part, path)
    return obj, parts[-1], _child(obj, parts[-1], path)


def resolve_value(model: object, path: str):
    """Resolve a recorded weight or state through modules, dicts and sequences."""
    obj = model
    for part in path.split(".") if path else []:
        obj = _child(obj, part, path)
    return obj


def _assign(parent: object, key: str, value: object) -> None:
    if isinstance(parent, (list, nn.ModuleList, nn.Sequential)):
        parent[int(key)] = value
    elif isinstance(parent, (dict, nn.ModuleDict)):
        parent[key] = value
    elif isinstance(parent, tuple):
        raise TypeError("cannot swap a child living in a tuple; the model must use lists")
    else:
        setattr(parent, key, value)


def install(model: object, path: str, wrapper: nn.Module) -> object:
    """Swap ``wrapper`` in at ``path``; returns the previous occupant for rollback."""
    parent, key, occupant = resolve(model, path)
    _assign(parent, key, wrapper)
    return occupant


def uninstall(model: object, path: str, occupant: object) -> None:
    parent, key, _ = resolve(model, path)
    _assign(parent, key, occupant)
