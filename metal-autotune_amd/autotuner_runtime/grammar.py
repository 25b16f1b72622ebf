"""The launch grammar: integer/boolean expressions over a call's input shapes.

Mirrors the reference's contract (autotuner_runtime/grammar.py:1-64): grid,
threadgroup, output shapes and fallback predicates are expressions in which
the only names are inputs ``in0, in1, ...`` with ``.shape[i]`` and ``.ndim``;
the only calls are ``min``, ``max`` and ``ceil_div`` with two positional
arguments; operators are ``+ - * // % /`` (``/`` is integer division),
single comparisons, ``and/or/not`` and unary minus; literals are ints and
bools. Anything else raises :class:`GrammarError` (a ``ValueError``) at parse
time; an input or axis out of range raises it at evaluation time.

Expressions are parsed once with :mod:`ast` and compiled into a tree of
closures; nothing is ever passed to ``eval``.
"""

from __future__ import annotations

import ast
import operator
from typing import Callable, Sequence

Shapes = Sequence[Sequence[int]]


class GrammarError(ValueError):
    """The expression is outside the launch grammar; the message says where."""


def _int_div(a, b):
    return a // b


def _ceil_div(a, b):
    return -((-a) // b)


_ARITH = {
    ast.Add: operator.add,
    ast.Sub: operator.sub,
    ast.Mult: operator.mul,
    ast.FloorDiv: _int_div,
    ast.Div: _int_div,
    ast.Mod: operator.mod,
}
_COMPARE = {
    ast.Lt: operator.lt,
    ast.LtE: operator.le,
    ast.Gt: operator.gt,
    ast.GtE: operator.ge,
    ast.Eq: operator.eq,
    ast.NotEq: operator.ne,
}
_CALLS = {"min": min, "max": max, "ceil_div": _ceil_div}

Node = Callable[[Shapes], "int | bool"]


class Expr:
    """A parsed expression; ``evaluate(shapes)`` with shapes[i] = input i's shape."""

    def __init__(self, text: str):
        self.text = text
        try:
            tree = ast.parse(text, mode="eval").body
        except (SyntaxError, ValueError, RecursionError, MemoryError) as e:
            raise GrammarError(f"cannot parse {text!r}: {type(e).__name__}: {e}") from None
        try:
            self._fn = self._build(tree)
        except RecursionError:
            raise GrammarError(f"{text!r}: expression nests too deeply") from None

    def evaluate(self, shapes: Shapes) -> int | bool:
        return self._fn(shapes)

    def __repr__(self) -> str:
        return f"Expr({self.text!r})"

    # -- compilation -------------------------------------------------------

    def _err(self, why: str) -> GrammarError:
        return GrammarError(f"{self.text!r}: {why}")

    def _build(self, node: ast.AST) -> Node:
        if isinstance(node, ast.Constant):
            value = node.value
            if type(value) not in (int, bool):
                raise self._err("only integer and boolean literals")
            return lambda shapes: value
        if isinstance(node, ast.BinOp):
            op = _ARITH.get(type(node.op))
            if op is None:
                raise self._err(f"operator {type(node.op).__name__} is outside the grammar")
            left, right = self._build(node.left), self._build(node.right)
            return lambda shapes: op(left(shapes), right(shapes))
        if isinstance(node, ast.UnaryOp):
            inner = self._build(node.operand)
            if isinstance(node.op, ast.USub):
                return lambda shapes: -inner(shapes)
            if isinstance(node.op, ast.Not):
                return lambda shapes: not inner(shapes)
            raise self._err(f"unary {type(node.op).__name__} is outside the grammar")
        if isinstance(node, ast.Compare):
            if len(node.ops) != 1:
                raise self._err("only single binary comparisons")
            op = _COMPARE.get(type(node.ops[0]))
            if op is None:
                raise self._err("only single binary comparisons")
            left, right = self._build(node.left), self._build(node.comparators[0])
            return lambda shapes: op(left(shapes), right(shapes))
        if isinstance(node, ast.BoolOp):
            parts = [self._build(v) for v in node.values]
            if isinstance(node.op, ast.And):
                return lambda shapes: all(p(shapes) for p in parts)
            return lambda shapes: any(p(shapes) for p in parts)
        if isinstance(node, ast.Call):
            if not isinstance(node.func, ast.Name) or node.func.id not in _CALLS:
                raise self._err("only min/max/ceil_div calls")
            if node.keywords or len(node.args) != 2:
                raise self._err("grammar calls take exactly two positional args")
            fn = _CALLS[node.func.id]
            a, b = (self._build(x) for x in node.args)
            return lambda shapes: fn(a(shapes), b(shapes))
        if isinstance(node, ast.Attribute):
            if node.attr != "ndim":
                raise self._err("only .ndim and .shape[i] accessors")
            idx = self._input(node.value)
            return lambda shapes: len(self._shape(shapes, idx))
        if isinstance(node, ast.Subscript):
            base = node.value
            if not (isinstance(base, ast.Attribute) and base.attr == "shape"):
                raise self._err("only .shape[i] subscripts")
            idx = self._input(base.value)
            axis = self._build(node.slice)

            def dim(shapes, idx=idx, axis=axis):
                shape = self._shape(shapes, idx)
                a = axis(shapes)
                try:
                    return shape[a]
                except (IndexError, TypeError):
                    raise self._err(f"axis {a} out of range for input {idx} with shape "
                                    f"{tuple(shape)}") from None
            return dim
        raise self._err(f"{type(node).__name__} is outside the launch grammar")

    def _input(self, node: ast.AST) -> int:
        if isinstance(node, ast.Name) and node.id.startswith("in") and node.id[2:].isdigit():
            return int(node.id[2:])
        raise self._err("inputs are named in0, in1, ...")

    def _shape(self, shapes: Shapes, idx: int):
        if idx >= len(shapes):
            raise self._err(f"input {idx} out of range, call has {len(shapes)} inputs")
        return shapes[idx]
