"""Graph-level delivery: a scope captured as one HIP graph per call signature.

The reference compiles a scope's original MLX graph with the certified
substitutions and reuses the compiled call for every warm call of the same
signature (autotuner_runtime/graph.py:1-27, GraphWrapper at :306). Cache
state goes in and comes out explicitly, plain attributes such as an offset
are part of the signature, and an unrecorded state is traced as its own
signature up to a limit (UNRECORDED_STATE_TRACES) before the original module
runs untouched.

On MI355X the scope's launches (region kernels and original ops alike) are
captured into a HIP graph (``torch.cuda.CUDAGraph``) the first time a
signature is seen and replayed afterwards: one graph launch instead of every
kernel's host-side dispatch.

- The signature of a call: each tensor argument's shape/dtype/device; each
  state holder (an object whose attributes hold tensors or plain values,
  e.g. a KV cache with its offset) by its attributes: plain values by value,
  tensors by shape/dtype and storage address (the graph writes into them in
  place, so the same buffers must come back).
- First call of a signature: the holders' attributes are saved, the scope
  runs once eagerly (library loading and allocation happen outside capture),
  the attributes are restored, the call is captured with its tensor
  arguments copied into static buffers, and the graph is replayed once.
  Attribute writes the scope made during capture (a new conv state tensor,
  a moved offset) are recorded.
- Warm call: the tensor arguments are copied into the static buffers, the
  graph replays, the recorded attribute writes are applied again, and the
  static outputs are returned. They stay valid until the next call of the
  same signature (the graph overwrites them), as with any graph replay.
- Carried state: an attribute the scope assigns a new tensor to (an LFM2
  conv state) is handed to the holder as its own copy on every replay, so
  two holders that replay one graph never share a state tensor. When such a
  state comes back in on a later call it is keyed by shape and dtype (not by
  storage) and copied into a static buffer the graph reads, so a chunked
  prefill or decode loop replays one graph instead of capturing per call.
- Beyond ``max_graphs`` signatures the original module runs eagerly.

Streams: capture and replay run on the caller's current stream. Graphs hold
no ``hipMemsetAsync`` nodes: every library kernel writes its outputs in full.
Each graph is captured inside its own ``hip.graph_workspaces()`` scope, so the
scratch buffers its kernels address (K-part sums, MLP tickets) belong to it
alone: two graphs replayed side by side on different streams never share one.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch
from torch import nn

MAX_GRAPHS = 8  # signatures captured per wrapper before calls run eagerly


def _is_holder(v) -> bool:
    return hasattr(v, "__dict__") and not isinstance(v, (nn.Module, torch.Tensor, type))


def _attr_sig(v, carried: bool):
    if isinstance(v, torch.Tensor):
        if carried:  # fed through a static buffer: only its layout matters
            return ("c", tuple(v.shape), str(v.dtype), str(v.device))
        # read or written in place by the graph: the same storage must come back
        return ("t", tuple(v.shape), str(v.dtype), str(v.device), v.data_ptr())
    if v is None or isinstance(v, (bool, int, float, str)):
        return ("v", v)
    return ("o", type(v).__name__)


def signature(args, carried=frozenset()) -> tuple:
    """The capture key of a call. ``carried``: (holder type name, attribute)
    pairs that a scope assigns a fresh tensor to (state handed from call to
    call, such as a conv state); those are keyed by layout, not storage."""
    sig = []
    for a in args:
        if isinstance(a, torch.Tensor):
            sig.append(("T", tuple(a.shape), str(a.dtype), str(a.device)))
        elif _is_holder(a):
            name = type(a).__name__
            sig.append(("H", name, tuple(sorted(
                (k, _attr_sig(v, (name, k) in carried)) for k, v in vars(a).items()))))
        elif isinstance(a, (list, tuple)):
            sig.append(("L", signature(a, carried)))
        else:
            sig.append(("V", a))
    return tuple(sig)


def _holders(args) -> list:
    out = []
    for a in args:
        if _is_holder(a):
            out.append(a)
        elif isinstance(a, (list, tuple)):
            out.extend(_holders(a))
    return out


@dataclass
class _Entry:
    graph: torch.cuda.CUDAGraph
    static_args: list
    outputs: object
    feeds: list = field(default_factory=list)   # (holder index, attribute, static tensor)
    writes: list = field(default_factory=list)  # (holder index, attribute, value)


class GraphWrapper(nn.Module):
    """Wraps a module (a layer, or a whole model step) so each call signature
    runs as one replayed HIP graph. ``stats`` counts captures, replays and
    eager calls."""

    def __init__(self, wrapped: nn.Module, max_graphs: int = MAX_GRAPHS):
        super().__init__()
        self.wrapped = wrapped
        self.max_graphs = max_graphs
        object.__setattr__(self, "_graphs", {})
        object.__setattr__(self, "_carried", set())
        object.__setattr__(self, "stats", {"captures": 0, "replays": 0, "eager": 0})

    def forward(self, *args):
        if not any(isinstance(a, torch.Tensor) and a.is_cuda for a in args):
            return self.wrapped(*args)
        key = signature(args, frozenset(self._carried))
        entry = self._graphs.get(key)
        if entry is None:
            if len(self._graphs) >= self.max_graphs:
                self.stats["eager"] += 1
                return self.wrapped(*args)
            entry = self._capture(args)
            self._graphs[key] = entry
            self.stats["captures"] += 1
        else:
            self.stats["replays"] += 1
        self._replay(entry, args)
        return entry.outputs

    @staticmethod
    def _replay(entry: _Entry, args) -> None:
        """Feed the call's tensors and carried state into the graph's static
        buffers, replay, then hand each holder its own copy of every tensor
        the scope assigned (the graph reuses its buffers on the next replay,
        and other holders may replay the same graph)."""
        for static, a in zip(entry.static_args, args):
            if isinstance(a, torch.Tensor) and static is not a:
                static.copy_(a)
        holders = _holders(args)
        for i, name, static in entry.feeds:
            static.copy_(getattr(holders[i], name))
        entry.graph.replay()
        for i, name, value in entry.writes:
            setattr(holders[i], name, value.clone() if isinstance(value, torch.Tensor) else value)

    def _capture(self, args) -> _Entry:
        holders = _holders(args)
        before = [dict(vars(h)) for h in holders]

        def restore():
            for h, saved in zip(holders, before):
                for k in list(vars(h)):
                    if k not in saved:
                        delattr(h, k)
                for k, v in saved.items():
                    setattr(h, k, v)

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.wrapped(*args)  # eager run: library loading and allocations outside capture
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        restore()
        # carried state the scope reads comes in through static buffers
        feeds = []
        for i, h in enumerate(holders):
            for k, v in list(vars(h).items()):
                if isinstance(v, torch.Tensor) and (type(h).__name__, k) in self._carried:
                    static = v.clone()
                    setattr(h, k, static)
                    feeds.append((i, k, static))
        start = [dict(vars(h)) for h in holders]
        static_args = [a.clone() if isinstance(a, torch.Tensor) else a for a in args]
        graph = torch.cuda.CUDAGraph()
        from . import hip  # (the binding; imported here to keep graph.py torch-only at import)
        with hip.graph_workspaces(), torch.cuda.graph(graph):
            outputs = self.wrapped(*static_args)
        writes = []
        for i, (h, saved) in enumerate(zip(holders, start)):
            for k, v in vars(h).items():
                if k not in saved or saved[k] is not v:
                    writes.append((i, k, v))
                    if isinstance(v, torch.Tensor):
                        self._carried.add((type(h).__name__, k))
        restore()
        return _Entry(graph, static_args, outputs, feeds, writes)
