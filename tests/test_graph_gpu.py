"""Graph-level delivery: GraphWrapper captures a scope once per call
signature as a HIP graph and replays it; outputs and cache state must equal
the eager scope's bit for bit, on replays after the first too (with eager work
and synchronisations in between)."""

from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")


def test_signature_distinguishes_state_and_shapes():
    from autotuner_runtime.graph import signature

    class Cache:
        def __init__(self, t, offset):
            self.keys, self.offset = t, offset

    t = torch.zeros(4, 8)
    a = signature((torch.zeros(2, 3), Cache(t, 0)))
    assert a == signature((torch.ones(2, 3), Cache(t, 0)))        # values do not matter
    assert a != signature((torch.zeros(2, 4), Cache(t, 0)))       # shapes do
    assert a != signature((torch.zeros(2, 3), Cache(t, 5)))       # plain state does
    assert a != signature((torch.zeros(2, 3), Cache(t.clone(), 0)))  # and the buffer identity


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_graph_wrapper_qwen3_prefill_replays_equal_eager():
    from workloads import qwen3
    from autotuner_runtime.graph import GraphWrapper

    cfg = qwen3.Qwen3Config()
    model = qwen3.build(cfg, seed=4, num_layers=2)
    qwen3.install_regions(model)
    gw = GraphWrapper(model, max_graphs=2)
    caches_g, caches_e = model.make_cache(256), model.make_cache(256)
    ids = [qwen3.tokens(s, 128, cfg.vocab_size) for s in (1, 2, 3)]
    for i, t in enumerate(ids):
        for c in caches_g + caches_e:
            c.offset = 0
        got = gw(t, caches_g).clone()
        want = model(t, caches_e)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {i}"
        assert all(cg.offset == 128 for cg in caches_g)
        assert all(torch.equal(a.keys, b.keys) and torch.equal(a.values, b.values)
                   for a, b in zip(caches_g, caches_e))
        _ = torch.randn(1000, device="cuda").sum().item()  # eager work between replays
    assert gw.stats == {"captures": 1, "replays": 2, "eager": 0}
    # a new prompt length is a new signature; beyond max_graphs calls run eagerly
    for L, kind in ((64, "captures"), (32, "eager")):
        for c in caches_g + caches_e:
            c.offset = 0
        t = qwen3.tokens(9, L, cfg.vocab_size)
        got, want = gw(t, caches_g).clone(), model(t, caches_e)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
    assert gw.stats == {"captures": 2, "replays": 2, "eager": 1}


@pytest.mark.gpu
def test_graph_wrapper_carries_conv_state():
    """An LFM2 conv layer sets cache.state during its call: a replay hands the
    caller the graph's state tensor, equal to the eager state."""
    from workloads import lfm2
    from autotuner_runtime.graph import GraphWrapper

    cfg = lfm2.Lfm2Config()
    model = lfm2.build(cfg, seed=6, num_layers=1, layer_types=("conv",))
    layer = lfm2.Lfm2ConvRegions(model.model.layers[0], lfm2.layer_specs(cfg))
    gw = GraphWrapper(layer)
    for seed in (1, 2, 3):
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        x = torch.randn((1, 96, cfg.hidden_size), generator=g, device="cuda").to(torch.bfloat16)
        cg, ce = lfm2.ConvCache(), lfm2.ConvCache()
        got = gw(x, cg).clone()
        want = layer(x, ce)
        torch.cuda.synchronize()
        assert torch.equal(got, want) and torch.equal(cg.state, ce.state)
    assert gw.stats["captures"] == 1 and gw.stats["replays"] == 2


@pytest.mark.gpu
def test_graph_wrapper_two_live_conv_states_over_chunks():
    """Two conv caches, each through two chunks, interleaved: every holder
    keeps its own state (a replay hands each its own copy), the second chunk
    of each replays one graph (the carried state is keyed by layout and fed
    through a static buffer), and both states and outputs equal eager."""
    from workloads import lfm2
    from autotuner_runtime.graph import GraphWrapper

    cfg = lfm2.Lfm2Config()
    model = lfm2.build(cfg, seed=7, num_layers=1, layer_types=("conv",))
    layer = lfm2.Lfm2ConvRegions(model.model.layers[0], lfm2.layer_specs(cfg))
    gw = GraphWrapper(layer)

    def chunk(seed):
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        return torch.randn((1, 64, cfg.hidden_size), generator=g, device="cuda").to(torch.bfloat16)

    import numpy as np

    import oracle
    from conftest import to_np
    from test_lfm2_gpu import _close, export_layer

    W = export_layer(layer)
    graph_caches = {"a": lfm2.ConvCache(), "b": lfm2.ConvCache()}
    eager_caches = {"a": lfm2.ConvCache(), "b": lfm2.ConvCache()}
    order = [("a", 11), ("b", 12), ("a", 13), ("b", 14)]
    for name, seed in order:
        x = chunk(seed)
        state_in = graph_caches[name].state
        state_in = None if state_in is None else to_np(state_in)
        got = gw(x, graph_caches[name]).clone()
        want = layer(x, eager_caches[name])
        torch.cuda.synchronize()
        assert torch.equal(got, want), (name, seed)
        # independent leg: a replayed call against the oracle's conv layer
        o_want, o_state = oracle.lfm2_conv_layer(to_np(x), W, cfg, state_in)
        _close(to_np(got), o_want)
        _close(to_np(graph_caches[name].state), o_state)
        for n in ("a", "b"):
            gs, es = graph_caches[n].state, eager_caches[n].state
            assert (gs is None) == (es is None)
            if gs is not None:
                assert torch.equal(gs, es), (n, "after", name, seed)
    ga, gb = graph_caches["a"].state, graph_caches["b"].state
    assert ga.data_ptr() != gb.data_ptr()
    assert gw.stats == {"captures": 2, "replays": 2, "eager": 0}


@pytest.mark.gpu
def test_graphs_captured_in_separate_scopes_own_their_workspaces():
    """Each graph_workspaces() scope (GraphWrapper opens one per capture) gets
    scratch buffers no other scope or eager stream shares, so two captured
    K-part projections replayed side by side on two streams each equal their
    eager result."""
    from autotuner_runtime import hip, ops
    from workloads.quantize import random_quantized

    gen = torch.Generator(device="cuda")
    gen.manual_seed(77)
    M, N, K = 128, 2560, 4096  # o_proj shape: the _ws entry runs K parts
    w = [random_quantized(N, K, gen, "cuda") for _ in range(2)]
    xs = [torch.randn((M, K), generator=gen, device="cuda").to(torch.bfloat16) for _ in range(2)]
    rs = [torch.randn((M, N), generator=gen, device="cuda").to(torch.bfloat16) for _ in range(2)]
    eager = [ops.qmm_residual(xs[i], *w[i], rs[i]) for i in range(2)]
    torch.cuda.synchronize()

    def capture(i):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            ops.qmm_residual(xs[i], *w[i], rs[i])
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with hip.graph_workspaces(), torch.cuda.graph(g):
            out = ops.qmm_residual(xs[i], *w[i], rs[i])
            ptr = hip._workspace("qmm", xs[i].device, torch.cuda.current_stream().cuda_stream,
                                 1).data_ptr()
        return g, out, ptr

    (g0, o0, p0), (g1, o1, p1) = capture(0), capture(1)
    eager_ptr = hip._workspace("qmm", xs[0].device, torch.cuda.current_stream().cuda_stream,
                               1).data_ptr()
    assert len({p0, p1, eager_ptr}) == 3
    s0, s1 = torch.cuda.Stream(), torch.cuda.Stream()
    for _ in range(5):
        s0.wait_stream(torch.cuda.current_stream())
        s1.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s0):
            g0.replay()
        with torch.cuda.stream(s1):
            g1.replay()
        torch.cuda.current_stream().wait_stream(s0)
        torch.cuda.current_stream().wait_stream(s1)
        torch.cuda.synchronize()
        assert torch.equal(o0, eager[0]) and torch.equal(o1, eager[1])
