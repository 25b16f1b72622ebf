"""Size-generic serving on the GPU: each region kernel of the Qwen3 layer
checked against the original ops at prompt lengths from 1 to 200 (bit for
bit, both timed), served ranges planned around the primary size, gating
verified, and the ranges carried through an exported artifact."""

from __future__ import annotations

import json

import pytest

torch = pytest.importorskip("torch")

SIZES = [1, 2, 3, 8, 9, 16, 33, 64, 100, 128, 160, 200]  # timed; every size 1..200 is checked


def _layer():
    from workloads import qwen3

    cfg = qwen3.Qwen3Config()
    model = qwen3.build(cfg, seed=21, num_layers=1)
    return cfg, model.model.layers[0]


def _make_call(cfg):
    from workloads import qwen3

    gen = torch.Generator(device="cuda")

    def call(mod, n):
        gen.manual_seed(1000 + n)
        x = torch.randn((1, n, cfg.hidden_size), generator=gen, device="cuda").to(torch.bfloat16)
        cache = qwen3.KVCache(cfg.num_key_value_heads, cfg.head_dim, 256, "cuda")
        return (mod(x, cache), cache.keys, cache.values, x)
    return call


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_qwen3_kernels_checked_over_sizes_and_ranges_planned():
    from autotuner_runtime import serve
    from workloads import qwen3

    cfg, layer = _layer()
    specs = qwen3.layer_specs(cfg)
    every = list(range(1, 201))
    res = serve.check_sizes(layer, lambda s: qwen3.Qwen3LayerRegions(layer, s), specs, every,
                            _make_call(cfg), timed=SIZES, reps=3)
    assert sorted(res) == sorted(s.kernel_id for s in specs.values())
    for kid, r in res.items():
        assert r["correct"] == every, f"{kid}: not bit-exact at {set(every) - set(r['correct'])}"
        assert sorted(r["clock"]) == SIZES
        print(f"\n{kid}: " + ", ".join(
            f"{n}:{c['ms_kernel'] / c['ms_original']:.2f}" for n, c in r["clock"].items()))
    ranges = serve.plan_ranges(res, primary=128)
    print("served ranges (primary 128):", ranges)
    for kid, rng in ranges.items():
        # the primary is served unless the kernel measurably lost there
        if not res[kid]["clock"][128]["loss"]:
            assert rng and rng[0][0] <= 128 <= rng[0][1], (kid, rng)


@pytest.mark.gpu
def test_ranges_gate_the_kernels(monkeypatch):
    """Outside its served range a kernel is not launched and the original ops
    run (same bits); inside it the kernel runs."""
    from autotuner_runtime import kernels
    from workloads import qwen3

    cfg, layer = _layer()
    w = qwen3.Qwen3LayerRegions(layer, qwen3.layer_specs(cfg))
    w.set_ranges({"qwen3_qkv_proj": [[64, 128]], "qwen3_o_proj_add_norm": [],
                  "qwen3_gate_up_swiglu": [[1, 2048]], "qwen3_down_add": [[100, 100]]})
    launched = []
    real = kernels.try_sized
    monkeypatch.setattr(kernels, "try_sized",
                        lambda spec, ins, init_value=None: launched.append(spec.kernel_id)
                        or real(spec, ins, init_value))
    # a served q/k/v cut runs fused with the attention prologue (one launch)
    fused = qwen3.ops.qkv_norm_rope

    def counting_fused(*a, **k):
        out = fused(*a, **k)
        if out is not None:
            launched.append("qwen3_qkv_proj")
        return out

    monkeypatch.setattr(qwen3.ops, "qkv_norm_rope", counting_fused)
    call = _make_call(cfg)
    for n, want in ((32, {"qwen3_gate_up_swiglu"}),
                    (100, {"qwen3_qkv_proj", "qwen3_gate_up_swiglu", "qwen3_down_add"})):
        launched.clear()
        got = call(w, n)
        assert set(launched) == want, (n, launched)
        ref = call(layer, n)
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(got, ref))
    # an independent leg at a served size: the layer against the oracle's
    import numpy as np

    import oracle
    from conftest import to_np
    from test_models_gpu import _close, export_layer

    kc = np.zeros((1, cfg.num_key_value_heads, 100, cfg.head_dim), np.float32)
    want = oracle.qwen3_layer(to_np(got[3]), export_layer(layer), cfg, 0, kc, np.zeros_like(kc))
    print(f"\nserved size 100 vs oracle: {_close(to_np(got[0]), want):.3e}")


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_ranges_travel_through_an_artifact(tmp_path):
    from autotuner_runtime import artifact
    from autotuner_runtime.apply import apply
    from workloads import qwen3

    cfg = qwen3.Qwen3Config()
    bundle = {"builder": {"module": "workloads.qwen3", "config": "Qwen3Config",
                          "function": "build", "kwargs": {"seed": 0, "num_layers": 2}},
              "workload": {"kind": "prefill", "label": "qwen3 prefill 48", "seed": 2,
                           "length": 48, "vocab": cfg.vocab_size},
              "correctness_rule": "exact"}
    ranges = {"qwen3_qkv_proj": [[2, 2048]], "qwen3_o_proj_add_norm": [[64, 2048]],
              "qwen3_gate_up_swiglu": [[2, 2048]], "qwen3_down_add": [[2, 40], [50, 60]]}
    art = artifact.export(artifact.build_model(bundle), tmp_path / "art", bundle, ranges)
    table = json.loads((art / "swap_table.json").read_text())
    assert table[0]["sizes"] == ranges
    patched = apply(artifact.build_model(bundle), art)
    layer = patched.model.layers[0]
    assert type(layer).RANGES == ranges
    res, = artifact.validate(art)
    assert res["passed"], res
