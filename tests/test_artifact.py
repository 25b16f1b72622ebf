"""Artifact directories on the CPU: export -> files -> apply wiring, and the
correctness policy of check_outputs (the reference's artifact/validate.py:
179-229 restated on torch): repeatability of both arms, structure, exact
bits vs atol + rtol * |original|, non-finite placement."""

from __future__ import annotations

import json

import pytest

torch = pytest.importorskip("torch")


def _runs(*outs):
    it = iter(outs)
    return lambda: next(it)


def test_check_outputs_exact_and_tolerance():
    from autotuner_runtime.artifact import check_outputs

    a = torch.tensor([1.0, -2.0, float("inf"), float("nan")], dtype=torch.bfloat16)
    r = check_outputs(_runs((a,), (a.clone(),)), _runs((a.clone(),), (a.clone(),)), "same")
    assert r["passed"] and r["rule"] == "exact" and r["max_abs"] == 0.0
    b = a.clone()
    b[0] = 1.0078125  # one bf16 ulp above 1
    r = check_outputs(_runs((a,), (a,)), _runs((b,), (b,)), "ulp")
    assert not r["passed"] and r["failure"]["index"] == 0 and r["reason"] == "outputs differ bitwise"
    r = check_outputs(_runs((a,), (a,)), _runs((b,), (b,)), "ulp", exact=False)
    assert r["passed"] and r["rule"] == "baseline_tolerance" and r["allowance"] > 0
    c = a.clone()
    c[1] = -2.5
    r = check_outputs(_runs((a,), (a,)), _runs((c,), (c,)), "far", exact=False)
    assert not r["passed"] and r["failure"]["index"] == 1
    d = a.clone()
    d[2] = 5.0  # an inf moved to a finite value is never within tolerance
    r = check_outputs(_runs((a,), (a,)), _runs((d,), (d,)), "inf", exact=False)
    assert not r["passed"] and r["failure"]["index"] == 2


def test_check_outputs_requires_repeatability_and_structure():
    from autotuner_runtime.artifact import check_outputs

    a = torch.zeros(3)
    b = torch.ones(3)
    r = check_outputs(_runs((a,), (b,)), _runs((a,), (a,)), "orig")
    assert not r["passed"] and r["reason"] == "original model is not bitwise repeatable"
    r = check_outputs(_runs((a,), (a,)), _runs((a,), (b,)), "patched")
    assert not r["passed"] and r["reason"] == "patched model is not bitwise repeatable"
    r = check_outputs(_runs((a,), (a,)), _runs((a, a), (a, a)), "shape")
    assert not r["passed"] and "structure" in r["reason"]
    r = check_outputs(_runs((a,), (a,)), _runs((a.double(),), (a.double(),)), "dtype")
    assert not r["passed"] and "structure" in r["reason"]
    # -0.0 vs 0.0: equal values, different bits -> exact fails, tolerance passes
    z = torch.tensor([-0.0])
    assert not check_outputs(_runs((torch.tensor([0.0]),) * 1, (torch.tensor([0.0]),)),
                             _runs((z,), (z,)), "signed zero")["passed"]


def test_export_writes_the_install_layout_and_apply_wires_it(tmp_path):
    """A tiny Qwen3-layout model built on the CPU: export writes one
    launch.json + .hip per kernel id, the swap table, generated wrappers and
    bundle.json; apply installs the generated classes with each region's spec
    under the role the wrapper looks it up by."""
    from autotuner_runtime import artifact
    from autotuner_runtime.apply import apply, load_specs
    from workloads import qwen3

    cfg = qwen3.Qwen3Config(hidden_size=256, num_attention_heads=4, num_key_value_heads=2,
                            head_dim=64, intermediate_size=512, vocab_size=300)
    bundle = {"builder": {"module": "workloads.qwen3", "config": "Qwen3Config",
                          "function": "build", "kwargs": {"seed": 0, "num_layers": 2}},
              "workload": {"kind": "prefill", "label": "tiny", "seed": 1, "length": 8,
                           "vocab": 300},
              "correctness_rule": "exact"}
    model = qwen3.build(cfg, seed=0, num_layers=2, device="cpu")
    out = artifact.export(model, tmp_path / "art", bundle)
    ids = sorted(p.name for p in (out / "kernels").iterdir())
    want_ids = sorted(qwen3.Qwen3LayerRegions.KERNEL_IDS)
    assert ids == sorted([f"{k}.hip" for k in want_ids] + [f"{k}.launch.json" for k in want_ids])
    assert (out / "kernels" / "qwen3_qkv_proj.hip").read_text().strip() == "mi_qmm_affine_grouped3"
    table = json.loads((out / "swap_table.json").read_text())
    assert [e["scope_path"] for e in table] == ["model.layers.0", "model.layers.1"]
    assert sorted(load_specs(out)) == want_ids
    with pytest.raises(ValueError, match="already exists"):
        artifact.export(model, out, bundle)

    fresh = qwen3.build(cfg, seed=0, num_layers=2, device="cpu")
    patched = apply(fresh, out)
    layer = patched.model.layers[1]
    assert type(layer).__name__ == table[1]["wrapper_class"]
    assert isinstance(layer, qwen3.Qwen3LayerRegions)
    assert set(layer._specs) == set(qwen3.layer_specs(cfg))
    assert layer._specs["qkv"].kernel_id == "qwen3_qkv_proj"
    assert layer._specs["qkv"] == qwen3.layer_specs(cfg)["qkv"]
