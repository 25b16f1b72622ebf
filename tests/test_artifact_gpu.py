"""Artifact round trip on the GPU: export the region cuts of a Qwen3 (config
3/4 shapes) and an LFM2 (config 5 shapes, 8-bit) model, install them with
apply() on freshly built models, and validate the artifact in a fresh Python
process (``python -m autotuner_runtime.artifact validate``), the analog of the
reference's exported validate.py. Rule: the patched model's logits equal the
original op streams' bit for bit, both models bitwise repeatable. The
installed Qwen3 artifact also has an independent leg: its layers and lm_head
against the CPU oracle on the same inputs (the reference validates against
the original MLX ops, an independent path: artifact/validate.py:179-229)."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

torch = pytest.importorskip("torch")

ROOT = Path(__file__).resolve().parents[1]


def _fresh_validate(art: Path) -> subprocess.CompletedProcess:
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join(
        [str(ROOT / "metal-autotune_amd"), str(ROOT), env.get("PYTHONPATH", "")])
    print(f"\nfresh-process validate {art}", flush=True)
    return subprocess.run([sys.executable, "-m", "autotuner_runtime.artifact", "validate",
                           str(art)], env=env, capture_output=True, text=True, timeout=600)


def _oracle_leg_qwen3(patched, run, cfg, n_layers=2):
    """An independent leg for the installed artifact: each of the first
    n_layers patched layers (the artifact's wrappers) against the oracle's
    decoder layer on the same input, and the tied lm_head on the final hidden
    state against the oracle's, <= 1e-2 max-abs-normalised."""
    import numpy as np

    import oracle
    from conftest import to_np
    from test_models_gpu import _close, _lin, export_layer

    seen = []
    hooks = [layer.register_forward_hook(lambda m, a, out: seen.append((to_np(a[0]), to_np(out))))
             for layer in list(patched.model.layers)[:n_layers]]
    final = []
    hooks.append(patched.model.norm.register_forward_hook(
        lambda m, a, out: final.append(to_np(a[0]))))
    try:
        logits = to_np(run(patched)[0])
    finally:
        for h in hooks:
            h.remove()
    assert len(seen) == n_layers and final
    for (x, y), layer in zip(seen, patched.model.layers):
        inner = layer.wrapped if hasattr(layer, "wrapped") else layer
        kc = np.zeros((1, cfg.num_key_value_heads, x.shape[1], cfg.head_dim), np.float32)
        want = oracle.qwen3_layer(x, export_layer(inner), cfg, 0, kc, np.zeros_like(kc))
        err = _close(y, want)
        print(f"artifact layer vs oracle: {err:.3e}")
    emb = patched.model.embed_tokens
    hn = oracle.rms_norm(final[-1][:, -1:], to_np(patched.model.norm.weight), cfg.rms_norm_eps,
                         "bfloat16")
    want = oracle.qmm_factored(hn, *_lin(emb), cfg.group_size, cfg.bits, "bfloat16")
    _close(logits.reshape(-1), want.reshape(-1))


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_qwen3_artifact_round_trip(tmp_path):
    from autotuner_runtime import artifact
    from autotuner_runtime.apply import apply
    from workloads import qwen3

    cfg = qwen3.Qwen3Config()
    bundle = {"builder": {"module": "workloads.qwen3", "config": "Qwen3Config",
                          "function": "build", "kwargs": {"seed": 0, "num_layers": 4}},
              "workload": {"kind": "prefill", "label": "qwen3 prefill 128", "seed": 1,
                           "length": 128, "vocab": cfg.vocab_size},
              "correctness_rule": "exact"}
    art = artifact.export(qwen3.build(cfg, seed=0, num_layers=4), tmp_path / "qwen3_art", bundle)

    # in process: apply() on a fresh model == install_regions == the original ops
    run = artifact.load_workload(bundle)
    original = artifact.build_model(bundle)
    direct = artifact.build_model(bundle)
    qwen3.install_regions(direct)
    patched = apply(artifact.build_model(bundle), art)
    want, = run(original)
    assert torch.equal(run(patched)[0], want) and torch.equal(run(direct)[0], want)
    res, = artifact.validate(art)
    assert res["passed"], res
    _oracle_leg_qwen3(patched, run, cfg)
    del original, direct, patched
    torch.cuda.empty_cache()

    proc = _fresh_validate(art)
    print(proc.stdout, proc.stderr[-2000:])
    assert proc.returncode == 0 and "PASS qwen3 prefill 128" in proc.stdout


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_lfm2_artifact_round_trip_and_a_bad_kernel_fails(tmp_path):
    """LFM2 8-bit (conv and attention layers) validates in a fresh process;
    the same artifact with the [qmm(out_proj), add, rms_norm] region's launch
    template edited to eps 0.1 (a region that no longer computes the
    original ops) fails the exact rule with a located element."""
    import json

    from autotuner_runtime import artifact
    from workloads import lfm2

    bundle = {"builder": {"module": "workloads.lfm2", "config": "Lfm2Config",
                          "config_kwargs": {"bits": 8},
                          "function": "build",
                          "kwargs": {"seed": 3, "layer_types": ["conv", "attn", "conv"]}},
              "workload": {"kind": "prefill", "label": "lfm2 prefill 512", "seed": 4,
                           "length": 512, "vocab": 65536},
              "correctness_rule": "exact"}
    model = artifact.build_model(bundle)
    art = artifact.export(model, tmp_path / "lfm2_art", bundle)
    del model
    proc = _fresh_validate(art)
    print(proc.stdout, proc.stderr[-2000:])
    assert proc.returncode == 0 and "PASS lfm2 prefill 512" in proc.stdout

    launch = art / "kernels" / "lfm2_out_proj_add_norm.launch.json"
    spec = json.loads(launch.read_text())
    spec["template"] = [["eps", "0.1"] if k == "eps" else [k, v] for k, v in spec["template"]]
    launch.write_text(json.dumps(spec))
    res, = artifact.validate(art)
    assert not res["passed"] and res["failure"] is not None, res
    print("tampered artifact:", artifact.describe(res))
