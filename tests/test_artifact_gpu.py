"""Artifact round trip on the GPU: export the region cuts of a Qwen3 (config
3/4 shapes) and an LFM2 (config 5 shapes, 8-bit) model, install them with
apply() on freshly built models, and validate the artifact in a fresh Python
process (``python -m autotuner_runtime.artifact validate``), the analog of the
reference's exported validate.py. Rule: the patched model's logits equal the
original op streams' bit for bit, both models bitwise repeatable."""

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
