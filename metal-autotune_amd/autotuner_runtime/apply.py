"""apply(): install an artifact's regions onto a freshly built model.

The reference's apply.py:19-60 on torch modules: read ``swap_table.json``
(entries of scope_path, wrapper_class, kernel_ids), load the wrapper classes
from ``patch/wrappers.py`` and the region specs from
``kernels/<id>.launch.json`` (+ ``<id>.hip`` naming the entry point), and swap
a wrapper instance in at each scope address. A root-scope entry ("") returns
the wrapper in place of the model, so callers use the return value.
"""

from __future__ import annotations

import importlib.util
import json
from pathlib import Path

from . import kernels as _kernels
from .swap import install, resolve


def load_specs(artifact_dir: str | Path) -> dict:
    specs = {}
    for launch in sorted((Path(artifact_dir) / "kernels").glob("*.launch.json")):
        spec = _kernels.load_spec(launch)
        specs[spec.kernel_id] = spec
    return specs


def apply(model: object, artifact_dir: str | Path, *, baseline: bool = False) -> object:
    artifact_dir = Path(artifact_dir)
    prefix = "baseline_" if baseline else ""
    table = json.loads((artifact_dir / f"{prefix}swap_table.json").read_text())
    module_spec = importlib.util.spec_from_file_location(
        "mi_patch_wrappers", artifact_dir / "patch" / f"{prefix}wrappers.py")
    wrappers = importlib.util.module_from_spec(module_spec)
    module_spec.loader.exec_module(wrappers)
    specs = {} if baseline else load_specs(artifact_dir)

    patched = model
    for entry in table:
        cls = getattr(wrappers, entry["wrapper_class"])
        kernel_specs = {kid: specs[kid] for kid in entry["kernel_ids"]}
        path = entry["scope_path"]
        if path == "":
            patched = cls(patched, kernel_specs)
        else:
            _, _, original = resolve(patched, path)
            install(patched, path, cls(original, kernel_specs))
    return patched
