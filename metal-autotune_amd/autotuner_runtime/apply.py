"""apply(): install an artifact's regions onto a freshly built model.

The same contract as the reference's apply (autotuner_runtime/apply.py:19-60),
on torch modules: the artifact's swap table lists, per scope address, the
wrapper class (from the generated ``patch/wrappers.py``) and the region kernel
ids it runs (``kernels/<id>.launch.json`` + ``<id>.hip`` naming the entry
point). Each listed scope gets a wrapper around what it holds now; a wrapper
at the root address ("") stands in for the model itself, so callers keep the
return value. ``baseline=True`` installs the artifact's baseline table and
wrappers, which run no region kernels.
"""

from __future__ import annotations

import importlib.util
import json
from pathlib import Path
from types import ModuleType

from . import kernels as _kernels
from .swap import install, resolve


def load_specs(artifact_dir: str | Path) -> dict:
    """Every region spec of an artifact, by kernel id."""
    found = (_kernels.load_spec(p)
             for p in sorted((Path(artifact_dir) / "kernels").glob("*.launch.json")))
    return {spec.kernel_id: spec for spec in found}


def _wrapper_module(source: Path) -> ModuleType:
    """The generated wrapper classes, imported from their file (no package)."""
    loader_spec = importlib.util.spec_from_file_location("mi_patch_wrappers", source)
    module = importlib.util.module_from_spec(loader_spec)
    loader_spec.loader.exec_module(module)
    return module


def apply(model: object, artifact_dir: str | Path, *, baseline: bool = False) -> object:
    root = Path(artifact_dir)
    stem = "baseline_" if baseline else ""
    entries = json.loads((root / f"{stem}swap_table.json").read_text())
    classes = _wrapper_module(root / "patch" / f"{stem}wrappers.py")
    by_id = {} if baseline else load_specs(root)

    def wrapper_for(entry: dict, target: object) -> object:
        wrapper_cls = getattr(classes, entry["wrapper_class"])
        return wrapper_cls(target, {kid: by_id[kid] for kid in entry["kernel_ids"]})

    top = model
    for entry in entries:
        address = entry["scope_path"]
        if not address:
            top = wrapper_for(entry, top)  # the wrapper replaces the model
            continue
        current = resolve(top, address)[2]
        install(top, address, wrapper_for(entry, current))
    return top
