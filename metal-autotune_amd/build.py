"""Build the gfx950 HIP library libmiqmm.so in-tree (next to this file).

Each csrc/*.hip is compiled to an object in parallel with hipcc, then linked
into one shared library exporting the C ABI of include/mi_qmm.h. The oracle's
C restatement (oracle/liboracle.so, test infrastructure) is built by
oracle/Makefile; `build_all()` runs both.

Flags: -O3, gfx950 only, packed-fp32 VALU forms disabled on the device
(`-packed-fp32-ops`); the host pass warns that it does not know the feature,
which is harmless. SOURCE_FLAGS adds per-file flags (mi_attn.hip: MFMA
results in arch VGPRs).
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIB = PKG / "libmiqmm.so"
BUILD = PKG / "_build"
ARCH = os.environ.get("MI_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


# Per-source device flags. mi_attn.hip: MFMA results in arch VGPRs. By
# default the compiler kept the attention accumulators in AGPRs and copied
# them through VGPRs for every tile's softmax rescale and stream merge
# (272 v_accvgpr_read/write in the 64-wide shared kernel, about 40 % of its
# loop's VALU), which also cost occupancy. Same instructions otherwise, same
# results.
SOURCE_FLAGS = {"mi_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        noise = "is not a recognized feature for this target"
        err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")


def build_hip(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libmiqmm.so (always rebuilds)."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objs = [BUILD / (s.stem + ".o") for s in sources]
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 4)))

    def compile_one(pair):
        src, obj = pair
        _run([HIPCC, *FLAGS, *SOURCE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)])
        if verbose:
            print(f"  compiled {src.name}", flush=True)

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(compile_one, zip(sources, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> Path:
    """oracle/liboracle.so via its Makefile (test infrastructure only)."""
    _run(["make", "-s", "-B", "-C", str(ROOT / "oracle")])
    return ROOT / "oracle" / "liboracle.so"


def build_all(verbose: bool = False) -> None:
    build_hip(verbose=verbose)
    build_oracle()


if __name__ == "__main__":
    build_all(verbose=True)
    print(LIB, file=sys.stderr)
