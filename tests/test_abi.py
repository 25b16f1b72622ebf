"""The C-ABI library: it loads, exports every symbol include/mi_qmm.h declares,
and the Python binding table covers exactly those symbols. CPU only (no compute
calls). Also: no product module imports the oracle."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mi_qmm.h"
LIB = ROOT / "metal-autotune_amd" / "libmiqmm.so"


def declared_symbols(header: Path = HEADER) -> list[str]:
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text)))


def all_declared_symbols() -> list[str]:
    names: set[str] = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        names.update(declared_symbols(h))
    return sorted(names)


def test_header_declares_the_entry_points():
    names = declared_symbols()
    for want in ("mi_qmm_affine", "mi_affine_dequant", "mi_sdpa", "mi_last_error", "mi_abi_version"):
        assert want in names


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built: run __graft_entry__.build()")
    return ctypes.CDLL(str(LIB))


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in all_declared_symbols() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def header_abi_version() -> int:
    return int(re.search(r"#define\s+MI_ABI_VERSION\s+(\d+)", HEADER.read_text()).group(1))


def test_abi_version_and_error_string(lib):
    import sys
    sys.path.insert(0, str(ROOT / "metal-autotune_amd"))
    from autotuner_runtime import hip

    lib.mi_abi_version.restype = ctypes.c_int
    lib.mi_last_error.restype = ctypes.c_char_p
    assert lib.mi_abi_version() == header_abi_version() == hip.ABI_VERSION
    assert isinstance(lib.mi_last_error(), bytes)


def test_documented_binding_runs_against_the_library():
    """INTEGRATION.md's reference-side ctypes binding, up to and including its
    ABI-version assertion, executed against the built library (no device)."""
    doc = (ROOT / "INTEGRATION.md").read_text()
    block = re.search(r"```python\n(# autotuner_runtime/hip_backend.py.*?)```", doc, re.S).group(1)
    setup = block[: block.index("_DT = ")]
    assert "assert _lib.mi_abi_version() ==" in setup
    setup = setup.replace("/path/to/metal-autotune_amd/libmiqmm.so", str(LIB))
    exec(compile(setup, "INTEGRATION.md", "exec"), {})  # raises if the version drifted


def test_argmax_workspace_query_needs_no_device(lib):
    """The workspace bound: 8 bytes per 2048-value span per row."""
    lib.mi_argmax_workspace_bytes.restype = ctypes.c_int64
    lib.mi_argmax_workspace_bytes.argtypes = [ctypes.c_int64, ctypes.c_int64]
    assert lib.mi_argmax_workspace_bytes(1, 151936) == 600
    assert lib.mi_argmax_workspace_bytes(4, 2049) == 64
    assert lib.mi_argmax_workspace_bytes(0, 10) == 0


def test_qmm_workspace_query_needs_no_device(lib):
    """K parts: 4 fp32 copies of the output for 16-bit 8 < M <= 128,
    K >= 4096; 0 (one K part) elsewhere."""
    lib.mi_qmm_workspace_bytes.restype = ctypes.c_int64
    I64, I = ctypes.c_int64, ctypes.c_int
    lib.mi_qmm_workspace_bytes.argtypes = [I64, I64, I64, I, I, I]
    assert lib.mi_qmm_workspace_bytes(128, 2560, 4096, 64, 4, 2) == 4 * 128 * 2560 * 4
    assert lib.mi_qmm_workspace_bytes(128, 2560, 9728, 64, 4, 1) == 4 * 128 * 2560 * 4
    assert lib.mi_qmm_workspace_bytes(128, 2560, 4096, 64, 4, 0) == 0
    assert lib.mi_qmm_workspace_bytes(8, 2560, 4096, 64, 4, 2) == 0
    assert lib.mi_qmm_workspace_bytes(128, 9728, 2560, 64, 4, 2) == 0
    # 4-bit g32, 64 < M <= 128: the parts tile's scale/bias tables outgrow the
    # LDS between K ~ 93k and ~184k, so the workspace entries take the
    # one-launch path there (no workspace asked for)
    assert lib.mi_qmm_workspace_bytes(100, 64, 92160, 32, 4, 2) == 4 * 100 * 64 * 4
    assert lib.mi_qmm_workspace_bytes(100, 64, 96000, 32, 4, 2) == 0
    assert lib.mi_qmm_workspace_bytes(100, 64, 160000, 32, 4, 2) == 0


def test_argument_errors_need_no_device(lib):
    """Shape/dtype checks run before any HIP call: a bad call returns
    MI_ERR_ARG / MI_ERR_UNSUPPORTED with a message, on the CPU."""
    lib.mi_qmm_affine.restype = ctypes.c_int
    lib.mi_last_error.restype = ctypes.c_char_p
    P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.mi_qmm_affine.argtypes = [P, P, P, P, P, I64, I64, I64, I, I, I, P]
    assert lib.mi_qmm_affine(None, None, None, None, None, 1, 8, 100, 64, 4, 2, None) == 1
    assert b"multiple of group_size" in lib.mi_last_error()
    assert lib.mi_qmm_affine(None, None, None, None, None, 1, 8, 128, 64, 3, 2, None) == 2
    assert lib.mi_qmm_affine(None, None, None, None, None, 1, 8, 128, 48, 4, 2, None) == 2


def test_binding_table_matches_header():
    import sys
    sys.path.insert(0, str(ROOT / "metal-autotune_amd"))
    from autotuner_runtime import hip

    assert sorted(hip.SIGNATURES) == declared_symbols()
    assert set(hip.BINDINGS) <= set(hip.SIGNATURES)
    # the measurement entries (include/mi_peaks.h) are bound by measure.py
    import measure
    assert sorted(measure.PEAK_SYMBOLS) == declared_symbols(ROOT / "include" / "mi_peaks.h")


def test_product_code_never_imports_the_oracle():
    for py in (ROOT / "metal-autotune_amd").rglob("*.py"):
        text = py.read_text()
        assert not re.search(r"^\s*(import|from)\s+oracle\b", text, flags=re.M), py
    for src in (ROOT / "metal-autotune_amd" / "csrc").glob("*"):
        assert "orc_" not in src.read_text(), src
