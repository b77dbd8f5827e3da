"""CPU checks of the C-ABI library: it loads, and it exports every symbol that
include/ramforge_hip.h declares (no compute calls: there is no GPU here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ramforge_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:[A-Za-z_][\w\s\*]*?)\b(rf_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("rf_matvec", "rf_dequantize_rows", "rf_attention_decode", "rf_rope", "rf_rmsnorm",
                     "rf_argmax", "rf_ctx_create", "rf_vram_alloc", "rf_vram_release", "rf_upload_async",
                     "rf_model_create", "rf_model_forward", "rf_model_generate"):
        assert required in names
    assert len(names) >= 50


def test_library_exports_every_declared_symbol():
    from ramforge_amd import _lib

    lib = _lib.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    # and every Python binding matches a declared symbol
    assert set(_lib.SIGNATURES) <= set(declared_functions())
    assert lib.rf_version().decode().startswith("ramforge_hip")


def test_error_plumbing_without_a_gpu():
    """Validation runs before any device work, so argument errors surface
    through rf_last_error on a machine without a GPU as well."""
    from ramforge_amd import _lib

    lib = _lib.load()
    rc = lib.rf_matvec(None, 8, None, 0, 1, 32, None, None, 0, _lib.RF_ALL_ROWS, None)
    assert rc == _lib.RF_ERR_INVALID
    assert "null context" in _lib.last_error()


def test_python_package_refuses_to_run_without_library(tmp_path, monkeypatch):
    from ramforge_amd import _lib

    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(_lib, "_LIB", None)
    with pytest.raises(ImportError, match="no CPU fallback"):
        _lib.load()
