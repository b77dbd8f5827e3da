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


def test_workspace_size_queries_without_a_gpu():
    """rf_attention_workspace_bytes covers the split kernel's records over
    every context up to the given length and the any-shape kernel's score
    rows; both are host arithmetic."""
    from ramforge_amd import _lib

    lib = _lib.load()
    assert lib.rf_attention_workspace_bytes(0, 32, 8, 128) == 0
    # 8192 positions, 32 q / 8 KV heads, hd 128: the score rows (32 x 8192
    # floats) exceed the 32-chunk split records (32 x 32 x 132 floats)
    assert lib.rf_attention_workspace_bytes(8192, 32, 8, 128) == 32 * 8192 * 4
    # short contexts: per query head, up to 8 chunks of hd + 4 floats (o, m,
    # l and two unused, 16-byte aligned)
    assert lib.rf_attention_workspace_bytes(64, 32, 8, 128) == max(8 * 32 * 132 * 4, 32 * 64 * 4)
    assert lib.rf_matmul_workspace_bytes(0, 4096, 8) == 0


def test_tune_switches_without_a_gpu():
    """The process-wide tune switches are host state: each returns the mode in
    effect, values outside its range only query, and the defaults are the
    measured choices (merged attention records, in-flight packed launches,
    packed weights, float x everywhere: the digit planes are opt-in, the
    one-pass attention kernel for launches per query head)."""
    from ramforge_amd import _lib

    lib = _lib.load()
    for name, default, modes in (("rf_tune_attention_merge", 1, (0, 1)), ("rf_tune_packed_inflight", 1, (0, 1)),
                                 ("rf_tune_packed_weights", 1, (0, 1)), ("rf_tune_matvec_digits", 0, (0, 1, 2)),
                                 ("rf_tune_attention_kernel", 1, (0, 1, 2)), ("rf_tune_matvec_kernel", 2, (0, 1, 2)),
                                 ("rf_tune_prefill_attention", 1, (0, 1, 2))):
        fn = getattr(lib, name)
        assert fn(-1) == default, name
        for m in modes:
            assert fn(m) == m and fn(99) == m, (name, m)
        assert fn(default) == default


def test_file_source_reads_ranges_on_threads(tmp_path):
    """rf_file_source_read (host code, no GPU): ranges split over threads
    equal the file's bytes at every offset and length, including ranges
    shorter than one 4 MiB piece; a range past the end of the file fails."""
    import numpy as np

    import ramforge_amd as rf

    data = np.random.default_rng(44).integers(0, 256, size=(19 << 20) + 123, dtype=np.uint8)
    path = tmp_path / "blob.bin"
    path.write_bytes(data.tobytes())
    src = rf.FileSource(str(path), threads=5)
    try:
        for off, n in ((0, data.size), (7, 1), (4095, (9 << 20) + 17), (data.size - 1000, 1000), (12345, 0)):
            dst = np.zeros(max(n, 1), np.uint8)
            assert src.callback(src.user, off, n, dst.ctypes.data) == 0, (off, n)
            assert np.array_equal(dst[:n], data[off:off + n]), (off, n)
        dst = np.zeros(64, np.uint8)
        assert src.callback(src.user, data.size - 10, 64, dst.ctypes.data) != 0
    finally:
        src.close()
    with pytest.raises(rf.RamforgeError, match="cannot open"):
        rf.FileSource(str(tmp_path / "missing.bin"))
