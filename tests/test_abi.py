"""CPU-side checks of the C-ABI library: it loads (no GPU needed to load) and exports every
entry point include/spx.h declares."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "spx.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(spx_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from spindle_amd import _lib
    assert os.path.exists(_lib.LIB_PATH), "libspx.so not built"
    lib = ctypes.CDLL(_lib.LIB_PATH)
    syms = declared_symbols()
    assert len(syms) >= 10
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing


def test_binding_covers_header():
    from spindle_amd import _lib
    assert set(declared_symbols()) <= set(_lib.SIGNATURES), set(declared_symbols()) - set(_lib.SIGNATURES)


def test_row_bytes_matches_reference_table():
    from spindle_amd import _lib
    lib = _lib.load()
    for dt, n, want in [(12, 2048, 1152), (14, 768, 630), (8, 1024, 1088), (6, 576, 396), (0, 10, 40), (12, 100, 0)]:
        assert lib.spx_row_bytes(dt, n) == want


def test_errors_are_reported_without_gpu():
    from spindle_amd import _lib
    lib = _lib.load()
    h = ctypes.c_void_p()
    rc = lib.spx_create(99, ctypes.byref(h))
    assert rc != 0 and lib.spx_last_error()
