"""The C-ABI library loads and exports every symbol include/doe_mi355x.h
declares (no compute calls: CPU only)."""
import ctypes as C
import re

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "doe_mi355x.h"


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(doe_[a-z0-9_]+)\s*\(", text))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert {"doe_init", "doe_last_error", "doe_q4k_gemv", "doe_q4k_dequant"} <= syms


def test_library_exports_every_declared_symbol():
    from doe_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} is not built")
    lib = C.CDLL(str(_lib.LIB_PATH))
    missing = [s for s in sorted(declared_symbols()) if not hasattr(lib, s)]
    assert not missing, missing


def test_binding_signatures_cover_the_header():
    from doe_amd import _lib
    assert set(_lib.SIGNATURES) | {"doe_last_error"} == declared_symbols()


def test_calls_before_init_report_not_init():
    from doe_amd import _lib
    lib = _lib.load()
    ptr = C.c_void_p()
    assert lib.doe_malloc(C.byref(ptr), 16) == -2
    assert b"doe_init" in lib.doe_last_error()
