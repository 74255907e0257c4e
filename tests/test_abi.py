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


def test_gemv_args_struct_layout_matches_the_header(tmp_path):
    """ops.Q4kGemvArgs mirrors doe_q4k_gemv_args: every field at the offset
    a C compiler gives it (gcc on the header), and the same size."""
    import shutil
    import subprocess

    from doe_amd.ops import Q4kGemvArgs

    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    names = [f[0] for f in Q4kGemvArgs._fields_]
    src = tmp_path / "layout.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "doe_mi355x.h"\nint main(void) {\n'
                   + "".join(f'  printf("%zu\\n", offsetof(doe_q4k_gemv_args, {n}));\n' for n in names)
                   + '  printf("%zu\\n", sizeof(doe_q4k_gemv_args));\n  return 0;\n}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    want = [getattr(Q4kGemvArgs, n).offset for n in names] + [C.sizeof(Q4kGemvArgs)]
    assert got == want


def test_tune_keys_take_their_documented_values():
    """doe_tune_set (host state only, no GPU needed): each key accepts the
    values the header documents and rejects the rest with DOE_E_INVALID;
    0 restores the automatic choice.  Unknown keys are rejected."""
    from doe_amd import _lib
    lib = _lib.load()
    cases = {
        "q4k_gemv.bpw": ([0, 1, 4], [-1, 5]),
        "q4k_gemv.stream": ([-1, 0, 1, 16], [-2, 17]),
        "q4k_gemv.stream_depth": ([0, 2, 3, 4, 6], [1, 5, 7]),
        "q4k_gemv.ksplit": ([0, 1, 2, 4], [-1, 5]),
        "q4k_gemv.forms": ([0, 1, 2, 3], [-1, 4]),
        "q4k_gemv.kernel": ([0, 1, 2], [3]),
        "int4_gemv.kernel": ([0, 1, 2], [3]),
        "int4_gemv.depth": ([0, 2, 3], [1, 4]),
        "int4_gemv.xcd": ([0, 1], [2, -1]),
    }
    try:
        for key, (good, bad) in cases.items():
            for v in good:
                assert lib.doe_tune_set(key.encode(), v) == 0, (key, v, lib.doe_last_error())
            for v in bad:
                assert lib.doe_tune_set(key.encode(), v) == -1, (key, v)
                assert key.encode() in lib.doe_last_error()
    finally:
        for key in cases:
            lib.doe_tune_set(key.encode(), 0)
    assert lib.doe_tune_set(b"no_such.key", 1) == -1
    assert b"unknown tuning key" in lib.doe_last_error()
