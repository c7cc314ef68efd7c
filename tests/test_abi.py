"""The C ABI library (CPU): it loads without a GPU, exports every function that
include/dtmi.h declares, and the ctypes binding covers exactly that set."""
import ctypes
import re
import subprocess

import pytest

from dtmi import _lib


def test_library_loads_and_exports_every_declared_symbol():
    assert _lib.LIB_PATH.exists(), "build libdtmi.so first (__graft_entry__.build())"
    L = _lib.load()
    declared = _lib.header_symbols()
    assert len(declared) >= 30
    missing = [s for s in declared if not hasattr(L, s)]
    assert not missing, missing
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (dtmi_\w+)", nm))
    assert set(declared) <= exported
    # nothing exported that the header does not declare
    assert exported <= set(declared), sorted(exported - set(declared))


def test_ctypes_signatures_cover_the_header():
    declared = set(_lib.header_symbols()) - {"dtmi_last_error"}
    assert declared == set(_lib.SIGNATURES), (declared ^ set(_lib.SIGNATURES))


def test_uninitialised_calls_fail_with_a_message():
    """Without dtmi_init every entry point returns DTMI_ERR_NOT_INITIALIZED (no GPU touched)."""
    L = _lib.load()
    if _lib._initialised:
        pytest.skip("library already initialised in this process")
    p = ctypes.c_void_p()
    rc = L.dtmi_malloc(ctypes.byref(p), 16)
    assert rc == 4
    assert b"dtmi_init" in L.dtmi_last_error()
    assert L.dtmi_adamw(0, None, None, None, None, 10, 1e-3, .9, .95, 1e-8, .1, .1, .05, .1, .05, 1.0, None) == 4
