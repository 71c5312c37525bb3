"""The C ABI library loads without a GPU and exports exactly what
include/dpep.h declares; argument validation happens before any HIP call."""
import ctypes
import os
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "dpep.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dpep_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_the_binding_table():
    import dpep
    assert declared_functions() == sorted(dpep.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    import dpep
    lib = dpep.load_library()
    path = dpep.LIB_PATH
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True,
                         capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (dpep_\w+)", out))
    for name in declared_functions():
        assert name in exported, name
        assert getattr(lib, name) is not None
    assert exported == set(declared_functions())


def test_abi_version_and_info():
    import dpep
    lib = dpep.load_library()
    assert lib.dpep_abi_version() == 6
    assert b"abi 6" in lib.dpep_build_info()
    assert b"gfx950" in lib.dpep_build_info()


@pytest.mark.parametrize("M,N", [(7, 8), (8, 12), (4, 4), (16384, 8), (8, 0)])
def test_create_rejects_unsupported_grids(M, N):
    import dpep
    lib = dpep.load_library()
    h = ctypes.c_void_p()
    rc = lib.dpep_create(M, N, 10, 0.0, 0.0, 1.0, 1.0, 0, 0, ctypes.byref(h))
    assert rc == 5 and not h.value
    assert "powers of two" in dpep.last_error()


def test_create_rejects_bad_arguments():
    import dpep
    lib = dpep.load_library()
    h = ctypes.c_void_p()
    assert lib.dpep_create(8, 8, -1, 0.0, 0.0, 1.0, 1.0, 0, 0, ctypes.byref(h)) == 1
    assert lib.dpep_create(8, 8, 1, 0.0, 0.0, 0.0, 1.0, 0, 0, ctypes.byref(h)) == 1
    assert lib.dpep_create(8, 8, 1, 0.0, 0.0, 1.0, 1.0, 7, 0, ctypes.byref(h)) == 1
    assert lib.dpep_create(8, 8, 1, 0.0, 0.0, 1.0, 1.0, 0, 0x100, ctypes.byref(h)) == 1
    assert lib.dpep_create(8192, 8192, 1, 0.0, 0.0, 1.0, 1.0, 1, 0, ctypes.byref(h)) == 5
    assert lib.dpep_create(8, 8, 1, 0.0, 0.0, 1.0, 1.0, 0, 0, None) == 1


def test_null_context_is_an_error():
    import dpep
    lib = dpep.load_library()
    assert lib.dpep_compute(None) == 1
    assert lib.dpep_sync(None) == 1
    assert lib.dpep_destroy(None) == 0
    with pytest.raises(ValueError):
        dpep.Context(12, 8, 1, 0, 0, 1, 1)
