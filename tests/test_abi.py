"""CPU-side checks of the C ABI: the library loads and exports every symbol
the public header declares (no compute call: this container has no GPU)."""
import ctypes
import os

import pytest

from zerogravity_amd import _lib as L


def test_library_exports_every_header_symbol():
    lib = ctypes.CDLL(L.LIB_PATH)
    declared = L.header_symbols()
    assert len(declared) >= 15
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing


def test_python_binding_covers_every_header_symbol():
    assert set(L.header_symbols()) <= set(L._SIGS)


def test_version_string_without_device():
    assert b"gfx950" in L.lib().zg_version()


def test_library_is_gfx950_code_object():
    data = open(L.LIB_PATH, "rb").read()
    assert b"gfx950" in data


def test_product_library_does_not_reference_the_oracle():
    data = open(L.LIB_PATH, "rb").read()
    assert b"zgo_" not in data and b"zg_oracle" not in data
