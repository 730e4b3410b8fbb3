"""CPU checks of the C ABI: the library loads, exports every symbol that
include/dismoen_hip.h declares, and fails cleanly where no GPU is present."""
import ctypes as C
import os
import re

import pytest

from conftest import ROOT


def header_symbols():
    text = open(os.path.join(ROOT, "include", "dismoen_hip.h")).read()
    return sorted(set(re.findall(r"\b(dmh_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_symbols():
    from dismoen._lib import EXPORTS
    assert header_symbols() == sorted(EXPORTS)


def test_library_exports_every_declared_symbol():
    from dismoen import lib
    L = lib()
    for name in header_symbols():
        assert hasattr(L, name), name


def test_version_without_gpu():
    from dismoen import lib
    assert lib().dmh_version().startswith(b"dismoen_hip")


def test_create_reports_errors_cleanly():
    from dismoen import lib
    L = lib()
    h = C.c_void_p()
    e = C.create_string_buffer(512)
    rc = L.dmh_create(-1, C.byref(h), e, 512)
    assert rc != 0 and e.value and not h.value


def test_oracle_library_symbols(oracle):
    text = open(os.path.join(ROOT, "oracle", "dm_oracle.h")).read()
    for name in set(re.findall(r"\b(or_[a-z0-9_]+)\s*\(", text)):
        assert hasattr(oracle.lib(), name), name
