"""The C ABI: the built library loads and exports every entry point the
header declares, and the ctypes table matches the header (CPU only; no
kernel is launched)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from opengenie_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "opengenie_amd.h")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(oga_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "oga_fp8_linear" in names and "oga_adazero_from_ada" in names
    assert len(names) >= 20


def test_ctypes_table_matches_header():
    assert sorted(_lib.SIGNATURES) == declared_functions()


@pytest.mark.skipif(not _lib.available(), reason="library not built")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


@pytest.mark.skipif(not _lib.available(), reason="library not built")
def test_abi_version_and_error_reporting():
    lib = _lib.load()
    assert lib.oga_abi_version() == 1
    # Argument errors are reported without touching a device.
    rc = lib.oga_fp8_linear(None, 0, None, 0, None, None, None, 0, None, 0, 1, 1, 128, None)
    assert rc == -1
    assert b"null" in lib.oga_last_error()
    rc = lib.oga_bias_add_bf16(None, None, 0, None, 1, 1, None)
    assert rc == -1
