"""The C-ABI library loads and exports every entry point the header declares.

No compute call is made here (no GPU on the CPU runner).
"""

from __future__ import annotations

import ctypes
import re

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "trnsparse_hip.h"
LIB = ROOT / "trnsparse_amd" / "libtrnsparse_hip.so"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tsp_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "tsp_bsr_spmm" in names and "tsp_last_error" in names and "tsp_version" in names


@pytest.mark.skipif(not LIB.exists(), reason="library not built (run __graft_entry__.build())")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(LIB))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


@pytest.mark.skipif(not LIB.exists(), reason="library not built (run __graft_entry__.build())")
def test_binding_signatures_match_header():
    """Every declared function has a ctypes signature in the binding and vice versa."""
    from trnsparse_amd.hip import _lib

    assert sorted(_lib.SIGNATURES) == declared_functions()


@pytest.mark.skipif(not LIB.exists(), reason="library not built (run __graft_entry__.build())")
def test_version_and_error_string_without_gpu():
    lib = ctypes.CDLL(str(LIB))
    lib.tsp_version.restype = ctypes.c_int
    lib.tsp_last_error.restype = ctypes.c_char_p
    assert lib.tsp_version() >= 100
    assert isinstance(lib.tsp_last_error(), bytes)


@pytest.mark.skipif(not LIB.exists(), reason="library not built (run __graft_entry__.build())")
def test_argument_validation_is_host_side():
    """Bad sizes are rejected before any device work (no GPU needed)."""
    from trnsparse_amd.hip import _lib

    lib = _lib.load()
    st = lib.tsp_bsr_spmm(None, 0, None, None, 0, 0, 1, 1, None, 1, 1, None, 1, 0, None, None)
    assert st == -1 and b"block_size" in lib.tsp_last_error()
    st = lib.tsp_bsr_spmm(None, 7, None, None, 0, 128, 1, 1, None, 1, 1, None, 1, 0, None, None)
    assert st == -2
