"""The build's guard for the inline-asm LDS loads (csrc/lds_dma.h): no
compiler-generated instruction may use M0 in kernels that include it.

The scanner is checked on synthetic assembly (a use outside the asm blocks
is reported, uses inside are not), and on the assembly the last build
emitted for each such kernel, when present.
"""

from __future__ import annotations

import pytest

from conftest import ROOT
from trnsparse_amd import build_lib


def test_scanner_flags_only_uses_outside_asm():
    text = "\n".join([
        "kernel:",
        "\ts_mov_b32 s4, 0",
        "\t;;#ASMSTART",
        "\ts_mov_b32 m0, s5",
        "\tglobal_load_lds_dwordx4 v1, off",
        "\t;;#ASMEND",
        "\tv_readlane_b32 s6, v2, 3 ; comment naming m0 is ignored",
        "\ts_mov_b32 m0, -1",
        "\tv_movrels_b32 v1, v2",
        "\t.amdhsa_kernel kernel ; m0 in a directive is ignored",
    ])
    assert build_lib.m0_uses_outside_asm(text) == ["s_mov_b32 m0, -1"]
    assert build_lib.m0_uses_outside_asm(text.replace("\ts_mov_b32 m0, -1\n", "")) == []


def test_last_build_assembly_has_no_m0_outside_asm():
    srcs = [s for s in build_lib._sources() if build_lib.DMA_HEADER in s.read_text()]
    assert srcs, "no kernel includes the LDS load helpers"
    asms = [build_lib.BUILD / (s.stem + ".s") for s in srcs]
    if not all(a.exists() for a in asms):
        pytest.skip("library not built in this tree (run __graft_entry__.build())")
    for a in asms:
        assert build_lib.m0_uses_outside_asm(a.read_text()) == [], a.name
