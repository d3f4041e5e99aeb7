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
    # CSR structure ops: entries without rows, bad dtype, short workspace
    assert lib.tsp_csr_row_indices(None, 0, 5, None, None) == -1
    assert lib.tsp_csr_transpose(None, 0, None, None, 0, 4, 5, None, None, None, None, 0, None) == -1
    assert lib.tsp_csr_transpose(None, 9, None, None, 3, 4, 5, None, None, None, None, 0, None) == -2
    assert lib.tsp_csr_sum(None, None, None, 2, None, None, None, 0, 0, 0, 4, None, None, None, None, 0, None) == -1
    assert lib.tsp_csr_transpose_workspace_size(10, 3, 4, 9) == -1 and lib.tsp_csr_sum_workspace_size(-1, 0, 3, 4, 0) == -1
    # BSR block-column view: blocks without block rows, null outputs, bad sizes
    assert lib.tsp_bsr_col_view(None, None, 0, 4, 3, None, None, None, None, None, 0, None) == -1
    assert lib.tsp_bsr_col_view(None, None, 2, 4, 3, None, None, None, None, None, 0, None) == -1
    assert lib.tsp_bsr_col_view_workspace_size(-1, 4) == -1 and lib.tsp_bsr_col_view_workspace_size(10, 4) > 0
    # the device sort's 32-bit positions: more than 2^32 - 1 entries are refused with a message
    assert lib.tsp_coo_to_csr_workspace_size(1 << 33, 10, 10) == -1 and b"2^32" in lib.tsp_last_error()
    assert lib.tsp_csr_transpose(None, 0, None, None, 4, 4, 1 << 33, None, None, None, None, 0, None) == -2
    assert lib.tsp_csr_sum(None, None, None, 1, None, None, None, 1, 0, 2, 4, None, None, None, None, 0, None) == -1
    # CSR SDDMM: bad dtype, bad index type, leading dimension below ncols, null pointers
    assert lib.tsp_csr_sddmm(None, None, 1, 4, 4, 3, None, 8, None, 8, 8, 2, 1.0, None, None) == -2
    assert lib.tsp_csr_sddmm(None, None, 7, 4, 4, 3, None, 8, None, 8, 8, 0, 1.0, None, None) == -1
    assert lib.tsp_csr_sddmm(None, None, 1, 4, 4, 3, None, 4, None, 8, 8, 0, 1.0, None, None) == -1
    assert lib.tsp_csr_sddmm(None, None, 1, 4, 4, 3, None, 8, None, 8, 8, 0, 1.0, None, None) == -1
    assert lib.tsp_csr_sddmm(None, None, 1, 4, 4, 0, None, 8, None, 8, 8, 0, 1.0, None, None) == 0  # nothing to do


@pytest.mark.skipif(not LIB.exists(), reason="library not built (run __graft_entry__.build())")
def test_screened_noalloc_size_limit_is_host_side():
    """The allocation-free screened SpMM refuses m past its scratch before any
    device work (dummy non-null pointers: nothing is dereferenced)."""
    from trnsparse_amd.hip import _lib

    lib = _lib.load()
    dummy = ctypes.c_void_p(256)
    for code in (_lib.TSP_F32, _lib.TSP_F64):
        mmax = lib.tsp_screened_spmm_noalloc_max_rows(code)
        assert mmax >= 4096  # BASELINE config 4 fits
        st = lib.tsp_screened_spmm_noalloc(dummy, 0, mmax + 128, dummy, code, 1e-5, mmax + 128, dummy, 8, 8, dummy, 8,
                                           None)
        assert st == -1 and b"scratch" in lib.tsp_last_error()
    assert lib.tsp_screened_spmm_noalloc_max_rows(7) == -1
    assert lib.tsp_screened_spmm_noalloc(None, 0, 4, None, 0, 0.0, 4, None, 0, 0, None, 0, None) == 0  # no columns


def _plan(cp, H, S, b):
    import numpy as np

    from trnsparse_amd.hip import _lib

    lib = _lib.load()
    cp = np.ascontiguousarray(cp, dtype=np.int64)
    n = lib.tsp_bsa_bwd_plan(cp.ctypes.data, len(cp) - 1, H, S, b, None, 0)
    assert n >= 4
    plan = np.zeros(n, np.int32)
    assert lib.tsp_bsa_bwd_plan(cp.ctypes.data, len(cp) - 1, H, S, b, plan.ctypes.data, n) == n
    ni, ns, npart, L = plan[:4]
    items = plan[4 : 4 + 4 * ni].reshape(-1, 4)
    splits = plan[4 + 4 * ni :].reshape(-1, 4)
    assert len(splits) == ns
    return items, splits, int(npart), int(L)


@pytest.mark.skipif(not LIB.exists(), reason="library not built (run __graft_entry__.build())")
@pytest.mark.parametrize(
    "counts,H,S",
    [
        ([64, 63] + [4] * 62, 32, 8192),   # cfg5-like: two global key columns
        ([8, 1, 0, 5], 1, 512),            # small: L = 4, columns split, an empty column
        ([3, 0, 2], 2, 300),               # ragged S: 3 key block columns
        ([2, 2], 1, 200),                  # mask narrower than S? (2 columns, S needs 2)
        ([100] * 3, 64, 384),              # L capped at 64
    ],
)
def test_attention_backward_plan(counts, H, S):
    """tsp_bsa_bwd_plan (host code): every key block column is covered, each
    column's block rows exactly once in contiguous segments of at most L,
    split columns own consecutive partial slots, heaviest items first."""
    import numpy as np

    b = 128
    cp = np.concatenate([[0], np.cumsum(counts)])
    items, splits, npart, L = _plan(cp, H, S, b)
    ncols = -(-S // b)
    assert 4 <= L <= 64
    w = items[:, 2] - items[:, 1]
    assert (np.diff(w) <= 0).all()                       # heaviest first
    assert (w <= L).all()
    for c in range(ncols):
        mine = items[items[:, 0] == c]
        mine = mine[np.argsort(mine[:, 1])]
        n = counts[c] if c < len(counts) else 0
        lo = cp[c] if c < len(counts) else 0
        assert len(mine) >= 1
        assert mine[0, 1] == lo and mine[-1, 2] == lo + n
        assert (mine[1:, 1] == mine[:-1, 2]).all()
        if len(mine) == 1:
            assert mine[0, 3] == -1 and n <= L
        else:
            sp = splits[splits[:, 0] == c]
            assert len(sp) == 1 and sp[0, 2] == len(mine)
            assert sorted(mine[:, 3]) == list(range(sp[0, 1], sp[0, 1] + sp[0, 2]))
            assert (mine[:, 3] == np.arange(sp[0, 1], sp[0, 1] + sp[0, 2])).all()
    assert set(items[:, 0]) == set(range(ncols))
    assert npart == sum(int(s[2]) for s in splits)
    if counts[0] == 64:                                  # cfg5: the global columns are cut
        assert L == 24 and len(splits) == 2   # ceil(32 * 375 / 256 / 2)
