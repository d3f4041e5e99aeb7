"""Device-side format construction through the C ABI (csrc/formats.hip).

Each function takes and returns device tensors and builds exactly the
structure the reference's torch code builds (trnsparse/formats.py): the
`formats` dataclasses call these when their input lives on the GPU and the
HIP backend is in effect. The two-phase ops (from_dense) read the entry
count back to the host between the phases, as the reference's `nonzero()`
does.
"""

from __future__ import annotations

import functools

import torch

from . import _lib

DEVICE_DTYPES = (torch.float32, torch.float64, torch.bfloat16)


# Entry points the public API calls: they run the library through ctypes and
# the registered operators, which torch.compile does not trace into; under
# compilation each call is a graph break and runs eagerly. The compiler's
# disable wrapper is made only once compilation is under way: merely loading
# the compiler stack at import (torch.compiler.disable at module level) made
# the headline product 9 % slower, with a lower GPU clock.
def _library_call(fn):
    guarded = []

    @functools.wraps(fn)
    def call(*args, **kwargs):
        if torch.compiler.is_compiling():
            if not guarded:
                guarded.append(torch.compiler.disable(fn))
            return guarded[0](*args, **kwargs)
        return fn(*args, **kwargs)

    return call


def _row_major(A: torch.Tensor) -> tuple[torch.Tensor, int]:
    """A with unit column stride and its row stride (elements)."""
    if A.dim() == 2 and A.stride(1) == 1 and A.stride(0) >= max(A.shape[1], 1):
        return A, A.stride(0)
    A = A.contiguous()
    return A, max(A.shape[1], 1)


def _stream(dev: torch.device) -> int:
    return _lib.stream_handle(dev)


@_library_call
def bsr_from_dense(A: torch.Tensor, block_size: int, threshold: float):
    """(blocks, block_col_indices, block_row_ptrs) of BSRMatrix.from_dense
    (reference formats.py:183-221) on A's device."""
    m, n = A.shape
    b = block_size
    dev = A.device
    A, lda = _row_major(A)
    mb, nbc = -(-m // b), -(-n // b)
    code = _lib.dtype_code(A.dtype)
    with torch.cuda.device(dev):
        keep = torch.empty(max(mb * nbc, 1), dtype=torch.uint8, device=dev)
        rp = torch.empty(mb + 1, dtype=torch.int64, device=dev)
        ws = torch.empty(_lib.load().tsp_format_workspace_size(mb), dtype=torch.uint8, device=dev)
        _lib.call("tsp_bsr_from_dense_pattern", A.data_ptr(), code, lda, m, n, b, float(threshold), keep.data_ptr(),
                  rp.data_ptr(), ws.data_ptr(), _stream(dev))
        nnzb = int(rp[-1].item())
        col = torch.empty(nnzb, dtype=torch.int64, device=dev)
        blocks = torch.empty(nnzb, b, b, dtype=A.dtype, device=dev)
        _lib.call("tsp_bsr_from_dense_fill", A.data_ptr(), code, lda, m, n, b, keep.data_ptr(), rp.data_ptr(), nnzb,
                  col.data_ptr(), blocks.data_ptr(), _stream(dev))
    return blocks, col, rp


@_library_call
def bsr_to_dense(blocks: torch.Tensor, row_ptrs: torch.Tensor, col_indices: torch.Tensor, shape, block_size: int):
    """BSRMatrix.to_dense (reference formats.py:233-251) on the blocks' device."""
    m, n = shape
    dev = blocks.device
    rp = row_ptrs.to(dev, torch.int64).contiguous()
    ci = col_indices.to(dev, torch.int64).contiguous()
    bl = blocks.contiguous()
    with torch.cuda.device(dev):
        out = torch.empty(m, n, dtype=blocks.dtype, device=dev)
        _lib.call("tsp_bsr_to_dense", bl.data_ptr(), _lib.dtype_code(bl.dtype), rp.data_ptr(), ci.data_ptr(),
                  bl.shape[0], block_size, m, n, out.data_ptr(), max(n, 1), _stream(dev))
    return out


@_library_call
def csr_from_dense(A: torch.Tensor, threshold: float):
    """(values, col_indices, row_ptrs) of formats.from_dense (reference
    formats.py:269-278) on A's device."""
    m, n = A.shape
    dev = A.device
    A, lda = _row_major(A)
    code = _lib.dtype_code(A.dtype)
    with torch.cuda.device(dev):
        rp = torch.empty(m + 1, dtype=torch.int64, device=dev)
        ws = torch.empty(_lib.load().tsp_format_workspace_size(m), dtype=torch.uint8, device=dev)
        _lib.call("tsp_csr_from_dense_pattern", A.data_ptr(), code, lda, m, n, float(threshold), rp.data_ptr(),
                  ws.data_ptr(), _stream(dev))
        nnz = int(rp[-1].item())
        col = torch.empty(nnz, dtype=torch.int64, device=dev)
        val = torch.empty(nnz, dtype=A.dtype, device=dev)
        _lib.call("tsp_csr_from_dense_fill", A.data_ptr(), code, lda, m, n, float(threshold), rp.data_ptr(),
                  col.data_ptr(), val.data_ptr(), _stream(dev))
    return val, col, rp


@_library_call
def csr_to_dense(values: torch.Tensor, col_indices: torch.Tensor, row_ptrs: torch.Tensor, shape):
    """CSRMatrix.to_dense (reference formats.py:49-52; duplicates add up)."""
    m, n = shape
    dev = values.device
    v = values.contiguous()
    ci = col_indices.to(dev, torch.int64).contiguous()
    rp = row_ptrs.to(dev, torch.int64).contiguous()
    with torch.cuda.device(dev):
        out = torch.empty(m, n, dtype=values.dtype, device=dev)
        _lib.call("tsp_csr_to_dense", v.data_ptr(), _lib.dtype_code(v.dtype), ci.data_ptr(), rp.data_ptr(), m, n,
                  out.data_ptr(), max(n, 1), _stream(dev))
    return out


@_library_call
def csr_row_indices(row_ptrs: torch.Tensor, m: int, nnz: int, dev: torch.device) -> torch.Tensor:
    """Row index of every entry (the expansion in CSRMatrix.to_coo,
    reference formats.py:54-65)."""
    rp = row_ptrs.to(dev, torch.int64).contiguous()
    with torch.cuda.device(dev):
        rows = torch.empty(nnz, dtype=torch.int64, device=dev)
        _lib.call("tsp_csr_row_indices", rp.data_ptr(), m, nnz, rows.data_ptr(), _stream(dev))
    return rows


@_library_call
def coo_to_csr(values: torch.Tensor, row_indices: torch.Tensor, col_indices: torch.Tensor, shape):
    """(values, col_indices, row_ptrs) of COOMatrix.to_csr (reference
    formats.py:104-124): stable sort by row*n + col on the device."""
    m, n = shape
    dev = values.device
    v = values.contiguous()
    ri = row_indices.to(dev, torch.int64).contiguous()
    ci = col_indices.to(dev, torch.int64).contiguous()
    nnz = v.shape[0]
    with torch.cuda.device(dev):
        rp = torch.empty(m + 1, dtype=torch.int64, device=dev)
        col = torch.empty(nnz, dtype=torch.int64, device=dev)
        val = torch.empty(nnz, dtype=v.dtype, device=dev)
        wsb = _lib.load().tsp_coo_to_csr_workspace_size(nnz, m, n)
        if wsb < 0:
            raise RuntimeError(f"tsp_coo_to_csr_workspace_size failed: {_lib.last_error()}")
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        _lib.call("tsp_coo_to_csr", v.data_ptr(), _lib.dtype_code(v.dtype), ri.data_ptr(), ci.data_ptr(), nnz, m, n,
                  rp.data_ptr(), col.data_ptr(), val.data_ptr(), ws.data_ptr(), wsb, _stream(dev))
    return val, col, rp


@_library_call
def coo_sum_to_csr(values: torch.Tensor, row_indices: torch.Tensor, col_indices: torch.Tensor, shape):
    """(values, col_indices, row_ptrs) with duplicate coordinates summed in
    input order — the coalesce in sparse_add (reference ops.py:107-132)."""
    m, n = shape
    dev = values.device
    v = values.contiguous()
    ri = row_indices.to(dev, torch.int64).contiguous()
    ci = col_indices.to(dev, torch.int64).contiguous()
    nnz = v.shape[0]
    with torch.cuda.device(dev):
        rp = torch.empty(m + 1, dtype=torch.int64, device=dev)
        col = torch.empty(max(nnz, 1), dtype=torch.int64, device=dev)
        val = torch.empty(max(nnz, 1), dtype=v.dtype, device=dev)
        wsb = _lib.load().tsp_coo_sum_to_csr_workspace_size(nnz, m, n)
        if wsb < 0:
            raise RuntimeError(f"tsp_coo_sum_to_csr_workspace_size failed: {_lib.last_error()}")
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        _lib.call("tsp_coo_sum_to_csr", v.data_ptr(), _lib.dtype_code(v.dtype), ri.data_ptr(), ci.data_ptr(), nnz, m,
                  n, rp.data_ptr(), col.data_ptr(), val.data_ptr(), ws.data_ptr(), wsb, _stream(dev))
        u = int(rp[-1].item())
    return val[:u], col[:u], rp


@_library_call
def csr_transpose(values: torch.Tensor, col_indices: torch.Tensor, row_ptrs: torch.Tensor, shape):
    """(values, col_indices, row_ptrs) of A^T (reference ops.py:145-154): a
    stable device sort of the entries by column, rows carried along."""
    m, n = shape
    dev = values.device
    v = values.contiguous()
    ci = col_indices.to(dev, torch.int64).contiguous()
    rp = row_ptrs.to(dev, torch.int64).contiguous()
    nnz = v.shape[0]
    code = _lib.dtype_code(v.dtype)
    with torch.cuda.device(dev):
        out_rp = torch.empty(n + 1, dtype=torch.int64, device=dev)
        out_col = torch.empty(nnz, dtype=torch.int64, device=dev)
        out_val = torch.empty(nnz, dtype=v.dtype, device=dev)
        wsb = _lib.load().tsp_csr_transpose_workspace_size(nnz, m, n, code)
        if wsb < 0:
            raise RuntimeError(f"tsp_csr_transpose_workspace_size failed: {_lib.last_error()}")
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        _lib.call("tsp_csr_transpose", v.data_ptr(), code, ci.data_ptr(), rp.data_ptr(), m, n, nnz, out_rp.data_ptr(),
                  out_col.data_ptr(), out_val.data_ptr(), ws.data_ptr(), wsb, _stream(dev))
    return out_val, out_col, out_rp


@_library_call
def csr_sum(a_values: torch.Tensor, a_cols: torch.Tensor, a_row_ptrs: torch.Tensor, b_values: torch.Tensor,
            b_cols: torch.Tensor, b_row_ptrs: torch.Tensor, shape):
    """(values, col_indices, row_ptrs) of the union sum of two CSR operands
    with duplicates summed in input order (the coalesce in sparse_add,
    reference ops.py:107-132): per row, A's entries then B's, stably sorted
    by column on the device."""
    m, n = shape
    dev = a_values.device
    av, bv = a_values.contiguous(), b_values.to(dev).contiguous()
    ac, bc = (c.to(dev, torch.int64).contiguous() for c in (a_cols, b_cols))
    ar, br = (r.to(dev, torch.int64).contiguous() for r in (a_row_ptrs, b_row_ptrs))
    na, nb = av.shape[0], bv.shape[0]
    code = _lib.dtype_code(av.dtype)
    with torch.cuda.device(dev):
        rp = torch.empty(m + 1, dtype=torch.int64, device=dev)
        col = torch.empty(max(na + nb, 1), dtype=torch.int64, device=dev)
        val = torch.empty(max(na + nb, 1), dtype=av.dtype, device=dev)
        wsb = _lib.load().tsp_csr_sum_workspace_size(na, nb, m, n, code)
        if wsb < 0:
            raise RuntimeError(f"tsp_csr_sum_workspace_size failed: {_lib.last_error()}")
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        _lib.call("tsp_csr_sum", av.data_ptr(), ac.data_ptr(), ar.data_ptr(), na, bv.data_ptr(), bc.data_ptr(),
                  br.data_ptr(), nb, code, m, n, rp.data_ptr(), col.data_ptr(), val.data_ptr(), ws.data_ptr(), wsb,
                  _stream(dev))
        u = int(rp[-1].item())
    # leading views of the outputs (sized for the union without repeats)
    return val[:u], col[:u], rp

