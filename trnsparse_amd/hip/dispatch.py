"""HIP dispatch: the MI355X side of the ops seam.

Replaces the reference's NKI dispatch layer (trnsparse/nki/dispatch.py):
each `hip_*` function is what `ops.py` calls when the HIP backend is in
effect. It places operands on the GPU (inputs on the host are copied over
and the result is returned on the caller's device, as the reference's
`_to_xla` / `.to(orig_device)` round trip does, dispatch.py:88-94),
prepares the cached per-pattern plan, allocates outputs and calls the C ABI
on the current HIP stream. Autograd wrappers keep the reference's
signatures; the BSR SpMM, CSR matmul and attention backward passes call
their own kernels through the C ABI, the screened SpMM backward (two dense
masked products) runs as torch ops on the device.

Kernel failures raise RuntimeError; nothing falls back to another path.
"""

from __future__ import annotations

import functools
import math

import numpy as np
import torch
import torch.nn.functional as F

from . import _lib


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


def _target_device(*tensors) -> torch.device:
    for t in tensors:
        if isinstance(t, torch.Tensor) and t.is_cuda:
            return t.device
    return torch.device("cuda", torch.cuda.current_device())


def _on(t: torch.Tensor, dev: torch.device, dtype: torch.dtype | None = None) -> torch.Tensor:
    return t.to(device=dev, dtype=dtype or t.dtype).contiguous()


# --------------------------------------------------------------------- BSR


def _bsr_plan(col_idx: torch.Tensor, row_ptrs: torch.Tensor, mb: int, dev: torch.device, holder=None):
    """Device copies of the pattern plus the heaviest-first row order.

    Cached on `holder` (the BSRMatrix) keyed by the pattern tensors, so a
    matrix reused across calls pays for the transfer and the plan once.
    """
    key = (
        str(dev),
        row_ptrs.data_ptr(),
        row_ptrs._version,
        row_ptrs.numel(),
        col_idx.data_ptr(),
        col_idx._version,
        col_idx.numel(),
    )
    cached = getattr(holder, "_hip_plan", None) if holder is not None else None
    if cached is not None and cached[0] == key:
        return cached[1]
    if row_ptrs.numel() != mb + 1:
        raise AssertionError(f"block_row_ptrs has {row_ptrs.numel()} entries, expected {mb + 1}")
    rp = _on(row_ptrs, dev, torch.int64)
    ci = _on(col_idx, dev, torch.int64)
    order = torch.empty(mb, dtype=torch.int32, device=dev)
    _lib.call("tsp_bsr_row_order", rp.data_ptr(), mb, order.data_ptr(), _lib.stream_handle(dev))
    plan = (rp, ci, order)
    if holder is not None:
        try:
            # the source tensors ride along: while the entry lives their
            # addresses cannot be reused by new tensors with the same key
            holder._hip_plan = (key, plan, (row_ptrs, col_idx))
        except AttributeError:
            pass
    return plan


def _bsr_spmm_launch(blocks, rp, ci, order, shape, b, B, out_dtype, dev) -> torch.Tensor:
    m, n = shape
    ncols = B.shape[1]
    if blocks.dtype != B.dtype:
        raise RuntimeError(f"bsr_spmm: blocks dtype {blocks.dtype} and B dtype {B.dtype} differ")
    blocks_d = _on(blocks, dev)
    B_d = _on(B, dev)
    if ncols == 1 and out_dtype == blocks.dtype:
        # one vector: the bandwidth-bound BSR-SpMV kernel
        x = B_d.reshape(-1)
        C = torch.empty((m, 1), dtype=out_dtype, device=dev)
        _lib.call("tsp_bsr_spmv", blocks_d.data_ptr(), _lib.dtype_code(blocks_d.dtype), rp.data_ptr(), ci.data_ptr(),
                  blocks_d.shape[0], b, m, n, x.data_ptr(), 1.0, None, 0.0, None, 0.0, None, 0.0, C.data_ptr(),
                  order.data_ptr() if order is not None else None, _lib.stream_handle(dev))
        return C
    ldb = ncols
    vec = {torch.float32: 4, torch.bfloat16: 8, torch.float64: 2}.get(B_d.dtype)
    if vec and b == 128 and ncols % vec:
        # Row stride a multiple of 16 bytes for the vectorised B panel loads.
        B_d = F.pad(B_d, (0, vec - ncols % vec))
        ldb = B_d.shape[1]
    # (a padded B is passed as its first ncols columns: the row stride stays ldb)
    return _lib.ops().bsr_spmm(blocks_d, rp, ci, order, m, n, b, B_d[:, :ncols], out_dtype)


class _BSRSpMMFunction(torch.autograd.Function):
    """Autograd wrapper of BSR SpMM (reference dispatch.py:290-369).

    Forward: tsp_bsr_spmm. Backward, also on the device through the C ABI:
      dA_blocks[k] = dC[row block of k] @ B[col block of k]^T   (tsp_bsr_sddmm)
      dB           = A^T @ dC over the block-column view        (tsp_bsr_spmm_t)
    The pattern carries no gradient.
    """

    @staticmethod
    def forward(ctx, A_blocks, A_block_col_indices, A_block_row_ptrs, A_shape, A_block_size, B, out_dtype=None, plan=None):
        m, n = A_shape
        b = A_block_size
        if B.dim() != 2 or B.shape[0] != n:
            raise AssertionError(f"Dimension mismatch: A is {A_shape}, B is {tuple(B.shape)}")
        orig = B.device
        dev = _target_device(B, A_blocks)
        mb = (m + b - 1) // b
        with torch.cuda.device(dev):
            rp, ci, order = plan if plan is not None else _bsr_plan(A_block_col_indices, A_block_row_ptrs, mb, dev)
            C = _bsr_spmm_launch(A_blocks, rp, ci, order, A_shape, b, B, out_dtype or A_blocks.dtype, dev)
        ctx.save_for_backward(A_blocks, B)
        ctx.pattern = (rp, ci)
        ctx.A_shape = A_shape
        ctx.A_block_size = b
        return C.to(orig)

    @staticmethod
    def backward(ctx, grad_out):
        A_blocks, B = ctx.saved_tensors
        rp, ci = ctx.pattern
        b = ctx.A_block_size
        m, n = ctx.A_shape
        dev = rp.device
        mb = rp.numel() - 1
        nbc = (n + b - 1) // b
        ncols = grad_out.shape[1]
        dt = A_blocks.dtype
        _lib.dtype_code(dt)  # raises for a dtype the kernels do not take
        with torch.cuda.device(dev):
            blocks = _on(A_blocks, dev)
            G = _on(grad_out, dev, dt)
            brow, cp, cbid, crow, corder = _bsr_bwd_plan(rp, ci, mb, nbc, dev)
            grad_blocks = grad_B = None
            if ctx.needs_input_grad[0]:
                Bd = _on(B, dev, dt)
                gb = _lib.ops().bsr_sddmm(G, Bd, brow, ci, m, n, b)
                grad_blocks = gb.to(A_blocks.device)
            if ctx.needs_input_grad[5]:
                dB = _lib.ops().bsr_spmm_t(blocks, cp, cbid, crow, corder, m, n, b, G)
                grad_B = dB.to(B.device, B.dtype)
        return grad_blocks, None, None, None, None, grad_B, None, None


def _bsr_bwd_plan(rp: torch.Tensor, ci: torch.Tensor, mb: int, nbc: int, dev: torch.device):
    """Pattern views for the backward kernels, built on the device by
    tsp_bsr_col_view: the block row of every stored block, and the
    block-column view (col_ptrs; per column, in increasing block-row order,
    the stored block index and its block row), plus the heaviest-first order
    of the block columns (tsp_bsr_row_order on col_ptrs)."""
    nnzb = ci.numel()
    i64 = dict(dtype=torch.int64, device=dev)
    brow = torch.empty(max(nnzb, 1), **i64)
    cp = torch.empty(nbc + 1, **i64)
    cbid = torch.empty(max(nnzb, 1), **i64)
    crow = torch.empty(max(nnzb, 1), **i64)
    lib = _lib.load()
    wsz = lib.tsp_bsr_col_view_workspace_size(nnzb, nbc)
    if wsz < 0:
        raise RuntimeError(f"tsp_bsr_col_view_workspace_size failed for {nnzb} blocks, {nbc} block columns")
    ws = torch.empty(max(int(wsz), 1), dtype=torch.uint8, device=dev)
    st = _lib.stream_handle(dev)
    _lib.call("tsp_bsr_col_view", rp.data_ptr(), ci.data_ptr(), mb, nbc, nnzb, brow.data_ptr(), cp.data_ptr(),
              cbid.data_ptr(), crow.data_ptr(), ws.data_ptr(), int(wsz), st)
    corder = torch.empty(max(nbc, 1), dtype=torch.int32, device=dev)
    if nbc:
        _lib.call("tsp_bsr_row_order", cp.data_ptr(), nbc, corder.data_ptr(), st)
    return brow[:nnzb], cp, cbid[:nnzb], crow[:nnzb], corder


@_library_call
def hip_bsr_matvec_update(A, x: torch.Tensor, alpha: float, out: torch.Tensor, u=None, beta: float = 0.0, v=None,
                          gamma: float = 0.0, w=None, delta: float = 0.0) -> torch.Tensor:
    """out = alpha * (A @ x) + beta * u + gamma * v + delta * w in one pass
    over A (tsp_bsr_spmv). All vectors on one GPU in A's dtype; out must not
    be x. Used by the fixed-step solvers."""
    m, n = A.shape
    dev = x.device
    rp, ci, order = _bsr_plan(A.block_col_indices, A.block_row_ptrs, (m + A.block_size - 1) // A.block_size, dev,
                              holder=A)
    blocks = A.blocks if A.blocks.device == dev else _bsr_blocks_on(A, dev)
    _lib.call("tsp_bsr_spmv", blocks.data_ptr(), _lib.dtype_code(blocks.dtype), rp.data_ptr(), ci.data_ptr(),
              blocks.shape[0], A.block_size, m, n, x.data_ptr(), float(alpha), _lib.ptr(u), float(beta), _lib.ptr(v),
              float(gamma), _lib.ptr(w), float(delta), out.data_ptr(), order.data_ptr(), _lib.stream_handle(dev))
    return out


def _bsr_blocks_on(A, dev):
    """A's blocks on `dev`, cached on A (keyed by the tensor's identity and version)."""
    key = (str(dev), A.blocks.data_ptr(), A.blocks._version)
    cached = getattr(A, "_hip_blocks", None)
    if cached is not None and cached[0] == key:
        return cached[1]
    blocks = A.blocks.to(dev).contiguous()
    try:
        A._hip_blocks = (key, blocks, A.blocks)  # source kept alive, as for the pattern plans
    except AttributeError:
        pass
    return blocks


@_library_call
def hip_bsr_spmm(A, B: torch.Tensor, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """BSR SpMM entry point (replaces nki_bsr_spmm, reference dispatch.py:372-381).

    fp16 blocks and B are widened to fp32 (exact; the casts carry autograd)
    and the result rounded to the output dtype once."""
    m, _ = A.shape
    b = A.block_size
    dev = _target_device(B, A.blocks)
    with torch.cuda.device(dev):
        plan = _bsr_plan(A.block_col_indices, A.block_row_ptrs, (m + b - 1) // b, dev, holder=A)
    if A.blocks.dtype == torch.float16 and B.dtype == torch.float16:
        C = _BSRSpMMFunction.apply(A.blocks.float(), A.block_col_indices, A.block_row_ptrs, A.shape, A.block_size,
                                   B.float(), torch.float32, plan)
        return C.to(out_dtype or torch.float16)
    return _BSRSpMMFunction.apply(
        A.blocks, A.block_col_indices, A.block_row_ptrs, A.shape, A.block_size, B, out_dtype, plan
    )


# --------------------------------------------------------------------- CSR


def _key(*ts):
    return tuple((t.data_ptr(), t._version, t.numel(), t.dtype) for t in ts)


def _csr_device(A, dev: torch.device):
    """Device copies of (values, col_indices, row_ptrs) plus the SpMV window
    table, cached on the CSRMatrix keyed by its tensors."""
    key = (str(dev),) + _key(A.values, A.col_indices, A.row_ptrs)
    cached = getattr(A, "_hip_csr", None)
    if cached is not None and cached[0] == key:
        return cached[1]
    m, n = A.shape
    if A.row_ptrs.numel() != m + 1:
        raise AssertionError(f"row_ptrs has {A.row_ptrs.numel()} entries, expected {m + 1}")
    itype = A.col_indices.dtype if A.col_indices.dtype == A.row_ptrs.dtype else torch.int64
    if itype not in (torch.int32, torch.int64):
        itype = torch.int64
    vals = _on(A.values, dev)
    cols = _on(A.col_indices, dev, itype)
    ptrs = _on(A.row_ptrs, dev, itype)
    nnz = vals.numel()
    size = _lib.load().tsp_csr_plan_size(m, nnz)
    win = torch.empty(size, dtype=torch.int64, device=dev)
    _lib.call("tsp_csr_plan", ptrs.data_ptr(), _lib.index_code(itype), m, nnz, win.data_ptr(), _lib.stream_handle(dev))
    res = (vals, cols, ptrs, win)
    try:
        A._hip_csr = (key, res, (A.values, A.col_indices, A.row_ptrs))  # sources kept alive, as above
    except AttributeError:
        pass
    return res


def _csr_forward(vals, cols, ptrs, win, shape, X, alpha, Y, beta, dev, colplan=None):
    """out = alpha * A @ X (+ beta * Y). `colplan` is None (windowed kernel),
    ("colplan", geometry, plan) or ("bucketed", plan, n_medium, n_long) for a
    vector X."""
    m, n = shape
    if vals.dtype != X.dtype:
        raise RuntimeError(f"CSR values dtype {vals.dtype} and dense operand dtype {X.dtype} differ")
    code = _lib.dtype_code(vals.dtype)
    if code == _lib.TSP_BF16:
        raise RuntimeError("HIP CSR kernels support float32 and float64 values")
    _lib.index_code(cols.dtype)  # raises for an index dtype the kernels do not take
    Xd = _on(X, dev)
    use_y = Y is not None and beta != 0.0
    Yd = _on(Y, dev, vals.dtype) if use_y else None
    if Xd.dim() == 1:
        if use_y and Yd.shape != (m,):
            Yd = Yd.expand(m).contiguous()
        if colplan is not None and colplan[0] == "bucketed":
            _, plan, n_med, n_long = colplan
            out = torch.empty(m, dtype=vals.dtype, device=dev)
            _lib.call("tsp_csr_bucketed_spmv", vals.data_ptr(), code, cols.data_ptr(), ptrs.data_ptr(),
                      _lib.index_code(cols.dtype), m, n, vals.numel(), plan.data_ptr(), n_med, n_long, Xd.data_ptr(),
                      float(alpha), _lib.ptr(Yd), float(beta), out.data_ptr(), _lib.stream_handle(dev))
            return out
        if colplan is not None:
            _, geom, plan = colplan
            return _lib.ops().csr_colplan_spmv(plan, _geometry_list(geom), vals, cols, ptrs, m, n, Xd, float(alpha),
                                               Yd, float(beta))
        return _lib.ops().csr_spmv(vals, cols, ptrs, win, m, n, Xd, float(alpha), Yd, float(beta))
    ncols = Xd.shape[1]
    if use_y and Yd.shape != (m, ncols):
        Yd = Yd.expand(m, ncols).contiguous()
    return _lib.ops().csr_spmm(vals, cols, ptrs, m, n, Xd, float(alpha), Yd, float(beta))


def _geometry_list(geom) -> list[int]:
    """The column plan's 10 host int64 geometry values as the operator's
    `int[]` argument."""
    return [int(v) for v in geom]


# SpMV over the column-sorted plan (tsp_csr_colplan_*): "auto" builds the
# plan the second time an unchanged fp32 matrix with at least
# COLPLAN_MIN_NNZ entries meets a vector (a one-off matrix keeps the
# windowed kernel, which needs no reordered copy), "always" on first use,
# "never" not at all. New values on a cached pattern are regathered into
# the plan without sorting again. "bucketed" runs the row-per-wavefront
# kernels with long rows split out by length (tsp_csr_bucketed_spmv)
# instead of either.
_SPMV_PLAN_MODES = ("auto", "always", "never", "bucketed")
_spmv_plan_mode = "auto"
COLPLAN_MIN_NNZ = 1 << 18


def set_spmv_plan(mode: str) -> None:
    """Select when spmv uses the column-sorted plan: "auto", "always",
    "never"; or "bucketed" for the length-bucketed row kernels.

    Each kernel is deterministic, but the windowed kernel and the plan add a
    row's products in different orders, so under "auto" (windowed kernel on
    a matrix's first product, the plan from the second) two identical
    spmv(A, x) calls can differ in the last bits. "never" or "always" give
    bit-identical repeated calls."""
    global _spmv_plan_mode
    if mode not in _SPMV_PLAN_MODES:
        raise AssertionError(f"spmv plan mode must be one of {_SPMV_PLAN_MODES}, got {mode!r}")
    _spmv_plan_mode = mode


def get_spmv_plan() -> str:
    return _spmv_plan_mode


def _csr_bucket_plan(A, ptrs: torch.Tensor, dev: torch.device):
    """(plan, n_medium, n_long) of the length-bucketed SpMV, cached on A by
    pattern: the lists of rows with more than 32 and more than 2048 entries
    (tsp_csr_bucket_plan) and their counts, read back once."""
    m = A.shape[0]
    key = (str(dev),) + _key(A.row_ptrs)
    cached = getattr(A, "_hip_bucket_plan", None)
    if cached is not None and cached[0] == key:
        return cached[1]
    plan = torch.empty(_lib.load().tsp_csr_bucket_plan_size(m) // 4, dtype=torch.int32, device=dev)
    _lib.call("tsp_csr_bucket_plan", ptrs.data_ptr(), _lib.index_code(ptrs.dtype), m, plan.data_ptr(),
              _lib.stream_handle(dev))
    n_med, n_long = (int(v) for v in plan[:2].cpu())
    out = (plan, n_med, n_long)
    try:
        A._hip_bucket_plan = (key, out)
    except AttributeError:
        pass
    return out


def _csr_colplan(A, vals, cols, ptrs, dev, rows_per_block_log2: int = 0, tiles_hint: int = 0):
    """The column-sorted SpMV plan of A, cached on the matrix, or None when
    the plan does not apply (mode, dtype, size) or is not due yet."""
    mode = _spmv_plan_mode
    nnz = vals.numel()
    if mode in ("never", "bucketed") or vals.dtype != torch.float32 or nnz == 0:
        return None
    if mode == "auto" and nnz < COLPLAN_MIN_NNZ:
        return None
    m, n = A.shape
    skey = (str(dev), rows_per_block_log2, tiles_hint) + _key(A.col_indices, A.row_ptrs)
    vkey = _key(A.values)
    cached = getattr(A, "_hip_colplan", None)
    if cached is not None and cached[0] == skey:
        _, ckey, geom, plan, uses = cached
        if ckey != vkey:
            # New values on the cached pattern: regathering them into the plan
            # costs about three plan SpMVs, more than one windowed SpMV, so under
            # "auto" they are regathered only when the same values come back.
            if mode == "auto" and getattr(A, "_hip_colplan_pending", None) != vkey:
                try:
                    A._hip_colplan_pending = vkey
                except AttributeError:
                    pass
                return None
            _lib.call("tsp_csr_colplan_refresh", vals.data_ptr(), _lib.TSP_F32, ptrs.data_ptr(),
                      _lib.index_code(ptrs.dtype), m, n, nnz, geom.ctypes.data, plan.data_ptr(),
                      _lib.stream_handle(dev))
        A._hip_colplan = (skey, vkey, geom, plan, uses + 1)
        return geom, plan
    if mode == "auto":
        seen = getattr(A, "_hip_colplan_seen", None)
        if seen != (skey, vkey):
            try:
                A._hip_colplan_seen = (skey, vkey)
            except AttributeError:
                pass
            return None
    geom = np.zeros(10, dtype=np.int64)
    _lib.call("tsp_csr_colplan_geometry", m, n, nnz, rows_per_block_log2, tiles_hint, geom.ctypes.data)
    plan = torch.empty(int(geom[6]), dtype=torch.uint8, device=dev)
    work = torch.empty(int(geom[7]), dtype=torch.uint8, device=dev)
    _lib.call("tsp_csr_colplan_build", vals.data_ptr(), _lib.TSP_F32, cols.data_ptr(), ptrs.data_ptr(),
              _lib.index_code(cols.dtype), m, n, nnz, geom.ctypes.data, plan.data_ptr(), work.data_ptr(),
              _lib.stream_handle(dev))
    try:
        A._hip_colplan = (skey, vkey, geom, plan, 1)
    except AttributeError:
        pass
    return geom, plan


def _csr_plan(ptrs: torch.Tensor, m: int, nnz: int, dev: torch.device) -> torch.Tensor:
    """SpMV work-partition table of a device CSR pattern."""
    size = _lib.load().tsp_csr_plan_size(m, nnz)
    win = torch.empty(size, dtype=torch.int64, device=dev)
    _lib.call("tsp_csr_plan", ptrs.data_ptr(), _lib.index_code(ptrs.dtype), m, nnz, win.data_ptr(), _lib.stream_handle(dev))
    return win


class _CSRMatMulFunction(torch.autograd.Function):
    """alpha * A @ X (+ beta * Y) for CSR A and dense X (vector or matrix).

    Forward: the gfx950 SpMV / SpMM kernels. Backward, on the device:
      d values[p] = alpha * <dOut[row p], X[col p]>   (tsp_csr_sddmm, pattern fixed)
      dX          = alpha * A^T @ dOut                (tsp_csr_transpose, then SpMV / SpMM)
      dY          = beta * dOut
    """

    @staticmethod
    def forward(ctx, values, col_indices, row_ptrs, shape, X, alpha, Y, beta, prepared):
        vals, cols, ptrs, win, colplan = prepared
        dev = vals.device
        out = _csr_forward(vals, cols, ptrs, win, shape, X, alpha, Y, beta, dev, colplan)
        ctx.save_for_backward(values, X)
        ctx.pattern = (cols, ptrs)
        ctx.shape, ctx.alpha, ctx.beta, ctx.has_y = shape, alpha, beta, Y is not None and beta != 0.0
        ctx.y_meta = (Y.device, Y.dtype, Y.shape) if Y is not None else None
        return out.to(X.device)

    @staticmethod
    def backward(ctx, g):
        values, X = ctx.saved_tensors
        cols, ptrs = ctx.pattern
        dev = cols.device
        m, n = ctx.shape
        vdt = values.dtype
        gd = g.to(dev, vdt).contiguous()
        Xd = X.to(dev, vdt).contiguous()
        nnz = cols.numel()
        st = _lib.stream_handle(dev)
        gv = gx = gy = None
        with torch.cuda.device(dev):
            if ctx.needs_input_grad[0]:
                ncols = gd.shape[1] if gd.dim() == 2 else 1
                gvd = torch.empty(nnz, dtype=vdt, device=dev)
                _lib.call("tsp_csr_sddmm", cols.data_ptr(), ptrs.data_ptr(), _lib.index_code(cols.dtype), m, n, nnz,
                          gd.data_ptr(), ncols, Xd.data_ptr(), ncols, ncols, _lib.dtype_code(vdt), float(ctx.alpha),
                          gvd.data_ptr(), st)
                gv = gvd.to(values.device)
            if ctx.needs_input_grad[4]:
                from . import formats as hf

                tv, tc, tp = hf.csr_transpose(values.to(dev).contiguous(), cols, ptrs, (m, n))
                win = _csr_plan(tp, n, nnz, dev) if gd.dim() == 1 else None
                gxd = _csr_forward(tv, tc, tp, win, (n, m), gd, ctx.alpha, None, 0.0, dev)
                gx = gxd.to(X.device, X.dtype)
        if ctx.needs_input_grad[6] and ctx.has_y:
            ydev, ydt, yshape = ctx.y_meta
            gy = (ctx.beta * gd).sum_to_size(yshape).to(ydev, ydt)
        return gv, None, None, None, gx, None, gy, None, None


def _csr_apply(A, X, alpha, Y, beta):
    dev = _target_device(X, A.values)
    with torch.cuda.device(dev):
        prepared = _csr_device(A, dev)
        colplan = None
        if X.dim() == 1 and _spmv_plan_mode == "bucketed":
            colplan = ("bucketed",) + _csr_bucket_plan(A, prepared[2], dev)
        elif X.dim() == 1:
            cp = _csr_colplan(A, *prepared[:3], dev)
            colplan = ("colplan",) + cp if cp is not None else None
        prepared = prepared + (colplan,)
        return _CSRMatMulFunction.apply(A.values, A.col_indices, A.row_ptrs, tuple(A.shape), X, alpha, Y, beta, prepared)


@_library_call
def hip_spmv(A, x: torch.Tensor, alpha: float = 1.0, y: torch.Tensor | None = None, beta: float = 0.0) -> torch.Tensor:
    """CSR SpMV entry point (the reference's spmv runs torch.sparse_csr @ x, ops.py:30-48)."""
    return _csr_apply(A, x, alpha, y, beta)


@_library_call
def hip_spmm(A, B: torch.Tensor, alpha: float = 1.0, C: torch.Tensor | None = None, beta: float = 0.0) -> torch.Tensor:
    """CSR SpMM entry point (replaces nki_spmm, reference dispatch.py:181-190)."""
    return _csr_apply(A, B, alpha, C, beta)


# ---------------------------------------------------------------- screened


def _screened_forward(A, diag, threshold, B, dev):
    import math

    M, K = A.shape
    if A.dtype != B.dtype:
        raise RuntimeError(f"screened_spmm: A dtype {A.dtype} and B dtype {B.dtype} differ")
    if A.dtype in (torch.bfloat16, torch.float16):
        # 16-bit A and B: widened on the device (exact), the fp32 kernel, one
        # rounding of C back to A's dtype; the mask stays in diag's precision
        return _screened_forward(_on(A, dev, torch.float32), diag, threshold, _on(B, dev, torch.float32),
                                 dev).to(A.dtype)
    if A.dtype not in (torch.float32, torch.float64):
        raise RuntimeError(f"HIP screened_spmm supports float32, float64, bfloat16 and float16, got {A.dtype}")
    if diag.dtype not in (torch.float32, torch.float64):
        raise RuntimeError(f"HIP screened_spmm needs float32 or float64 diag_integrals, got {diag.dtype}")
    if B.dim() != 2 or B.shape[0] != K:
        raise RuntimeError(f"screened_spmm: B shape {tuple(B.shape)} does not match A {tuple(A.shape)}")
    Ad, Bd, dd = _on(A, dev), _on(B, dev), _on(diag, dev)
    ncols = Bd.shape[1]
    return _lib.ops().screened_spmm(Ad, dd, Bd, math.sqrt(threshold))


def _screened_backward(A, diag, threshold, B, G, need_a: bool, need_b: bool, dev):
    """(dA, dB) of C = (A * mask) @ B through tsp_screened_spmm_backward: dA =
    (dC @ B^T) * mask, dB = (A * mask)^T @ dC, the mask never formed (reference
    dispatch.py:478-484 builds it). 16-bit operands are widened to fp32 on the
    device and the gradients rounded back once, as in the forward."""
    import math

    if A.dtype in (torch.bfloat16, torch.float16):
        dA, dB = _screened_backward(_on(A, dev, torch.float32), diag, threshold, _on(B, dev, torch.float32),
                                    _on(G, dev, torch.float32), need_a, need_b, dev)
        return (dA.to(A.dtype) if dA is not None else None, dB.to(A.dtype) if dB is not None else None)
    Ad, Bd, Gd, dd = _on(A, dev), _on(B, dev), _on(G, dev, A.dtype), _on(diag, dev)
    dA, dB = _lib.ops().screened_spmm_backward(Ad, dd, Bd, math.sqrt(threshold), Gd, bool(need_a), bool(need_b))
    return (dA if need_a else None, dB if need_b else None)


class _ScreenedSpMMFunction(torch.autograd.Function):
    """Autograd wrapper of the fused screened SpMM (reference dispatch.py:447-484).

    Forward: the gfx950 kernel (mask applied while staging A tiles).
    Backward: tsp_screened_spmm_backward, dA = (dC @ B^T) * mask and dB =
    (A * mask)^T @ dC with fully masked tile pairs skipped; no gradient to
    diag_integrals or threshold (the mask is discrete).
    """

    @staticmethod
    def forward(ctx, A, diag_integrals, threshold, B):
        dev = _target_device(B, A, diag_integrals)
        with torch.cuda.device(dev):
            C = _screened_forward(A, diag_integrals, threshold, B, dev)
        ctx.save_for_backward(A, diag_integrals, B)
        ctx.threshold = threshold
        return C.to(B.device)

    @staticmethod
    def backward(ctx, grad_out):
        A, diag, B = ctx.saved_tensors
        need_a, need_b = ctx.needs_input_grad[0], ctx.needs_input_grad[3]
        if not (need_a or need_b):
            return None, None, None, None
        dev = _target_device(B, A, diag)
        with torch.cuda.device(dev):
            dA, dB = _screened_backward(A, diag, ctx.threshold, B, grad_out, need_a, need_b, dev)
        return (dA.to(A.device) if dA is not None else None, None, None,
                dB.to(B.device) if dB is not None else None)


@_library_call
def hip_screened_spmm(A, diag_integrals, B, threshold: float):
    """Screened SpMM entry point (replaces nki_screened_spmm, reference dispatch.py:487-494)."""
    return _ScreenedSpMMFunction.apply(A, diag_integrals, threshold, B)


# --------------------------------------------------------------- attention


def _fused_d512(t: torch.Tensor, block_size: int, scale: float) -> bool:
    """bf16 with 256 < head_dim <= 512 runs the one-pass d = 512 MFMA kernel
    (operands zero-padded to 512); other head_dims over 256 run as block
    products."""
    return t.dtype == torch.bfloat16 and block_size == 128 and 256 < t.shape[-1] <= 512 and scale > 0


def _mfma_head_dim(t: torch.Tensor, block_size: int) -> int | None:
    """The head_dim an fp32 / bf16 operand of head_dim d < 256 other than 64
    and 128 is zero-padded to (64, 128 or 256), and a bf16 one with
    256 < d < 512 to 512, so that the MFMA attention kernels serve it (zero
    columns change neither the scores nor the other columns of the
    results); None when no padding applies."""
    d = t.shape[-1]
    if block_size != 128 or t.dtype not in (torch.float32, torch.bfloat16) or d in (64, 128, 256, 512) or d == 0:
        return None
    if d > 256:
        return 512 if t.dtype == torch.bfloat16 and d < 512 else None
    return 64 if d < 64 else (128 if d < 128 else 256)


def _pad_head_dim(t: torch.Tensor, dp: int) -> torch.Tensor:
    return torch.nn.functional.pad(t, (0, dp - t.shape[-1]))


@_library_call
def hip_block_sparse_attention(Q, K, V, mask_bsr, scale: float, return_stats: bool = False):
    """Block-sparse attention forward (replaces nki_bsr_attn_tiled, reference
    dispatch.py:580-677). Q/K/V (S, D) or (..., S, D) sharing one mask.
    Honours `scale` (the reference NKI path used head_dim**-0.5 regardless).
    Stats come back as (..., S // b, b) in float32 (float64 for float64 input).
    fp32 / bf16 with 128-blocks run the MFMA kernels at head_dim 64, 128 and
    256 (bf16 also 512), and on operands zero-padded to the next of those;
    the other head_dims over 256 run as block products over the mask stacked
    over heads (SDDMM scores, an elementwise block softmax, a BSR SpMM with
    V) when the sequence is a whole number of 128-blocks; fp16 runs in fp32
    (widened operands, O rounded back once).
    """
    if not (Q.shape == K.shape == V.shape):
        raise RuntimeError(f"Q, K, V shapes differ: {tuple(Q.shape)}, {tuple(K.shape)}, {tuple(V.shape)}")
    if not (Q.dtype == K.dtype == V.dtype):
        raise RuntimeError("Q, K, V dtypes differ")
    if Q.dtype == torch.float16:  # widened to fp32 (exact), O rounded back once
        res = hip_block_sparse_attention(Q.float(), K.float(), V.float(), mask_bsr, scale, return_stats)
        return res.half() if not return_stats else (res[0].half(),) + tuple(res[1:])
    dp = _mfma_head_dim(Q, mask_bsr.block_size)
    if dp is not None and scale > 0:
        res = hip_block_sparse_attention(*(_pad_head_dim(t, dp) for t in (Q, K, V)), mask_bsr, scale, return_stats)
        if not return_stats:
            return res[..., : Q.shape[-1]].contiguous()
        return (res[0][..., : Q.shape[-1]].contiguous(),) + tuple(res[1:])
    fused = _fused_d512(Q, mask_bsr.block_size, scale)
    bd = _blocks_head_dim(Q, mask_bsr.block_size) if Q.shape[-1] > 256 and not fused else None
    if bd is not None:
        # head_dim over 256: block products over the mask stacked over heads
        d = Q.shape[-1]
        lead, S = Q.shape[:-2], Q.shape[-2]
        orig = Q.device
        dev = _target_device(Q, K, V)
        with torch.cuda.device(dev):
            Qd, Kd, Vd = (_pad_head_dim(_on(t, dev).reshape(math.prod(lead), S, d), bd).contiguous() for t in (Q, K, V))
            O, rmax, rden = _attention_blocks_fwd(Qd, Kd, Vd, mask_bsr, scale, dev)
        out = O[..., :d].reshape(*lead, S, d).to(orig)
        if not return_stats:
            return out
        return out, rmax.reshape(*lead, S // 128, 128).to(orig), rden.reshape(*lead, S // 128, 128).to(orig)
    _lib.dtype_code(Q.dtype)  # raises for a dtype the kernels do not take
    lead = Q.shape[:-2]
    S, D = Q.shape[-2:]
    b = mask_bsr.block_size
    Mt = S // b
    orig = Q.device
    dev = _target_device(Q, K, V)
    with torch.cuda.device(dev):
        rp, ci, _ = _bsr_plan(mask_bsr.block_col_indices, mask_bsr.block_row_ptrs,
                              mask_bsr.block_row_ptrs.numel() - 1, dev, holder=mask_bsr)
        if rp.numel() < Mt + 1:
            raise IndexError(f"mask has {rp.numel() - 1} block rows, attention needs {Mt}")
        Qd, Kd, Vd = (_on(t, dev).reshape(math.prod(lead), S, D) for t in (Q, K, V))
        H = Qd.shape[0]
        O, rmax, rden = _lib.ops().bsa_fwd(Qd, Kd, Vd, rp, ci, b, float(scale), bool(return_stats))
    out = O.reshape(*lead, S, D).to(orig)
    if not return_stats:
        return out
    return out, rmax.reshape(*lead, Mt, b).to(orig), rden.reshape(*lead, Mt, b).to(orig)


def _attn_bwd_plan(mask_bsr, H: int, S: int, dev: torch.device):
    """Column view of the mask restricted to the block rows below S // b and
    the column-pass plan (tsp_bsa_bwd_plan), built on the host and copied to
    the device. Cached on the mask's column-index tensor, keyed by the
    pattern's identity and version and (H, S, device).

    Returns (col_ptrs, col_block_rows, n_block_cols, plan, header) with
    header = (n_items, n_splits, n_partials).
    """
    b = mask_bsr.block_size
    Mt = S // b
    ci_t, rp_t = mask_bsr.block_col_indices, mask_bsr.block_row_ptrs
    key = (rp_t.data_ptr(), rp_t._version, rp_t.numel(), ci_t._version, ci_t.numel(), int(mask_bsr.shape[1]), H, S,
           str(dev))
    hit = getattr(ci_t, "_tsp_attn_bwd_plan", None)
    if hit is not None and hit[0] == key:
        return hit[1]
    rp = rp_t.detach().to("cpu", torch.int64).numpy()
    ci = ci_t.detach().to("cpu", torch.int64).numpy()
    end = int(rp[Mt])
    ci = ci[:end]
    nbc = (int(mask_bsr.shape[1]) + b - 1) // b
    if ci.size:
        nbc = max(nbc, int(ci.max()) + 1)
    brow = np.repeat(np.arange(Mt, dtype=np.int64), np.diff(rp[: Mt + 1]))
    order = np.argsort(ci * max(Mt, 1) + brow, kind="stable")
    crow = np.ascontiguousarray(brow[order])
    cp = np.zeros(nbc + 1, dtype=np.int64)
    if ci.size:
        cp[1:] = np.cumsum(np.bincount(ci, minlength=nbc))
    lib = _lib.load()
    n = lib.tsp_bsa_bwd_plan(cp.ctypes.data, nbc, H, S, b, None, 0)
    if n < 4:
        raise RuntimeError(f"tsp_bsa_bwd_plan failed: {_lib.last_error()}")
    plan = np.empty(n, dtype=np.int32)
    if lib.tsp_bsa_bwd_plan(cp.ctypes.data, nbc, H, S, b, plan.ctypes.data, n) != n:
        raise RuntimeError(f"tsp_bsa_bwd_plan failed: {_lib.last_error()}")
    header = (int(plan[0]), int(plan[1]), int(plan[2]))
    out = (torch.from_numpy(cp).to(dev), torch.from_numpy(crow if crow.size else np.zeros(1, np.int64)).to(dev), nbc,
           torch.from_numpy(plan).to(dev), header)
    try:
        ci_t._tsp_attn_bwd_plan = (key, out, rp_t)  # the row pointers kept alive with the entry
    except AttributeError:
        pass
    return out


# ------------------------------------------- attention as block products
#
# Head_dims the one-pass kernels do not hold in registers (over 256 except
# the bf16 forward up to 512; bf16 gradients at 256 and over) run as
# block-sparse products over the mask stacked over
# heads: stacked block row h * Mt + i holds mask block row i shifted by h * Mt
# block columns, so (H, S, D) operands are its (H * S, D) dense operands.
# Scores and score gradients are SDDMMs on that pattern (tsp_bsr_sddmm_ex,
# fp32 blocks), the softmax and its gradient are elementwise passes over the
# blocks (tsp_bsa_block_softmax, tsp_bsa_block_grad), and O, dQ, dK, dV are
# BSR SpMMs (tsp_bsr_spmm, tsp_bsr_spmm_t): every product on MFMA.


def _blocks_head_dim(t: torch.Tensor, block_size: int) -> int | None:
    """Head_dim the block-product path runs a (..., S, D) fp32 / bf16 operand
    at (D rounded up to a multiple of 8, the SDDMM's vector width), or None
    when the path does not apply (block size other than 128, a sequence that
    is not a whole number of blocks)."""
    S, d = t.shape[-2:]
    if block_size != 128 or t.dtype not in (torch.float32, torch.bfloat16) or S == 0 or S % 128 or d == 0:
        return None
    return (d + 7) // 8 * 8


def _attn_stack_plan(mask_bsr, H: int, S: int, dev: torch.device):
    """The mask's block rows below Mt = S // 128 and block columns below Mt
    (keys at or past S do not exist), stacked over H heads: (rp, ci, order,
    brow, cp, cbid, crow, corder, nnzb). Built on the host from the pattern
    and cached on the mask's column-index tensor, keyed by the pattern's
    identity and version and (H, S, device)."""
    b = mask_bsr.block_size
    Mt = S // b
    ci_t, rp_t = mask_bsr.block_col_indices, mask_bsr.block_row_ptrs
    key = (rp_t.data_ptr(), rp_t._version, rp_t.numel(), ci_t.data_ptr(), ci_t._version, ci_t.numel(), H, S,
           str(dev))
    hit = getattr(ci_t, "_tsp_attn_stack_plan", None)
    if hit is not None and hit[0] == key:
        return hit[1]
    rp = rp_t.detach().to("cpu", torch.int64).numpy()
    ci = ci_t.detach().to("cpu", torch.int64).numpy()
    if rp.size < Mt + 1:
        raise IndexError(f"mask has {rp.size - 1} block rows, attention needs {Mt}")
    brow0 = np.repeat(np.arange(Mt, dtype=np.int64), np.diff(rp[: Mt + 1]))
    col0 = ci[: int(rp[Mt])]
    keep = col0 < Mt
    brow0, col0 = brow0[keep], col0[keep]
    counts = np.bincount(brow0, minlength=Mt).astype(np.int64)
    shift = (Mt * np.arange(H, dtype=np.int64))[:, None]
    col = (col0[None, :] + shift).reshape(-1)
    rps = np.zeros(H * Mt + 1, dtype=np.int64)
    rps[1:] = np.cumsum(np.tile(counts, H))
    nbr = H * Mt
    rp_d = torch.from_numpy(rps).to(dev)
    ci_d = torch.from_numpy(col if col.size else np.zeros(0, np.int64)).to(dev)
    order = torch.empty(max(nbr, 1), dtype=torch.int32, device=dev)
    _lib.call("tsp_bsr_row_order", rp_d.data_ptr(), nbr, order.data_ptr(), _lib.stream_handle(dev))
    brow, cp, cbid, crow, corder = _bsr_bwd_plan(rp_d, ci_d, nbr, nbr, dev)
    out = (rp_d, ci_d, order, brow, cp, cbid, crow, corder, int(col.size))
    try:
        ci_t._tsp_attn_stack_plan = (key, out, rp_t)  # the row pointers kept alive with the entry
    except AttributeError:
        pass
    return out


def _block_scores(A: torch.Tensor, B: torch.Tensor, plan, dev) -> torch.Tensor:
    """fp32 blocks A B^T on the stacked pattern (A, B (rows, D) in fp32 / bf16)."""
    rp, ci, _, brow, _, _, _, _, nnzb = plan
    rows, D = A.shape
    out = torch.empty((max(nnzb, 1), 128, 128), dtype=torch.float32, device=dev)
    _lib.call("tsp_bsr_sddmm_ex", A.data_ptr(), D, rows, B.data_ptr(), D, rows, D, brow.data_ptr(), ci.data_ptr(), nnzb,
              128, _lib.dtype_code(A.dtype), out.data_ptr(), _lib.TSP_F32, _lib.stream_handle(dev))
    return out


def _attention_blocks_fwd(Qd, Kd, Vd, mask_bsr, scale: float, dev):
    """(O, row_max, row_denom) of (H, S, D) fp32 / bf16 operands on the
    block-product path; stats (H, S // 128, 128) fp32."""
    H, S, D = Qd.shape
    rows = H * S
    dt = Qd.dtype
    plan = _attn_stack_plan(mask_bsr, H, S, dev)
    rp, ci, order, _, _, _, _, _, nnzb = plan
    Sb = _block_scores(Qd.reshape(rows, D), Kd.reshape(rows, D), plan, dev)
    P = Sb if dt == torch.float32 else torch.empty(Sb.shape, dtype=dt, device=dev)
    rmax = torch.empty(rows, dtype=torch.float32, device=dev)
    rden = torch.empty(rows, dtype=torch.float32, device=dev)
    _lib.call("tsp_bsa_block_softmax", Sb.data_ptr(), rp.data_ptr(), rp.numel() - 1, 128, float(scale), P.data_ptr(),
              _lib.dtype_code(dt), rmax.data_ptr(), rden.data_ptr(), _lib.stream_handle(dev))
    del Sb
    O = _lib.ops().bsr_spmm(P[:nnzb], rp, ci, order, rows, rows, 128, Vd.reshape(rows, D), dt)
    Mt = S // 128
    return O.reshape(H, S, D), rmax.reshape(H, Mt, 128), rden.reshape(H, Mt, 128)


def _attention_blocks_bwd(q, k, v, o, do, mask_bsr, scale: float, rm, rd, dev):
    """(dQ, dK, dV) of (H, S, D) fp32 / bf16 operands on the block-product
    path, from the forward's O and fp32 stats."""
    H, S, D = q.shape
    rows = H * S
    dt = q.dtype
    plan = _attn_stack_plan(mask_bsr, H, S, dev)
    rp, ci, order, brow, cp, cbid, crow, corder, nnzb = plan
    q2, k2, v2, o2, do2 = (t.reshape(rows, D) for t in (q, k, v, o, do))
    st = _lib.stream_handle(dev)
    Drow = torch.empty(rows, dtype=torch.float32, device=dev)
    _lib.call("tsp_bsa_rowdot", o2.data_ptr(), do2.data_ptr(), _lib.dtype_code(dt), rows, D, Drow.data_ptr(), st)
    if dt == torch.float32:
        # fp32 scores as blocks, P and dS written over them
        Sb = _block_scores(q2, k2, plan, dev)
        dPb = _block_scores(do2, v2, plan, dev)
        _lib.call("tsp_bsa_block_grad", Sb.data_ptr(), dPb.data_ptr(), brow.data_ptr(), nnzb, 128, float(scale),
                  rm.data_ptr(), rd.data_ptr(), Drow.data_ptr(), Sb.data_ptr(), dPb.data_ptr(), _lib.TSP_F32, st)
        P, dS = Sb, dPb
    else:
        # bf16: both score products and the gradient in one kernel
        P = torch.empty((max(nnzb, 1), 128, 128), dtype=dt, device=dev)
        dS = torch.empty_like(P)
        _lib.call("tsp_bsa_block_pgrad", q2.data_ptr(), k2.data_ptr(), v2.data_ptr(), do2.data_ptr(),
                  _lib.dtype_code(dt), rows, D, brow.data_ptr(), ci.data_ptr(), nnzb, 128, float(scale), rm.data_ptr(),
                  rd.data_ptr(), Drow.data_ptr(), P.data_ptr(), dS.data_ptr(), st)
    ops = _lib.ops()
    dV = ops.bsr_spmm_t(P[:nnzb], cp, cbid, crow, corder, rows, rows, 128, do2)
    dK = ops.bsr_spmm_t(dS[:nnzb], cp, cbid, crow, corder, rows, rows, 128, q2)
    dQ = ops.bsr_spmm(dS[:nnzb], rp, ci, order, rows, rows, 128, k2, dt)
    return dQ.reshape(H, S, D), dK.reshape(H, S, D), dV.reshape(H, S, D)


@_library_call
def hip_block_sparse_attention_backward(Q, K, V, O, dO, mask_bsr, scale: float, row_max, row_denom):
    """Block-sparse attention backward (replaces nki_bsr_attn_bwd, reference
    dispatch.py:813-929, and the torch backward ops.py:360-473).

    Q/K/V/O/dO (S, D) or (..., S, D) sharing one mask; row_max / row_denom
    as hip_block_sparse_attention returns them. Returns (dQ, dK, dV).

    bf16 with 128-blocks: head_dims below 128 are zero-padded to 128 and
    run the bf16 MFMA kernels of head_dim 128 (zero columns change neither
    the scores nor the other gradient columns, and those kernels run at
    several times the rate of the fp32 ones on widened operands). bf16 at
    head_dim 256, and fp32 / bf16 at head_dims over 256, run as block
    products over the mask stacked over heads (SDDMMs for S and dP, the
    elementwise softmax gradient, BSR SpMMs for dQ, dK, dV) when the
    sequence is a whole number of 128-blocks. Other head_dims below 256 are
    zero-padded to 64, 128 or 256 first, as in the forward.
    """
    if not (Q.shape == K.shape == V.shape == O.shape == dO.shape):
        raise RuntimeError("Q, K, V, O, dO shapes differ")
    if Q.dtype == torch.float16:  # widened to fp32 (exact), gradients rounded back once
        grads = hip_block_sparse_attention_backward(*(t.float() for t in (Q, K, V, O, dO)), mask_bsr, scale,
                                                    row_max, row_denom)
        return tuple(gr.half() for gr in grads)
    if Q.dtype == torch.bfloat16 and 0 < Q.shape[-1] < 128 and mask_bsr.block_size == 128 and scale > 0:
        grads = hip_block_sparse_attention_backward(*(_pad_head_dim(t, 128) for t in (Q, K, V, O, dO)), mask_bsr,
                                                    scale, row_max, row_denom)
        return tuple(gr[..., : Q.shape[-1]].contiguous() for gr in grads)
    dp = _mfma_head_dim(Q, mask_bsr.block_size) if Q.shape[-1] <= 256 else None  # over 256: block products
    if dp is not None and scale > 0:
        grads = hip_block_sparse_attention_backward(*(_pad_head_dim(t, dp) for t in (Q, K, V, O, dO)), mask_bsr, scale,
                                                    row_max, row_denom)
        return tuple(gr[..., : Q.shape[-1]].contiguous() for gr in grads)
    d = Q.shape[-1]
    bd = _blocks_head_dim(Q, mask_bsr.block_size) if (d > 256 or (d == 256 and Q.dtype == torch.bfloat16)) else None
    if bd is not None:
        # block products over the mask stacked over heads (bf16 at 256: on the
        # bf16 MFMA kernels instead of the fp32 ones on widened operands)
        lead, S = Q.shape[:-2], Q.shape[-2]
        orig = Q.device
        dev = _target_device(Q, K, V, O, dO)
        with torch.cuda.device(dev):
            q, k, v, o, do = (_pad_head_dim(_on(t, dev, Q.dtype).reshape(math.prod(lead), S, d), bd).contiguous()
                              for t in (Q, K, V, O, dO))
            H = q.shape[0]
            rm = _on(row_max, dev, torch.float32).reshape(H, S)
            rd = _on(row_denom, dev, torch.float32).reshape(H, S)
            grads = _attention_blocks_bwd(q, k, v, o, do, mask_bsr, scale, rm, rd, dev)
        return tuple(g[..., :d].reshape(*lead, S, d).to(orig) for g in grads)
    dt = Q.dtype
    _lib.dtype_code(dt)  # raises for a dtype the kernels do not take
    lead = Q.shape[:-2]
    S, D = Q.shape[-2:]
    b = mask_bsr.block_size
    Mt = S // b
    orig = Q.device
    dev = _target_device(Q, K, V, O, dO)
    sdt = torch.float64 if dt == torch.float64 else torch.float32
    with torch.cuda.device(dev):
        mb = mask_bsr.block_row_ptrs.numel() - 1
        if mb < Mt:
            raise IndexError(f"mask has {mb} block rows, attention needs {Mt}")
        rp, ci, _ = _bsr_plan(mask_bsr.block_col_indices, mask_bsr.block_row_ptrs, mb, dev, holder=mask_bsr)
        q, k, v, o, do = (_on(t, dev, dt).reshape(math.prod(lead), S, D) for t in (Q, K, V, O, dO))
        H = q.shape[0]
        cp, crow, nbc, plan, (n_items, n_splits, n_partials) = _attn_bwd_plan(mask_bsr, H, S, dev)
        rm = _on(row_max, dev, sdt).reshape(H, Mt * b)
        rd = _on(row_denom, dev, sdt).reshape(H, Mt * b)
        dQ, dK, dV = _lib.ops().bsa_bwd(q, k, v, o, do, rp, ci, cp, crow, nbc, b, float(scale), rm, rd, plan, n_items,
                                        n_splits, n_partials)
    return tuple(g.reshape(*lead, S, D).to(orig) for g in (dQ, dK, dV))
