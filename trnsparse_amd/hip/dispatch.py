"""HIP dispatch: the MI355X side of the ops seam.

Replaces the reference's NKI dispatch layer (trnsparse/nki/dispatch.py):
each `hip_*` function is what `ops.py` calls when the HIP backend is in
effect. It places operands on the GPU (inputs on the host are copied over
and the result is returned on the caller's device, as the reference's
`_to_xla` / `.to(orig_device)` round trip does, dispatch.py:88-94),
prepares the cached per-pattern plan, allocates outputs and calls the C ABI
on the current HIP stream. Autograd wrappers keep the reference's
signatures; their backward passes run as torch ops on the device.

Kernel failures raise RuntimeError; nothing falls back to another path.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib


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
            holder._hip_plan = (key, plan)
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
    ldb = ncols
    if B_d.dtype == torch.float32 and b == 128 and ncols % 4:
        # Row stride multiple of 4 floats for the vectorised B panel loads.
        B_d = F.pad(B_d, (0, 4 - ncols % 4))
        ldb = B_d.shape[1]
    C = torch.empty((m, ncols), dtype=out_dtype, device=dev)
    _lib.call(
        "tsp_bsr_spmm",
        blocks_d.data_ptr(),
        _lib.dtype_code(blocks_d.dtype),
        rp.data_ptr(),
        ci.data_ptr(),
        blocks_d.shape[0],
        b,
        m,
        n,
        B_d.data_ptr(),
        ldb,
        ncols,
        C.data_ptr(),
        ncols,
        _lib.dtype_code(out_dtype),
        order.data_ptr() if order is not None else None,
        _lib.stream_handle(dev),
    )
    return C


class _BSRSpMMFunction(torch.autograd.Function):
    """Autograd wrapper of BSR SpMM (reference dispatch.py:290-369).

    Forward: the gfx950 kernel. Backward (torch ops on the device):
      dA_blocks[k] = dC[row block of k] @ B[col block of k]^T
      dB           = A^T @ dC  (per stored block, scattered by column block)
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
        work = torch.float64 if A_blocks.dtype == torch.float64 else torch.float32
        blocks = A_blocks.to(dev, work)
        go = torch.zeros(mb * b, ncols, dtype=work, device=dev)
        go[:m] = grad_out.to(dev, work)
        Bp = torch.zeros(nbc * b, ncols, dtype=work, device=dev)
        Bp[:n] = B.to(dev, work)
        counts = rp[1:] - rp[:-1]
        rows = torch.repeat_interleave(torch.arange(mb, device=dev), counts)
        go_panels = go.view(mb, b, ncols)[rows]
        grad_blocks = grad_B = None
        if ctx.needs_input_grad[0]:
            B_panels = Bp.view(nbc, b, ncols)[ci]
            grad_blocks = torch.bmm(go_panels, B_panels.transpose(1, 2).contiguous())
            grad_blocks = grad_blocks.to(A_blocks.device, A_blocks.dtype)
        if ctx.needs_input_grad[5]:
            contrib = torch.bmm(blocks.transpose(1, 2).contiguous(), go_panels)
            dB = torch.zeros(nbc, b, ncols, dtype=work, device=dev).index_add_(0, ci, contrib)
            grad_B = dB.view(nbc * b, ncols)[:n].to(B.device, B.dtype)
        return grad_blocks, None, None, None, None, grad_B, None, None


def hip_bsr_spmm(A, B: torch.Tensor, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """BSR SpMM entry point (replaces nki_bsr_spmm, reference dispatch.py:372-381)."""
    m, _ = A.shape
    b = A.block_size
    dev = _target_device(B, A.blocks)
    with torch.cuda.device(dev):
        plan = _bsr_plan(A.block_col_indices, A.block_row_ptrs, (m + b - 1) // b, dev, holder=A)
    return _BSRSpMMFunction.apply(
        A.blocks, A.block_col_indices, A.block_row_ptrs, A.shape, A.block_size, B, out_dtype, plan
    )
