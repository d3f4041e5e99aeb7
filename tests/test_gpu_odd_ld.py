"""Odd output leading dimensions through the C ABI.

The fp32 DMA kernels (`bsr_spmm_f32_dma`, `bsr_spmm_t_f32_dma`,
`screened_f32_dma`) store column pairs when the output row stride is even
and fall back to single stores otherwise; the Python layer always passes
ldc = ncols, so only the C ABI reaches the odd-stride path. Each case writes
into a NaN-filled buffer with ldc = ncols + 1 and checks the values against
the oracle and that the padding column is left untouched.
"""

import math

import numpy as np
import pytest
import torch

from oracle import ref
from trnsparse_amd import workloads as W
from trnsparse_amd.hip import _lib
from trnsparse_amd.hip import dispatch as D

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")


def _bsr_case(seed, mb=3, nbc=2):
    g = torch.Generator().manual_seed(seed)
    mask = torch.rand(mb, nbc, generator=g) < 0.7
    mask[:, 0] = True
    nnzb = int(mask.sum())
    A = W.bsr_from_block_mask(mask, 128, blocks=torch.randn(nnzb, 128, 128, generator=g))
    return A, g


@pytest.mark.parametrize("ncols", [64, 129])
def test_bsr_spmm_odd_ldc(ncols):
    A, g = _bsr_case(11)
    m, n = A.shape
    ldb = (ncols + 3) // 4 * 4
    B = torch.zeros(n, ldb)
    B[:, :ncols] = torch.randn(n, ncols, generator=g)
    ldc = ncols + 1 if ncols % 2 == 0 else ncols + 2  # odd
    assert ldc % 2 == 1
    C = torch.full((m, ldc), float("nan"), device=DEV)
    rp = A.block_row_ptrs.to(DEV)
    ci = A.block_col_indices.to(DEV)
    blocks = A.blocks.to(DEV).contiguous()
    Bd = B.to(DEV)
    _lib.call("tsp_bsr_spmm", blocks.data_ptr(), _lib.TSP_F32, rp.data_ptr(), ci.data_ptr(), A.n_blocks, 128, m, n,
              Bd.data_ptr(), ldb, ncols, C.data_ptr(), ldc, _lib.TSP_F32, None, _lib.stream_handle(DEV))
    torch.cuda.synchronize()
    Ch = C.cpu().numpy()
    want = ref.bsr_spmm(A.blocks.double().numpy(), A.block_col_indices.numpy(), A.block_row_ptrs.numpy(), (m, n), 128,
                        B[:, :ncols].double().numpy())[:m]
    scale = ref.bsr_spmm(A.blocks.double().numpy(), A.block_col_indices.numpy(), A.block_row_ptrs.numpy(), (m, n), 128,
                         B[:, :ncols].double().numpy(), absolute=True)[:m]
    err = np.abs(Ch[:, :ncols] - want) / np.maximum(scale, 1e-30)
    assert err.max() < 1e-5, err.max()
    assert np.isnan(Ch[:, ncols:]).all()


def test_bsr_spmm_t_odd_ldo():
    A, g = _bsr_case(12, mb=2, nbc=3)
    m, n = A.shape
    ncols = 64
    X = torch.randn(m, ncols, generator=g)
    mb = A.block_row_ptrs.numel() - 1
    nbc = n // 128
    rp = A.block_row_ptrs.to(DEV)
    ci = A.block_col_indices.to(DEV)
    _, cp, cbid, crow, corder = D._bsr_bwd_plan(rp, ci, mb, nbc, DEV)
    blocks = A.blocks.to(DEV).contiguous()
    Xd = X.to(DEV)
    ldo = ncols + 1
    out = torch.full((n, ldo), float("nan"), device=DEV)
    _lib.call("tsp_bsr_spmm_t", blocks.data_ptr(), _lib.TSP_F32, cp.data_ptr(), cbid.data_ptr(), crow.data_ptr(), nbc,
              128, m, n, Xd.data_ptr(), ncols, ncols, out.data_ptr(), ldo, corder.data_ptr(), _lib.stream_handle(DEV))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    dense = A.to_dense().double().numpy()
    want = dense.T @ X.double().numpy()
    scale = np.abs(dense.T) @ np.abs(X.double().numpy())
    err = np.abs(got[:, :ncols] - want) / np.maximum(scale, 1e-30)
    assert err.max() < 1e-5, err.max()
    assert np.isnan(got[:, ncols:]).all()


def test_screened_spmm_odd_ldc():
    g = torch.Generator().manual_seed(13)
    m, ncols = 256, 64
    A = torch.randn(m, m, generator=g)
    diag = torch.rand(m, generator=g) + 0.1
    B = torch.randn(m, ncols, generator=g)
    thr = 0.3
    ldc = ncols + 1
    ws = torch.empty(int(_lib.load().tsp_screened_workspace_size(m, _lib.TSP_F32)), dtype=torch.uint8, device=DEV)
    Ad, dd, Bd = A.to(DEV), diag.to(DEV), B.to(DEV)
    C = torch.full((m, ldc), float("nan"), device=DEV)
    _lib.call("tsp_screened_spmm", Ad.data_ptr(), _lib.TSP_F32, m, dd.data_ptr(), _lib.TSP_F32, math.sqrt(thr), m,
              Bd.data_ptr(), ncols, ncols, C.data_ptr(), ldc, ws.data_ptr(), _lib.stream_handle(DEV))
    torch.cuda.synchronize()
    got = C.cpu().numpy()
    want = ref.screened_spmm(A.numpy(), diag.numpy(), B.numpy(), thr)  # mask in diag's fp32, as the kernel
    scale = ref.screened_spmm(A.numpy(), diag.numpy(), B.numpy(), thr, absolute=True)
    err = np.abs(got[:, :ncols] - want) / np.maximum(scale, 1e-30)
    assert err.max() < 1e-5, err.max()
    assert np.isnan(got[:, ncols:]).all()
