"""Zero-size dimensions and strided inputs through the public API on the
hip backend, against the same call on the torch ("pytorch") backend, which
restates the reference's CPU path (trnsparse/ops.py). Empty operands must
give empty or zero results of the reference's shapes, never a launch error;
non-contiguous views must give the results of their contiguous copies.
"""

from __future__ import annotations

import pytest
import torch

import trnsparse_amd as ts
from trnsparse_amd import workloads as W

pytestmark = pytest.mark.gpu


def _both(fn):
    """fn() on the pytorch backend (CPU inputs) and on the hip backend."""
    prev = ts.get_backend()
    try:
        ts.set_backend("pytorch")
        want = fn("cpu")
        ts.set_backend("hip")
        got = fn("cuda")
    finally:
        ts.set_backend(prev)
    return want, got


def _same(want, got, tol=1e-5):
    assert got.shape == want.shape and got.dtype == want.dtype
    torch.testing.assert_close(got.cpu(), want, rtol=tol, atol=tol)


def _csr(m, n, dev, density=0.3, seed=0):
    g = torch.Generator().manual_seed(seed)
    d = torch.randn(m, n, generator=g) * (torch.rand(m, n, generator=g) < density)
    A = ts.from_dense(d)
    return ts.CSRMatrix(values=A.values.to(dev), col_indices=A.col_indices.to(dev), row_ptrs=A.row_ptrs.to(dev),
                        shape=A.shape)


@pytest.mark.parametrize("m,n", [(0, 7), (5, 0), (0, 0)])
def test_spmv_spmm_empty_dims(hip_backend, m, n):
    want, got = _both(lambda dev: ts.spmv(_csr(m, n, dev), torch.ones(n, device=dev)))
    _same(want, got)
    want, got = _both(lambda dev: ts.spmm(_csr(m, n, dev), torch.ones(n, 3, device=dev)))
    _same(want, got)


def test_spmm_zero_columns(hip_backend):
    want, got = _both(lambda dev: ts.spmm(_csr(40, 30, dev), torch.ones(30, 0, device=dev)))
    _same(want, got)


def test_bsr_spmm_zero_columns_and_rows(hip_backend):
    g = torch.Generator().manual_seed(1)
    dense = torch.randn(256, 256, generator=g)

    def run(dev, ncols):
        A = ts.BSRMatrix.from_dense(dense.to(dev), block_size=128)
        return ts.bsr_spmm(A, torch.ones(256, ncols, device=dev))

    for ncols in (0, 1, 5):
        want, got = _both(lambda dev: run(dev, ncols))
        _same(want, got, 1e-4)


def test_attention_empty_sequence(hip_backend):
    bsr = W.bsr_from_block_mask(torch.ones(1, 1, dtype=torch.bool), 128)
    want, got = _both(lambda dev: ts.block_sparse_attention_tiled(*(torch.zeros(2, 0, 64, device=dev)
                                                                   for _ in range(3)), bsr))
    _same(want, got)


def test_screened_empty(hip_backend):
    want, got = _both(lambda dev: ts.screened_spmm(torch.zeros(0, 0, device=dev), torch.zeros(0, device=dev),
                                                   torch.zeros(0, 4, device=dev), 1e-8))
    _same(want, got)
    want, got = _both(lambda dev: ts.screened_spmm(torch.ones(6, 6, device=dev), torch.ones(6, device=dev),
                                                   torch.zeros(6, 0, device=dev), 1e-8))
    _same(want, got)


def test_strided_views(hip_backend):
    """x[::2], a transposed B and permuted (B, S, H, D) -> (B, H, S, D) views."""
    g = torch.Generator().manual_seed(3)
    xx = torch.randn(2 * 300, generator=g)
    Bt = torch.randn(24, 256, generator=g)
    dense = torch.randn(256, 256, generator=g) * (torch.rand(256, 256, generator=g) < 0.5)
    qkv = torch.randn(3, 1, 256, 2, 64, generator=g)
    bsr = W.bsr_from_block_mask(W.cfg5_block_mask(2), 128)

    want, got = _both(lambda dev: ts.spmv(_csr(200, 300, dev, seed=4), xx.to(dev)[::2]))
    _same(want, got)
    want, got = _both(lambda dev: ts.bsr_spmm(ts.BSRMatrix.from_dense(dense.to(dev), block_size=128), Bt.to(dev).T))
    _same(want, got, 1e-4)
    want, got = _both(lambda dev: ts.block_sparse_attention_tiled(*(t.to(dev).permute(0, 2, 1, 3) for t in qkv), bsr))
    _same(want, got, 1e-4)


@pytest.mark.parametrize("mode", ["never", "always"])
def test_replaced_host_values_are_not_served_from_cache(hip_backend, mode):
    """A host-resident CSR matrix whose values tensor is replaced: the new
    tensor may be allocated where the freed one was, with the same version
    counter; the device copies cached on the matrix keep their source
    tensors alive, so the key cannot match and the product uses the new
    values."""
    from oracle import ref
    from trnsparse_amd.hip import dispatch as D

    prev = D.get_spmv_plan()
    D.set_spmv_plan(mode)
    try:
        A = _csr(3000, 2000, "cpu", density=0.01, seed=7)
        x = torch.randn(2000, generator=torch.Generator().manual_seed(8))
        nnz = A.values.numel()
        for rep in range(4):
            y = ts.spmv(A, x.cuda()).cpu()
            want = ref.csr_spmv(A.values.numpy(), A.col_indices.numpy(), A.row_ptrs.numpy(), A.shape, x.numpy())
            scale = ref.csr_spmv(A.values.numpy(), A.col_indices.numpy(), A.row_ptrs.numpy(), A.shape, x.numpy(),
                                 absolute=True)
            assert ref.scaled_error(y.numpy(), want, scale) <= 1e-4, rep
            A.values = None                                   # free the old values first
            A.values = torch.randn(nnz, generator=torch.Generator().manual_seed(20 + rep))
    finally:
        D.set_spmv_plan(prev)
