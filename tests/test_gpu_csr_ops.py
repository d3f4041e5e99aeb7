"""GPU versions of the remaining CSR ops — sparse_add, sparse_transpose,
spmv_symmetric — against the CPU torch path (restating the reference's
ops.py:81-154) and the oracle. Structure bit-exact; sparse_add values exact
for at most two duplicates per coordinate (a + b rounds the same either
way), otherwise within fp32 1e-6 relative; spmv_symmetric fp32 <= 1e-4
against the dot-product scale.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import trnsparse_amd as ts
from oracle import ref
from trnsparse_amd import workloads as W

pytestmark = pytest.mark.gpu


def _csr(m, n, density, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(m, n, generator=g, dtype=torch.float64) * (torch.rand(m, n, generator=g) < density)
    return ts.from_dense(A.to(dtype))


def _cuda(A: ts.CSRMatrix) -> ts.CSRMatrix:
    return ts.CSRMatrix(A.values.cuda(), A.col_indices.cuda(), A.row_ptrs.cuda(), A.shape)


def _same_structure(got: ts.CSRMatrix, want: ts.CSRMatrix):
    assert got.shape == want.shape
    assert torch.equal(got.row_ptrs.cpu(), want.row_ptrs.cpu().to(torch.int64))
    assert torch.equal(got.col_indices.cpu(), want.col_indices.cpu().to(torch.int64))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("m,n,da,db", [(200, 150, 0.05, 0.08), (64, 64, 0.5, 0.0), (1, 500, 0.3, 0.3)])
def test_sparse_add_matches_cpu(hip_backend, dtype, m, n, da, db):
    A, B = _csr(m, n, da, 1, dtype), _csr(m, n, db, 2, dtype)
    got = ts.sparse_add(_cuda(A), _cuda(B), alpha=2.0, beta=-0.5)
    assert got.values.is_cuda
    ts.set_backend("pytorch")
    try:
        want = ts.sparse_add(A, B, alpha=2.0, beta=-0.5)
    finally:
        ts.set_backend("hip")
    _same_structure(got, want)
    assert torch.equal(got.values.cpu(), want.values)
    v, c, p = ref.sparse_add((A.values.numpy(), A.col_indices.numpy(), A.row_ptrs.numpy(), A.shape),
                             (B.values.numpy(), B.col_indices.numpy(), B.row_ptrs.numpy(), B.shape), 2.0, -0.5)
    np.testing.assert_array_equal(got.row_ptrs.cpu().numpy(), p)
    np.testing.assert_array_equal(got.col_indices.cpu().numpy(), c)
    np.testing.assert_allclose(got.values.cpu().double().numpy(), v, rtol=1e-6 if dtype == torch.float32 else 1e-14)


def test_sparse_add_duplicates_and_cancellation(hip_backend):
    """Duplicates inside an operand are summed; an exact cancellation keeps
    an explicit zero entry (torch's coalesce keeps it)."""
    A = ts.CSRMatrix(torch.tensor([1.0, 2.0, 3.0]), torch.tensor([2, 2, 0]), torch.tensor([0, 2, 3]), (2, 3))
    B = ts.CSRMatrix(torch.tensor([-3.0, 5.0]), torch.tensor([2, 1]), torch.tensor([0, 1, 2]), (2, 3))
    got = ts.sparse_add(_cuda(A), _cuda(B))
    ts.set_backend("pytorch")
    try:
        want = ts.sparse_add(A, B)
    finally:
        ts.set_backend("hip")
    _same_structure(got, want)
    assert torch.equal(got.values.cpu(), want.values)
    assert got.values.cpu().tolist() == [0.0, 3.0, 5.0]  # (0, 2): 1 + 2 - 3 kept as an explicit zero


def test_sparse_add_unsorted_rows_with_repeats(hip_backend):
    """Both operands with unsorted columns inside rows and repeated
    coordinates (within A, within B and across): one entry per coordinate,
    sorted, duplicates summed in input order (A's before B's) — bit-exact
    against the CPU path, whose coalesce sorts the concatenated COO."""
    g = torch.Generator().manual_seed(9)
    m, n = 40, 7
    def rand_csr(nnz):
        rows = torch.sort(torch.randint(0, m, (nnz,), generator=g)).values
        cols = torch.randint(0, n, (nnz,), generator=g)
        vals = torch.randn(nnz, generator=g)
        rp = torch.zeros(m + 1, dtype=torch.int64)
        rp[1:] = torch.bincount(rows, minlength=m).cumsum(0)
        return ts.CSRMatrix(vals, cols, rp, (m, n))
    A, B = rand_csr(150), rand_csr(90)
    got = ts.sparse_add(_cuda(A), _cuda(B), alpha=0.5, beta=3.0)
    ts.set_backend("pytorch")
    try:
        want = ts.sparse_add(A, B, alpha=0.5, beta=3.0)
    finally:
        ts.set_backend("hip")
    _same_structure(got, want)
    np.testing.assert_allclose(got.values.cpu().double().numpy(), want.values.double().numpy(), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_sparse_add_wide_columns(hip_backend, dtype):
    """Columns past 2^26 take the 64-bit (column, position) sort keys of the
    wavefront kernel: rows whose union holds up to 32 entries (two rows per
    wavefront) and 33-64 entries (one row over all lanes), a few longer
    rows, repeats inside rows, columns spread up to n - 1."""
    rng = np.random.default_rng(11)
    m, n = 300, (1 << 27) + 5

    def rand_csr(lo, hi):
        lens = rng.integers(lo, hi, m)
        lens[::9] = rng.integers(20, 31, len(lens[::9]))  # unions of 40-60 entries
        lens[5] = 40                                      # a union past 64: the LDS kernel
        cols, vals = [], []
        for k in lens:
            pool = rng.integers(0, n, max(1, int(k) // 2 + 1))
            pool[0] = n - 1
            cols.append(rng.choice(pool, int(k)))         # repeats inside the row
            vals.append(rng.standard_normal(int(k)))
        rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        c = np.concatenate(cols).astype(np.int64)
        v = np.concatenate(vals)
        return v, c, rp

    (va, ca, pa), (vb, cb, pb) = rand_csr(0, 17), rand_csr(0, 17)
    A = ts.CSRMatrix(torch.from_numpy(va).to(dtype).cuda(), torch.from_numpy(ca).cuda(), torch.from_numpy(pa).cuda(),
                     (m, n))
    B = ts.CSRMatrix(torch.from_numpy(vb).to(dtype).cuda(), torch.from_numpy(cb).cuda(), torch.from_numpy(pb).cuda(),
                     (m, n))
    got = ts.sparse_add(A, B, alpha=2.0, beta=-0.5)
    v, c, p = ref.sparse_add((A.values.cpu().double().numpy(), ca, pa, (m, n)),
                             (B.values.cpu().double().numpy(), cb, pb, (m, n)), 2.0, -0.5)
    np.testing.assert_array_equal(got.row_ptrs.cpu().numpy(), p)
    np.testing.assert_array_equal(got.col_indices.cpu().numpy(), c)
    tol = 1e-6 if dtype == torch.float32 else 1e-12
    np.testing.assert_allclose(got.values.cpu().double().numpy(), v, rtol=tol, atol=tol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_sparse_add_long_rows(hip_backend, dtype):
    """Rows of every size class of the device coalesce: more than 4096
    entries (a workgroup per row, streamed through LDS in tiles), 65-4096
    (staged in LDS with their neighbours), at most 64 (a wavefront sort) and
    empty; many repeats per column."""
    g = torch.Generator().manual_seed(11)
    m, n = 6, 600
    def csr(counts):
        rows = torch.repeat_interleave(torch.arange(m), torch.tensor(counts))
        cols = torch.randint(0, n, (int(sum(counts)),), generator=g)
        vals = torch.randn(int(sum(counts)), generator=g, dtype=torch.float64).to(dtype)
        rp = torch.zeros(m + 1, dtype=torch.int64)
        rp[1:] = torch.tensor(counts).cumsum(0)
        return ts.CSRMatrix(vals, cols, rp, (m, n))
    A, B = csr([3000, 10, 0, 5000, 80, 1500]), csr([2500, 0, 0, 4100, 30, 900])
    got = ts.sparse_add(_cuda(A), _cuda(B), alpha=1.0, beta=-2.0)
    ts.set_backend("pytorch")
    try:
        want = ts.sparse_add(A, B, alpha=1.0, beta=-2.0)
    finally:
        ts.set_backend("hip")
    _same_structure(got, want)
    np.testing.assert_allclose(got.values.cpu().double().numpy(), want.values.double().numpy(),
                               rtol=1e-5 if dtype == torch.float32 else 1e-12, atol=1e-5 if dtype == torch.float32 else 1e-12)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16])
@pytest.mark.parametrize("m,n,density", [(300, 200, 0.05), (1, 40, 0.5), (50, 1, 0.5), (128, 128, 0.0)])
def test_sparse_transpose_matches_cpu(hip_backend, dtype, m, n, density):
    A = _csr(m, n, density, 3, dtype)
    got = ts.sparse_transpose(_cuda(A))
    assert got.values.is_cuda and got.values.dtype == dtype and got.shape == (n, m)
    want = ts.sparse_transpose(A)
    _same_structure(got, want)
    assert torch.equal(got.values.cpu(), want.values)
    v, c, p = ref.csr_transpose(A.values.float().numpy(), A.col_indices.numpy(), A.row_ptrs.numpy(), A.shape)
    np.testing.assert_array_equal(got.row_ptrs.cpu().numpy(), p)
    np.testing.assert_array_equal(got.col_indices.cpu().numpy(), c)


def test_sparse_transpose_duplicates_and_unsorted_columns(hip_backend):
    """A CSR with unsorted columns inside rows and repeated (row, col)
    entries: rows ascend within each output row and repeats keep their input
    order, as the reference's stable sort by (col, row) leaves them."""
    vals = torch.arange(1.0, 10.0)
    cols = torch.tensor([3, 0, 3, 1, 2, 2, 0, 3, 1])
    rp = torch.tensor([0, 3, 3, 6, 9])  # row 1 empty
    A = ts.CSRMatrix(vals, cols, rp, (4, 5))
    got = ts.sparse_transpose(_cuda(A))
    want = ts.sparse_transpose(A)
    _same_structure(got, want)
    assert torch.equal(got.values.cpu(), want.values)
    assert got.values.cpu().tolist() == [2.0, 7.0, 4.0, 9.0, 5.0, 6.0, 1.0, 3.0, 8.0]
    assert got.row_ptrs.cpu().tolist() == [0, 2, 4, 6, 9, 9]


@pytest.mark.parametrize("n,density", [(500, 0.02), (2048, 0.005)])
def test_spmv_symmetric_matches_oracle(hip_backend, n, density):
    g = torch.Generator().manual_seed(n)
    D = torch.randn(n, n, generator=g, dtype=torch.float64) * (torch.rand(n, n, generator=g) < density)
    U = ts.from_dense(torch.triu(D).float())
    x = torch.randn(n, generator=g)
    y = ts.spmv_symmetric(_cuda(U), x.cuda(), alpha=1.5)
    args = (U.values.numpy(), U.col_indices.numpy(), U.row_ptrs.numpy(), U.shape, x.numpy())
    exact = ref.spmv_symmetric(*args, alpha=1.5)
    scale = ref.spmv_symmetric(*args, alpha=1.5, absolute=True)
    assert ref.scaled_error(y.cpu().numpy(), exact, scale) <= 1e-4
    y2 = ts.spmv_symmetric(_cuda(U), x.cuda(), alpha=1.5)  # cached transpose
    assert torch.equal(y, y2)


def test_cfg2_scale_transpose_and_add(hip_backend):
    """cfg2 (1 M x 1 M, Poisson(16) rows, int64): transpose twice gives A
    back bit for bit; A + A^T has the union pattern of A and A^T (count
    identity nnz(A + A^T) = 2 nnz(A) - nnz(A o A^T) checked through the
    transposed pattern)."""
    v, c, p, _, shape = W.cfg2_csr(dist="poisson", index_dtype=np.int64)
    A = ts.CSRMatrix(torch.from_numpy(v).cuda(), torch.from_numpy(c).cuda(), torch.from_numpy(p).cuda(), shape)
    T = ts.sparse_transpose(A)
    TT = ts.sparse_transpose(T)
    _same_structure(TT, A)
    assert torch.equal(TT.values, A.values)
    S = ts.sparse_add(A, T)
    both = S.nnz
    # entries present in both A and A^T: sort keys of A and of A^T, intersect
    ka = (A.to_coo().row_indices * shape[1] + A.col_indices)
    kt = (T.to_coo().row_indices * shape[1] + T.col_indices)
    common = int(torch.isin(ka, kt).sum())
    assert both == 2 * A.nnz - common
