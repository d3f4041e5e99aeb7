"""GPU format construction (csrc/formats.hip) against the CPU path and the
oracle: structure bit-exact (row pointers, column indices), values exact
(the kernels only move them; CSR to_dense adds duplicates in entry order).

The CPU side is the torch path of trnsparse_amd.formats on CPU tensors
(vectorised restatements of the reference's torch code, trnsparse/
formats.py) and oracle.ref (numpy). bf16 matrices go to the oracle as
float32 arrays of the same values with the threshold rounded to bf16, as
torch compares a bf16 tensor with a Python float.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import trnsparse_amd as ts
from oracle import ref
from trnsparse_amd import workloads as W

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float64, torch.bfloat16]


def _np(t):
    return t.detach().float().cpu().numpy() if t.dtype == torch.bfloat16 else t.detach().cpu().numpy()


def _thr(thr, dtype):
    """The threshold as the comparison sees it (rounded to the dtype)."""
    return float(torch.tensor(thr, dtype=dtype).item()) if dtype != torch.float64 else thr


def _matrix(m, n, density, dtype, seed, nan_at=None):
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(m, n, generator=g, dtype=torch.float64) * (torch.rand(m, n, generator=g) < density)
    A = A.to(dtype)
    if nan_at is not None:
        A[nan_at] = float("nan")
    return A


def _same_bsr(got: ts.BSRMatrix, want: ts.BSRMatrix):
    assert got.shape == want.shape and got.block_size == want.block_size
    assert torch.equal(got.block_row_ptrs.cpu(), want.block_row_ptrs.cpu())
    assert torch.equal(got.block_col_indices.cpu(), want.block_col_indices.cpu())
    assert got.blocks.dtype == want.blocks.dtype
    assert torch.equal(got.blocks.cpu(), want.blocks.cpu())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(
    "m,n,b,density,thr",
    [
        (512, 384, 128, 0.002, 0.0),  # mostly empty blocks
        (300, 260, 128, 0.01, 0.0),   # ragged: padded edge blocks
        (300, 260, 128, 0.01, -1.0),  # negative threshold keeps every block (padding zeros pass)
        (96, 72, 8, 0.05, 0.5),       # small blocks, threshold
        (37, 91, 16, 0.2, 1.2),
        (0, 40, 8, 0.5, 0.0),         # no rows
    ],
)
def test_bsr_from_dense_matches_cpu_and_oracle(hip_backend, dtype, m, n, b, density, thr):
    A = _matrix(m, n, density, dtype, seed=m + n + b)
    got = ts.BSRMatrix.from_dense(A.cuda(), block_size=b, threshold=thr)
    assert got.blocks.is_cuda and got.block_row_ptrs.is_cuda
    want = ts.BSRMatrix.from_dense(A, block_size=b, threshold=thr)  # CPU torch path
    _same_bsr(got, want)
    blocks, col, ptr, shape = ref.bsr_from_dense(_np(A), b, _thr(thr, dtype))
    np.testing.assert_array_equal(got.block_row_ptrs.cpu().numpy(), ptr)
    np.testing.assert_array_equal(got.block_col_indices.cpu().numpy(), col)
    np.testing.assert_array_equal(_np(got.blocks), blocks)


@pytest.mark.parametrize("dtype", DTYPES)
def test_bsr_from_dense_nan_and_threshold_rounding(hip_backend, dtype):
    """A NaN drops its block (max|v| is NaN); values just above / at the
    threshold after rounding to the dtype decide like torch's compare."""
    b = 16
    A = torch.zeros(64, 64, dtype=dtype)
    A[0, 0] = 5.0
    A[1, 1] = float("nan")        # block (0, 0): 5 and NaN -> not kept
    A[20, 3] = 0.1                # block (1, 0): 0.1 vs threshold 0.1
    A[40, 40] = 0.25              # block (2, 2): kept
    A[63, 63] = -7.0              # block (3, 3): |v| kept
    for thr in (0.1, 0.0999, 0.2):
        got = ts.BSRMatrix.from_dense(A.cuda(), block_size=b, threshold=thr)
        want = ts.BSRMatrix.from_dense(A, block_size=b, threshold=thr)
        _same_bsr(got, want)
        assert 0 not in got.block_col_indices[: int(got.block_row_ptrs[1])].tolist()


@pytest.mark.parametrize("dtype", DTYPES)
def test_bsr_to_dense_matches_cpu(hip_backend, dtype):
    A = _matrix(300, 260, 0.01, dtype, seed=5)
    bsr = ts.BSRMatrix.from_dense(A, block_size=128)
    got = ts.BSRMatrix(bsr.blocks.cuda(), bsr.block_col_indices.cuda(), bsr.block_row_ptrs.cuda(), bsr.shape,
                       128).to_dense()
    assert got.is_cuda and got.shape == (300, 260)
    assert torch.equal(got.cpu(), bsr.to_dense())
    assert torch.equal(got.cpu(), A)


def test_bsr_to_dense_repeated_and_unsorted_blocks(hip_backend):
    """The reference's loop writes stored blocks in order, so a repeated
    block's last entry wins; columns need not be sorted."""
    b = 8
    blocks = torch.arange(4 * b * b, dtype=torch.float32).reshape(4, b, b)
    col = torch.tensor([2, 0, 2, 1])
    ptr = torch.tensor([0, 3, 4])
    bsr = ts.BSRMatrix(blocks, col, ptr, (16, 24), b)
    got = ts.BSRMatrix(blocks.cuda(), col.cuda(), ptr.cuda(), (16, 24), b).to_dense().cpu()
    assert torch.equal(got, bsr.to_dense())
    assert torch.equal(got[:8, 16:24], blocks[2])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,n,density,thr", [(257, 300, 0.05, 0.0), (64, 1000, 0.3, 0.7), (33, 7, 0.5, -1.0),
                                               (100, 64, 0.0, 0.0), (0, 10, 0.5, 0.0)])
def test_csr_from_dense_matches_cpu_and_oracle(hip_backend, dtype, m, n, density, thr):
    A = _matrix(m, n, density, dtype, seed=m * 7 + n, nan_at=(m // 2, n // 3) if m and n else None)
    got = ts.from_dense(A.cuda(), threshold=thr)
    assert got.values.is_cuda and got.row_ptrs.is_cuda
    want = ts.from_dense(A, threshold=thr)
    assert torch.equal(got.row_ptrs.cpu(), want.row_ptrs)
    assert torch.equal(got.col_indices.cpu(), want.col_indices)
    assert torch.equal(got.values.cpu(), want.values)
    v, c, p = ref.csr_from_dense(_np(A), _thr(thr, dtype))
    np.testing.assert_array_equal(got.row_ptrs.cpu().numpy(), p)
    np.testing.assert_array_equal(got.col_indices.cpu().numpy(), c)
    np.testing.assert_array_equal(_np(got.values), v)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_csr_to_dense_and_to_coo(hip_backend, dtype):
    A = _matrix(120, 90, 0.1, dtype, seed=8)
    csr = ts.from_dense(A)
    dev = ts.CSRMatrix(csr.values.cuda(), csr.col_indices.cuda(), csr.row_ptrs.cuda(), csr.shape)
    assert torch.equal(dev.to_dense().cpu(), A)
    coo = dev.to_coo()
    want = csr.to_coo()
    assert torch.equal(coo.row_indices.cpu(), want.row_indices)
    assert torch.equal(coo.col_indices.cpu(), want.col_indices)
    # duplicates in a row add up in entry order (torch's sparse CSR to_dense)
    vals = torch.tensor([1.0, 2.0, 5.0, 0.5], dtype=dtype)
    cols = torch.tensor([1, 1, 0, 1])
    ptrs = torch.tensor([0, 3, 4])
    got = ts.CSRMatrix(vals.cuda(), cols.cuda(), ptrs.cuda(), (2, 3)).to_dense().cpu()
    assert torch.equal(got, ts.CSRMatrix(vals, cols, ptrs, (2, 3)).to_dense())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(
    "m,n",
    [
        (500, 700),        # 32-bit sort keys; duplicates likely
        (65535, 65537),    # m * n = 2^32 - 1: the largest shape on 32-bit keys
        (65536, 65536),    # m * n = 2^32: 64-bit keys
        (100000, 50000),   # 64-bit keys
    ],
)
def test_coo_to_csr_matches_cpu_and_oracle(hip_backend, dtype, m, n):
    g = torch.Generator().manual_seed(21)
    nnz = 20000
    rows = torch.randint(0, m, (nnz,), generator=g)
    cols = torch.randint(0, n, (nnz,), generator=g)
    rows[:3] = torch.tensor([m - 1, m - 1, 0])  # the largest and smallest keys
    cols[:3] = torch.tensor([n - 1, n - 2, 0])
    vals = torch.randn(nnz, generator=g).to(dtype)
    got = ts.COOMatrix(vals.cuda(), rows.cuda(), cols.cuda(), (m, n)).to_csr()
    want = ts.COOMatrix(vals, rows, cols, (m, n)).to_csr()
    assert torch.equal(got.row_ptrs.cpu(), want.row_ptrs)
    assert torch.equal(got.col_indices.cpu(), want.col_indices)
    assert torch.equal(got.values.cpu(), want.values)
    v, c, p = ref.coo_to_csr(_np(vals), rows.numpy(), cols.numpy(), (m, n))
    np.testing.assert_array_equal(got.row_ptrs.cpu().numpy(), p)
    np.testing.assert_array_equal(got.col_indices.cpu().numpy(), c)
    np.testing.assert_array_equal(_np(got.values), v)
    empty = ts.COOMatrix(vals[:0].cuda(), rows[:0].cuda(), cols[:0].cuda(), (4, 5)).to_csr()
    assert empty.row_ptrs.cpu().tolist() == [0] * 5 and empty.nnz == 0


@pytest.mark.parametrize("nnz", [1, 2, 2047, 2048, 2049, 4095, 4096, 4097, 12289])
@pytest.mark.parametrize("kind", ["random", "equal", "two"])
def test_coo_to_csr_tile_edges_and_stability(hip_backend, nnz, kind):
    """The device radix sort at its tile boundaries (2048- and 4096-key
    tiles), a single entry, and all-equal or two-valued keys, where only
    stability fixes the order: compared bit for bit with a stable numpy sort."""
    from trnsparse_amd.hip import formats as HF

    g = torch.Generator().manual_seed(nnz)
    m, n = 300, 257
    if kind == "random":
        rows = torch.randint(0, m, (nnz,), generator=g)
        cols = torch.randint(0, n, (nnz,), generator=g)
    elif kind == "equal":
        rows = torch.full((nnz,), 7)
        cols = torch.full((nnz,), 255)
    else:
        pick = torch.randint(0, 2, (nnz,), generator=g)
        rows = torch.where(pick == 1, torch.tensor(m - 1), torch.tensor(0))
        cols = torch.where(pick == 1, torch.tensor(0), torch.tensor(n - 1))
    vals = torch.arange(nnz, dtype=torch.float32)  # the value is the input position
    key = rows.numpy() * n + cols.numpy()
    order = np.argsort(key, kind="stable")
    v, c, p = HF.coo_to_csr(vals.cuda(), rows.cuda(), cols.cuda(), (m, n))
    np.testing.assert_array_equal(v.cpu().numpy(), vals.numpy()[order])
    np.testing.assert_array_equal(c.cpu().numpy(), key[order] % n)
    np.testing.assert_array_equal(p.cpu().numpy(), np.searchsorted(key[order], np.arange(m + 1) * n))


def test_coo_large_sort_and_multi_level_scans(hip_backend):
    """17 M entries on a 4096 x 4096 grid (about one duplicate per cell):
    COO -> CSR sorts 8301 tiles (a two-level scan of the digit-count table)
    and the duplicate sum scans 17 M run heads (three scan levels). Integer
    values make every sum exact, so both are compared bit for bit with a
    stable numpy sort."""
    from trnsparse_amd.hip import formats as HF

    g = torch.Generator().manual_seed(31)
    m = n = 4096
    nnz = 17_000_000
    rows = torch.randint(0, m, (nnz,), generator=g)
    cols = torch.randint(0, n, (nnz,), generator=g)
    vals = torch.randint(-1000, 1001, (nnz,), generator=g).to(torch.float32)
    key = rows.numpy() * n + cols.numpy()
    order = np.argsort(key, kind="stable")
    ks = key[order]
    # COO -> CSR: the stable permutation
    v, c, p = HF.coo_to_csr(vals.cuda(), rows.cuda(), cols.cuda(), (m, n))
    np.testing.assert_array_equal(v.cpu().numpy(), vals.numpy()[order])
    np.testing.assert_array_equal(c.cpu().numpy(), ks % n)
    np.testing.assert_array_equal(p.cpu().numpy(), np.searchsorted(ks, np.arange(m + 1) * n))
    # duplicates summed: one entry per distinct key
    heads = np.ones(nnz, dtype=bool)
    heads[1:] = ks[1:] != ks[:-1]
    starts = np.flatnonzero(heads)
    want_v = np.add.reduceat(vals.numpy()[order].astype(np.float64), starts).astype(np.float32)
    uk = ks[starts]
    sv, sc, sp = HF.coo_sum_to_csr(vals.cuda(), rows.cuda(), cols.cuda(), (m, n))
    np.testing.assert_array_equal(sv.cpu().numpy(), want_v)
    np.testing.assert_array_equal(sc.cpu().numpy(), uk % n)
    np.testing.assert_array_equal(sp.cpu().numpy(), np.searchsorted(uk, np.arange(m + 1) * n))


def test_cfg3_round_trip_full_size(hip_backend):
    """cfg3 (16384^2, 1638 stored 128x128 blocks, fp32): to_dense then
    from_dense on the device gives back the same structure and blocks
    (no stored block is all zero), and BSR -> CSR -> BSR agrees."""
    A, _ = W.cfg3_bsr(dtype=torch.float32)
    dev = ts.BSRMatrix(A.blocks.cuda(), A.block_col_indices.cuda(), A.block_row_ptrs.cuda(), A.shape, 128)
    D = dev.to_dense()
    assert D.shape == (16384, 16384)
    back = ts.BSRMatrix.from_dense(D, block_size=128)
    _same_bsr(back, A)
    csr = ts.from_dense(D)
    assert csr.nnz == int(torch.count_nonzero(A.blocks))
    again = ts.BSRMatrix.from_csr(csr, block_size=128)
    _same_bsr(again, A)
