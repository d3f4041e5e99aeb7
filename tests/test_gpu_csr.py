"""GPU parity of CSR spmv / spmm (HIP kernels via the C ABI) against the oracle.

Known answers from the reference tests (tests/test_ops.py), the reference's
hardware SpMM grid (tests/test_nki_spmm.py:42-50), edge cases of the window
partition (empty rows, all-empty matrix, rows longer than a window), and the
full-size BASELINE config 2 (Poisson and Zipf rows, int64 and int32 indices)
against the C oracle with a float64 accumulator. fp32 tolerance: max error
<= 1e-4 relative to the (|A|.|x|)_i scale.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import trnsparse_amd as ts
from oracle import build as oracle_c
from oracle import ref
from trnsparse_amd import workloads as W

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _np(A: ts.CSRMatrix):
    return A.values.cpu().numpy(), A.col_indices.cpu().numpy(), A.row_ptrs.cpu().numpy(), A.shape


def _check_spmv(A, x, got, alpha=1.0, y=None, beta=0.0):
    v, c, p, sh = _np(A)
    xn = x.cpu().numpy()
    yn = None if y is None else y.cpu().numpy()
    exact = ref.csr_spmv(v, c, p, sh, xn, alpha, yn, beta)
    scale = ref.csr_spmv(v, c, p, sh, xn, alpha, yn, beta, absolute=True)
    err = ref.scaled_error(got.cpu().numpy(), exact, scale)
    assert err <= TOL, err


# ---------------------------------------------------- reference known answers


def test_spmv_identity(hip_backend):
    I = ts.eye_sparse(4)
    x = torch.tensor([1.0, 2.0, 3.0, 4.0])
    np.testing.assert_allclose(ts.spmv(I, x).numpy(), x.numpy())


def test_spmv_vs_dense_3x3(hip_backend):
    A = torch.tensor([[1.0, 0.0, 2.0], [0.0, 3.0, 0.0], [4.0, 0.0, 5.0]])
    x = torch.tensor([1.0, 2.0, 3.0])
    np.testing.assert_allclose(ts.spmv(ts.from_dense(A), x).numpy(), (A @ x).numpy(), atol=1e-6)


def test_spmv_alpha_beta_known_answer(hip_backend):
    csr = ts.from_dense(torch.tensor([[2.0, 0.0], [0.0, 3.0]]))
    y = torch.tensor([10.0, 20.0])
    out = ts.spmv(csr, torch.ones(2), alpha=2.0, y=y, beta=0.5)
    np.testing.assert_array_equal(out.numpy(), [9.0, 16.0])
    assert y.tolist() == [10.0, 20.0]  # y is not modified
    out = ts.spmv(csr, torch.ones(2), alpha=2.0, y=y, beta=0.0)
    np.testing.assert_array_equal(out.numpy(), [4.0, 6.0])


def test_spmv_large_sparse_seed42(hip_backend):
    torch.manual_seed(42)
    A = torch.randn(100, 100)
    A[torch.abs(A) < 1.5] = 0.0
    x = torch.randn(100)
    csr = ts.from_dense(A)
    np.testing.assert_allclose(ts.spmv(csr, x).numpy(), (A @ x).numpy(), atol=1e-5)


def test_spmm_known_answers(hip_backend):
    I = ts.eye_sparse(3)
    B = torch.tensor([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]])
    np.testing.assert_allclose(ts.spmm(I, B).numpy(), B.numpy())
    A = torch.tensor([[1.0, 0.0, 2.0], [0.0, 3.0, 0.0]])
    Bm = torch.tensor([[1.0, 0.0], [0.0, 1.0], [2.0, 3.0]])
    np.testing.assert_allclose(ts.spmm(ts.from_dense(A), Bm).numpy(), (A @ Bm).numpy(), atol=1e-6)
    out = ts.spmm(ts.from_dense(torch.eye(2)), torch.ones(2, 3), alpha=2.0, C=torch.ones(2, 3) * 10, beta=0.5)
    np.testing.assert_array_equal(out.numpy(), np.full((2, 3), 7.0))


@pytest.mark.parametrize("M,K,N,density", [(128, 128, 128, 0.1), (256, 256, 128, 0.05), (256, 256, 128, 0.01),
                                           (512, 256, 256, 0.05), (200, 137, 64, 0.05), (300, 500, 700, 0.02)])
def test_spmm_reference_grid(hip_backend, M, K, N, density):
    g = torch.Generator().manual_seed(0)
    dense = torch.randn(M, K, generator=g) * (torch.rand(M, K, generator=g) < density)
    A = ts.from_dense(dense)
    B = torch.randn(K, N)
    got = ts.spmm(A, B.cuda()).cpu()
    torch.testing.assert_close(got, dense @ B, atol=1e-3, rtol=1e-4)
    v, c, p, sh = _np(A)
    exact = ref.csr_spmm(v, c, p, sh, B.numpy())
    scale = ref.csr_spmm(v, c, p, sh, B.numpy(), absolute=True)
    assert ref.scaled_error(got.numpy(), exact, scale) <= TOL


@pytest.mark.parametrize("N", [4, 8, 12, 16, 20, 32, 60, 64, 100, 128, 132, 260])
@pytest.mark.parametrize("index_dtype", [np.int64, np.int32])
def test_spmm_narrow_b(hip_backend, N, index_dtype):
    """fp32 B with a multiple of 4 columns runs the narrow kernel (several
    rows per wavefront, a row's nonzeros split over lane groups, 128-column
    passes): rows of 0..300 nonzeros, alpha and beta with C."""
    lens = list(np.random.default_rng(N).poisson(12, 3000).clip(0, 300)) + [0, 300, 1, 97]
    A = _csr_from_lengths(lens, 2000, seed=N, index_dtype=index_dtype)
    g = torch.Generator().manual_seed(N)
    B = torch.randn(2000, N, generator=g)
    C = torch.randn(len(lens), N, generator=g)
    got = ts.spmm(A, B.cuda(), alpha=0.5, C=C.cuda(), beta=-2.0).cpu()
    v, c, p, sh = _np(A)
    exact = 0.5 * ref.csr_spmm(v, c, p, sh, B.numpy()) - 2.0 * C.numpy()
    scale = 0.5 * ref.csr_spmm(v, c, p, sh, B.numpy(), absolute=True) + 2.0 * np.abs(C.numpy())
    assert ref.scaled_error(got.numpy(), exact, scale) <= TOL


@pytest.mark.parametrize("N", [0, 1, 3, 8, 64, 130])
@pytest.mark.parametrize("index_dtype", [np.int64, np.int32])
def test_csr_matmul_backward_on_device(hip_backend, N, index_dtype):
    """Autograd of alpha * A @ X on the device (N = 0: the SpMV form): the
    values gradient through tsp_csr_sddmm, dX through the device transpose
    and SpMV / SpMM, both against float64 closed forms."""
    lens = list(np.random.default_rng(5).poisson(6, 400).clip(0, 50)) + [0, 120]
    A = _csr_from_lengths(lens, 300, seed=9, index_dtype=index_dtype)
    g = torch.Generator().manual_seed(N)
    vals = A.values.cuda().requires_grad_(True)
    X = (torch.randn(300, N, generator=g) if N else torch.randn(300, generator=g)).cuda().requires_grad_(True)
    Ad = ts.CSRMatrix(vals, A.col_indices.cuda(), A.row_ptrs.cuda(), A.shape)
    out = ts.spmm(Ad, X, alpha=1.5) if N else ts.spmv(Ad, X, alpha=1.5)
    G = torch.randn(out.shape, generator=g).cuda()
    out.backward(G)
    v, c, p, _ = _np(A)
    rows = np.repeat(np.arange(len(lens)), np.diff(p))
    Gn = G.double().cpu().numpy().reshape(len(lens), -1)
    Xn = X.detach().double().cpu().numpy().reshape(300, -1)
    exact_v = 1.5 * (Gn[rows] * Xn[c]).sum(axis=1)
    scale_v = 1.5 * (np.abs(Gn[rows]) * np.abs(Xn[c])).sum(axis=1)
    assert ref.scaled_error(vals.grad.double().cpu().numpy(), exact_v, scale_v) <= TOL
    exact_x = np.zeros_like(Xn)
    scale_x = np.zeros_like(Xn)
    np.add.at(exact_x, c, 1.5 * v[:, None].astype(np.float64) * Gn[rows])
    np.add.at(scale_x, c, 1.5 * np.abs(v[:, None].astype(np.float64) * Gn[rows]))
    assert ref.scaled_error(X.grad.double().cpu().numpy().reshape(300, -1), exact_x, scale_x) <= TOL


# ---------------------------------------------------- partition edge cases


def _csr_from_lengths(lens, n, seed, index_dtype=np.int64):
    vals, cols, ptr = W.random_csr(lens, n, np.random.default_rng(seed))
    return W.csr_matrix_from_arrays(vals, cols.astype(index_dtype), ptr.astype(index_dtype), (len(lens), n))


@pytest.mark.parametrize(
    "lens",
    [
        [0] * 5000,  # all rows empty
        [0, 0, 3, 0, 0] * 1000,  # sparse rows, many empty
        [1] * 10000,  # more rows than a window holds
        [5000] + [3] * 100 + [9000] + [0] * 50 + [2],  # rows longer than a window
        [2047, 1, 4095, 4096, 4097, 1, 0, 6000],  # lengths around the LDS capacity
        list(np.random.default_rng(3).zipf(1.5, 20000).clip(1, 4096)),  # skewed
    ],
    ids=["all_empty", "mostly_empty", "unit_rows", "long_rows", "lds_edges", "zipf_small"],
)
@pytest.mark.parametrize("index_dtype", [np.int64, np.int32])
def test_spmv_partition_edges(hip_backend, lens, index_dtype):
    A = _csr_from_lengths(lens, 20000, seed=len(lens), index_dtype=index_dtype)
    x = torch.randn(20000)
    y = torch.randn(len(lens))
    got = ts.spmv(A, x.cuda(), alpha=0.75, y=y.cuda(), beta=-1.5)
    _check_spmv(A, x, got, 0.75, y, -1.5)


def test_spmv_f64(hip_backend):
    A = _csr_from_lengths([7, 0, 130, 1], 200, seed=1)
    A64 = ts.CSRMatrix(A.values.double(), A.col_indices, A.row_ptrs, A.shape)
    x = torch.randn(200, dtype=torch.float64)
    got = ts.spmv(A64, x.cuda()).cpu()
    torch.testing.assert_close(got, A64.to_dense() @ x, rtol=1e-12, atol=1e-12)


def test_spmv_matrix_operand_routes_to_spmm(hip_backend):
    A = _csr_from_lengths([3, 4, 0, 5], 50, seed=2)
    X = torch.randn(50, 3)
    torch.testing.assert_close(ts.spmv(A, X.cuda()).cpu(), A.to_dense() @ X, atol=1e-5, rtol=1e-5)


def test_spmv_dimension_mismatch_asserts(hip_backend):
    with pytest.raises(AssertionError):
        ts.spmv(ts.eye_sparse(4), torch.ones(5).cuda())


def test_spmm_gradcheck_f64(hip_backend):
    A = _csr_from_lengths([2, 0, 3, 1], 6, seed=4)
    vals = A.values.double().cuda().requires_grad_(True)
    B = torch.randn(6, 3, dtype=torch.float64, device="cuda", requires_grad=True)

    def f(v, b):
        return ts.spmm(ts.CSRMatrix(v, A.col_indices.cuda(), A.row_ptrs.cuda(), A.shape), b, alpha=1.5)

    assert torch.autograd.gradcheck(f, (vals, B), eps=1e-6, atol=1e-6)


# ---------------------------------------------------- BASELINE config 2


@pytest.mark.parametrize("dist", ["poisson", "zipf"])
@pytest.mark.parametrize("index_dtype", [np.int64, np.int32])
def test_cfg2_full_size(hip_backend, dist, index_dtype):
    """The windowed kernel (deterministic: a repeat call is bit-identical);
    the column-sorted plan path has its own tests (test_gpu_csr_colplan.py)."""
    from trnsparse_amd.hip import dispatch as D

    prev = D.get_spmv_plan()
    D.set_spmv_plan("never")
    try:
        _cfg2_windowed(dist, index_dtype)
    finally:
        D.set_spmv_plan(prev)


def _cfg2_windowed(dist, index_dtype):
    v, c, p, x, shape = W.cfg2_csr(dist=dist, index_dtype=index_dtype)
    A = W.csr_matrix_from_arrays(v, c, p, shape, device="cuda")
    xd = torch.from_numpy(x).cuda()
    got = ts.spmv(A, xd).cpu().numpy()
    exact = oracle_c.csr_spmv_f64(v, c, p, shape[0], x)
    scale = oracle_c.csr_spmv_f64(v, c, p, shape[0], x, absolute=True)
    assert ref.scaled_error(got, exact, scale) <= TOL
    # checksum property: sum(y) = colsum(A) . x
    colsum = np.bincount(c.astype(np.int64), weights=v.astype(np.float64), minlength=shape[1])
    assert abs(got.astype(np.float64).sum() - colsum @ x) <= TOL * float(np.abs(v).astype(np.float64) @ np.abs(x[c]))
    # repeat call through the cached plan is bit-identical
    assert np.array_equal(ts.spmv(A, xd).cpu().numpy(), got)
