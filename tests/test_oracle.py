"""Pins of the CPU oracle (oracle/ref.py) against independent checks.

Each check is chosen so that a plausible mistake in the oracle (a dropped
block, a transposed operand, a wrong mask compare, a missing alpha/beta
term, an off-by-one block row) fails: closed forms via dense numpy/scipy,
the reference tests' known answers, brute force on tiny inputs.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import pytest
import scipy.sparse as sp

from oracle import ref


def _block_random(mb, nb, b, density, seed):
    rng = np.random.default_rng(seed)
    keep = rng.random((mb, nb)) < density
    A = np.zeros((mb * b, nb * b), np.float32)
    for i in range(mb):
        for j in range(nb):
            if keep[i, j]:
                A[i * b : (i + 1) * b, j * b : (j + 1) * b] = rng.standard_normal((b, b))
    return A, keep


# ------------------------------------------------------------------ BSR


def test_bsr_from_dense_brute_force():
    A, keep = _block_random(5, 4, 8, 0.4, seed=1)
    blocks, col, ptr, shape = ref.bsr_from_dense(A, 8)
    exp_cols, exp_ptr = [], [0]
    for i in range(5):
        for j in range(4):
            if np.abs(A[i * 8 : (i + 1) * 8, j * 8 : (j + 1) * 8]).max() > 0:
                exp_cols.append(j)
        exp_ptr.append(len(exp_cols))
    assert col.tolist() == exp_cols and ptr.tolist() == exp_ptr and shape == A.shape
    assert col.dtype == np.int64 and ptr.dtype == np.int64
    for idx, j in enumerate(exp_cols):
        i = np.searchsorted(ptr, idx, side="right") - 1
        np.testing.assert_array_equal(blocks[idx], A[i * 8 : (i + 1) * 8, j * 8 : (j + 1) * 8])


def test_bsr_threshold_and_empty():
    A = np.zeros((16, 16), np.float32)
    blocks, col, ptr, _ = ref.bsr_from_dense(A, 8)
    assert len(blocks) == 0 and ptr.tolist() == [0, 0, 0]
    A[3, 12] = 0.5
    _, col, ptr, _ = ref.bsr_from_dense(A, 8, threshold=0.5)
    assert ptr.tolist() == [0, 0, 0]  # strict >
    _, col, ptr, _ = ref.bsr_from_dense(A, 8, threshold=0.49)
    assert ptr.tolist() == [0, 1, 1] and col.tolist() == [1]


def test_bsr_roundtrip_unaligned():
    rng = np.random.default_rng(2)
    A = rng.standard_normal((20, 14)).astype(np.float32)
    blocks, col, ptr, shape = ref.bsr_from_dense(A, 8)
    assert shape == (20, 14) and len(ptr) == 4
    np.testing.assert_array_equal(ref.bsr_to_dense(blocks, col, ptr, shape, 8), A)


@pytest.mark.parametrize("shape,b,density", [((24, 24), 8, 0.5), ((20, 14), 8, 1.0), ((40, 40), 8, 0.1)])
def test_bsr_spmm_closed_form(shape, b, density):
    rng = np.random.default_rng(3)
    A = rng.standard_normal(shape) * (rng.random(shape) < density)
    B = rng.standard_normal((shape[1], 12))
    blocks, col, ptr, sh = ref.bsr_from_dense(A, b)
    np.testing.assert_allclose(ref.bsr_spmm(blocks, col, ptr, sh, b, B), A @ B, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(
        ref.bsr_spmm(blocks, col, ptr, sh, b, B, absolute=True), np.abs(A) @ np.abs(B), rtol=1e-12
    )


def test_bsr_spmm_empty_pattern_is_zero():
    A = np.zeros((16, 16))
    blocks, col, ptr, sh = ref.bsr_from_dense(A, 8)
    out = ref.bsr_spmm(blocks, col, ptr, sh, 8, np.ones((16, 8)))
    assert out.shape == (16, 8) and not out.any()


@pytest.mark.parametrize("shape,b,density", [((24, 24), 8, 0.5), ((20, 14), 8, 1.0), ((40, 40), 8, 0.3)])
def test_bsr_spmm_backward_vs_dense_autograd(shape, b, density):
    """dA on the stored blocks and dB equal torch float64 autograd through
    the dense product; the padding of unaligned blocks gets zero gradient."""
    rng = np.random.default_rng(7)
    A = rng.standard_normal(shape) * (rng.random(shape) < density)
    B = rng.standard_normal((shape[1], 6))
    G = rng.standard_normal((shape[0], 6))
    blocks, col, ptr, sh = ref.bsr_from_dense(A, b)
    dblk, dB = ref.bsr_spmm_backward(blocks, col, ptr, sh, b, B, G)
    At = torch.tensor(A, requires_grad=True)
    Bt = torch.tensor(B, requires_grad=True)
    (At @ Bt).backward(torch.tensor(G))
    np.testing.assert_allclose(dB, Bt.grad.numpy(), rtol=1e-12, atol=1e-12)
    m, n = shape
    for i in range(len(ptr) - 1):
        for idx in range(ptr[i], ptr[i + 1]):
            j = col[idx]
            r1, c1 = min(b, m - i * b), min(b, n - j * b)
            np.testing.assert_allclose(dblk[idx][:r1, :c1], At.grad.numpy()[i * b : i * b + r1, j * b : j * b + c1],
                                       rtol=1e-12, atol=1e-12)
            assert not dblk[idx][r1:].any() and not dblk[idx][:, c1:].any()
    sd, sB = ref.bsr_spmm_backward(blocks, col, ptr, sh, b, B, G, absolute=True)
    assert (sd >= np.abs(dblk) - 1e-12).all() and (sB >= np.abs(dB) - 1e-12).all()
    Z = ref.bsr_from_dense(np.zeros((16, 16)), 8)
    zd, zB = ref.bsr_spmm_backward(*Z, 8, np.ones((16, 3)), np.ones((16, 3)))
    assert zd.shape == (0, 8, 8) and not zB.any()


def test_csr_from_dense_vs_scipy_and_brute_force():
    rng = np.random.default_rng(12)
    A = rng.standard_normal((37, 53)) * (rng.random((37, 53)) < 0.3)
    for thr in (0.0, 0.5):
        v, c, p = ref.csr_from_dense(A, thr)
        s = sp.csr_matrix(np.where(np.abs(A) > thr, A, 0.0))
        s.sort_indices()
        np.testing.assert_array_equal(p, s.indptr)
        np.testing.assert_array_equal(c, s.indices)
        np.testing.assert_array_equal(v, s.data)
    B = A.copy()
    B[3, 4] = np.nan
    for thr in (-1.0, 0.25):  # negative: every finite entry (zeros too); NaN never passes
        v, c, p = ref.csr_from_dense(B, thr)
        ev, ec, ep = [], [], [0]
        for i in range(B.shape[0]):
            for j in range(B.shape[1]):
                if abs(B[i, j]) > thr:
                    ev.append(B[i, j])
                    ec.append(j)
            ep.append(len(ec))
        np.testing.assert_array_equal(p, ep)
        np.testing.assert_array_equal(c, ec)
        np.testing.assert_array_equal(v, ev)


def test_coo_to_csr_vs_scipy_and_brute_force():
    rng = np.random.default_rng(13)
    m, n, nnz = 40, 30, 300
    flat = rng.choice(m * n, nnz, replace=False)  # distinct coordinates, shuffled
    rows, cols = flat // n, flat % n
    vals = rng.standard_normal(nnz)
    v, c, p = ref.coo_to_csr(vals, rows, cols, (m, n))
    s = sp.coo_matrix((vals, (rows, cols)), shape=(m, n)).tocsr()
    s.sort_indices()
    np.testing.assert_array_equal(p, s.indptr)
    np.testing.assert_array_equal(c, s.indices)
    np.testing.assert_array_equal(v, s.data)
    # duplicates keep their input order
    rows = rng.integers(0, 5, 80)
    cols = rng.integers(0, 3, 80)
    vals = np.arange(80.0)
    v, c, p = ref.coo_to_csr(vals, rows, cols, (5, 3))
    order = [t[2] for t in sorted((int(r), int(cc), k) for k, (r, cc) in enumerate(zip(rows, cols)))]
    np.testing.assert_array_equal(v, vals[order])
    np.testing.assert_array_equal(c, cols[order])
    np.testing.assert_array_equal(p, np.concatenate([[0], np.cumsum(np.bincount(rows, minlength=5))]))


def test_sparse_add_transpose_symmetric_vs_scipy():
    rng = np.random.default_rng(14)
    m, n = 30, 30
    A = rng.standard_normal((m, n)) * (rng.random((m, n)) < 0.2)
    B = rng.standard_normal((m, n)) * (rng.random((m, n)) < 0.2)
    ca, cb = sp.csr_matrix(A), sp.csr_matrix(B)
    ta = (ca.data, ca.indices.astype(np.int64), ca.indptr.astype(np.int64), (m, n))
    tb = (cb.data, cb.indices.astype(np.int64), cb.indptr.astype(np.int64), (m, n))
    v, c, p = ref.sparse_add(ta, tb, 2.0, -0.5)
    # union pattern (scipy drops exact cancellations; here none occur), values summed
    want = sp.csr_matrix(2.0 * A - 0.5 * B)
    want.sort_indices()
    pattern = sp.csr_matrix((np.abs(A) + np.abs(B)) > 0)
    np.testing.assert_array_equal(p, pattern.indptr)
    np.testing.assert_array_equal(c, pattern.indices)
    np.testing.assert_allclose(v, np.asarray((2.0 * A - 0.5 * B)[pattern.nonzero()]).ravel(), rtol=1e-12)
    # duplicates inside one operand are summed too; a cancellation stays as an explicit zero
    vd, cd, pd = ref.coo_sum_to_csr(np.array([1.0, 2.0, -1.0, 4.0]), np.array([0, 0, 0, 1]), np.array([2, 2, 2, 0]),
                                    (2, 3))
    np.testing.assert_array_equal(pd, [0, 1, 2])
    np.testing.assert_array_equal(cd, [2, 0])
    np.testing.assert_array_equal(vd, [2.0, 4.0])
    vz, cz, pz = ref.coo_sum_to_csr(np.array([1.0, -1.0]), np.array([0, 0]), np.array([1, 1]), (1, 2))
    assert len(vz) == 1 and vz[0] == 0.0
    vt, ct, pt = ref.csr_transpose(*ta)
    t = ca.T.tocsr()
    t.sort_indices()
    np.testing.assert_array_equal(pt, t.indptr)
    np.testing.assert_array_equal(ct, t.indices)
    np.testing.assert_array_equal(vt, t.data)
    x = rng.standard_normal(n)
    U = np.triu(A)
    cu = sp.csr_matrix(U)
    y = ref.spmv_symmetric(cu.data, cu.indices.astype(np.int64), cu.indptr.astype(np.int64), (m, n), x, alpha=1.5)
    np.testing.assert_allclose(y, 1.5 * (U + np.triu(U, 1).T) @ x, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------ CSR


def _csr(A):
    s = sp.csr_matrix(A)
    return s.data, s.indices.astype(np.int64), s.indptr.astype(np.int64), A.shape


def test_spmv_known_answer_alpha_beta():
    # reference tests/test_ops.py:25-32: 2*[2,3] + 0.5*[10,20] = [9, 16]
    v, c, p, sh = _csr(np.array([[2.0, 0.0], [0.0, 3.0]]))
    out = ref.csr_spmv(v, c, p, sh, np.ones(2), alpha=2.0, y=np.array([10.0, 20.0]), beta=0.5)
    np.testing.assert_array_equal(out, [9.0, 16.0])
    # y ignored when beta == 0
    out = ref.csr_spmv(v, c, p, sh, np.ones(2), alpha=2.0, y=np.array([10.0, 20.0]), beta=0.0)
    np.testing.assert_array_equal(out, [4.0, 6.0])


def test_spmv_vs_scipy_with_empty_rows():
    rng = np.random.default_rng(4)
    A = rng.standard_normal((300, 200)) * (rng.random((300, 200)) < 0.03)
    A[17] = 0.0
    A[-1] = 0.0
    v, c, p, sh = _csr(A)
    x = rng.standard_normal(200)
    np.testing.assert_allclose(ref.csr_spmv(v, c, p, sh, x), sp.csr_matrix(A) @ x, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("idx", [np.int64, np.int32])
def test_c_oracle_spmv_vs_ref(idx):
    """oracle/csr_spmv.c (the full-size cfg2 oracle) against ref.csr_spmv and
    scipy: int32 and int64 indices, alpha / beta / y, absolute=True, empty
    rows (first, middle, last) and a row longer than 4096 entries."""
    from oracle import build as oracle_c

    rng = np.random.default_rng(11)
    m, n = 700, 9000
    lens = rng.integers(0, 40, m)
    lens[[0, 350, m - 1]] = 0
    lens[123] = 5000
    lens[124] = 4097
    ptr = np.zeros(m + 1, np.int64)
    np.cumsum(lens, out=ptr[1:])
    cols = np.concatenate([np.sort(rng.choice(n, size=k, replace=False)) for k in lens]).astype(np.int64)
    vals = rng.standard_normal(len(cols)).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    y = rng.standard_normal(m).astype(np.float32)
    c, p = cols.astype(idx), ptr.astype(idx)
    dense = sp.csr_matrix((vals.astype(np.float64), cols, ptr), shape=(m, n))
    for alpha, yy, beta in ((1.0, None, 0.0), (-2.5, y, 0.75), (0.5, y, 0.0)):
        exact = ref.csr_spmv(vals, cols, ptr, (m, n), x, alpha=alpha, y=yy, beta=beta)
        got64 = oracle_c.csr_spmv_f64(vals, c, p, m, x, alpha=alpha, y=yy, beta=beta)
        np.testing.assert_allclose(got64, exact, rtol=1e-12, atol=1e-12)
        expect = alpha * (dense @ x.astype(np.float64))
        if yy is not None and beta != 0.0:
            expect = expect + beta * yy.astype(np.float64)
        np.testing.assert_allclose(got64, expect, rtol=1e-12, atol=1e-12)
        scale = ref.csr_spmv(vals, cols, ptr, (m, n), x, alpha=alpha, y=yy, beta=beta, absolute=True)
        np.testing.assert_allclose(oracle_c.csr_spmv_f64(vals, c, p, m, x, alpha=alpha, y=yy, beta=beta,
                                                         absolute=True), scale, rtol=1e-12, atol=1e-12)
        got32 = oracle_c.csr_spmv_f32(vals, c, p, m, x, alpha=alpha, y=yy, beta=beta)
        assert got32.dtype == np.float32
        assert ref.scaled_error(got32, exact, scale) < 1e-5
        for r in (0, 350, m - 1):  # empty rows: beta * y, or exactly zero
            assert got32[r] == (np.float32(beta) * y[r] if yy is not None and beta else 0.0)
    # the long rows reach the C loop's end: a wrong bound drops their tails
    assert abs(got64[123] - exact[123]) <= 1e-9 * scale[123]


def test_spmm_known_answer_and_scipy():
    # reference tests/test_ops.py:61-67: 2*I@ones + 0.5*10 = 7
    v, c, p, sh = _csr(np.eye(2))
    out = ref.csr_spmm(v, c, p, sh, np.ones((2, 3)), alpha=2.0, C=np.full((2, 3), 10.0), beta=0.5)
    np.testing.assert_array_equal(out, np.full((2, 3), 7.0))
    rng = np.random.default_rng(5)
    A = rng.standard_normal((200, 137)) * (rng.random((200, 137)) < 0.05)
    B = rng.standard_normal((137, 64))
    v, c, p, sh = _csr(A)
    np.testing.assert_allclose(ref.csr_spmm(v, c, p, sh, B), A @ B, rtol=1e-12, atol=1e-12)


# -------------------------------------------------------------- screened


def test_screened_threshold_zero_is_matmul():
    rng = np.random.default_rng(6)
    A = rng.standard_normal((64, 64))
    d = np.abs(rng.standard_normal(64)).astype(np.float32) + 0.1
    B = rng.standard_normal((64, 16))
    np.testing.assert_allclose(ref.screened_spmm(A, d, B, 0.0), A @ B, rtol=1e-12)


def test_screened_huge_threshold_is_exact_zero():
    rng = np.random.default_rng(7)
    out = ref.screened_spmm(rng.standard_normal((64, 64)), np.abs(rng.standard_normal(64)).astype(np.float32),
                            rng.standard_normal((64, 16)), 1e30)
    assert not out.any()


def test_screened_mask_is_fp32_compare():
    """Q_i*Q_j equal to fl32(1e-10) is NOT kept for threshold 1e-20: torch
    compares in fp32 (fl32(1e-10) > 1e-10 would hold in float64)."""
    t32 = np.float32(1e-10)
    above = np.nextafter(t32, np.float32(1))
    # Q values whose fp32 product lands exactly on t32 / above: Q_0 = 1, Q_1 = product.
    for target, keep in ((t32, False), (above, True)):
        d = np.array([1.0, np.float32(target) ** 2], dtype=np.float32)
        Q = np.sqrt(np.abs(d)).astype(np.float32)
        if np.float32(Q[0] * Q[1]) != target:
            pytest.skip("sqrt round trip does not land on the target")
        mask = ref.screened_mask(d, 1e-20)
        assert bool(mask[0, 1]) is keep and bool(mask[1, 0]) is keep
    # the threshold conversion: float64 1e-10 vs its float32 rounding differ
    assert float(t32) > 1e-10


def test_screened_mask_matches_torch_semantics():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(8)
    d = (10.0 ** rng.uniform(-14, 0, 512)).astype(np.float32)
    for thr in (1e-20, 1e-12, 0.5e-9, 0.3):
        Q = torch.sqrt(torch.abs(torch.from_numpy(d)))
        tmask = ((Q.unsqueeze(-1) * Q.unsqueeze(0)) > math.sqrt(thr)).numpy()
        np.testing.assert_array_equal(ref.screened_mask(d, thr), tmask)


def test_screened_backward_vs_torch_autograd():
    """ref.screened_spmm_backward against float64 torch autograd of
    (A * mask) @ B with the mask built by torch (a different route to the
    same gradients), on a mask that keeps part of the pairs."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(9)
    n, N = 48, 7
    d = (10.0 ** rng.uniform(-6, 0, n)).astype(np.float32)
    A, B, G = rng.standard_normal((n, n)), rng.standard_normal((n, N)), rng.standard_normal((n, N))
    thr = 1e-4
    At = torch.tensor(A, requires_grad=True)
    Bt = torch.tensor(B, requires_grad=True)
    Q = torch.sqrt(torch.abs(torch.from_numpy(d)))
    mask = ((Q.unsqueeze(-1) * Q.unsqueeze(0)) > math.sqrt(thr)).double()
    assert 0 < mask.sum() < n * n
    ((At * mask) @ Bt).backward(torch.from_numpy(G))
    dA, dB = ref.screened_spmm_backward(A, d, B, thr, G)
    np.testing.assert_allclose(dA, At.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dB, Bt.grad.numpy(), rtol=1e-12, atol=1e-12)


def test_screened_backward_closed_forms():
    """Threshold 0 (every pair kept): dA = dC B^T, dB = A^T dC; a threshold
    above every pair: both zero; the absolute form bounds the signed one."""
    rng = np.random.default_rng(10)
    n, N = 33, 5
    d = np.abs(rng.standard_normal(n)).astype(np.float32) + 0.1
    A, B, G = rng.standard_normal((n, n)), rng.standard_normal((n, N)), rng.standard_normal((n, N))
    dA, dB = ref.screened_spmm_backward(A, d, B, 0.0, G)
    np.testing.assert_allclose(dA, G @ B.T, rtol=1e-12)
    np.testing.assert_allclose(dB, A.T @ G, rtol=1e-12)
    dA, dB = ref.screened_spmm_backward(A, d, B, 1e30, G)
    assert not dA.any() and not dB.any()
    sA, sB = ref.screened_spmm_backward(A, d, B, 0.05, G, absolute=True)
    dA, dB = ref.screened_spmm_backward(A, d, B, 0.05, G)
    assert (np.abs(dA) <= sA + 1e-12).all() and (np.abs(dB) <= sB + 1e-12).all()


# ------------------------------------------------------------- attention


def _local_block_mask(nb, window):
    i = np.arange(nb)
    return np.abs(i[:, None] - i[None, :]) <= window


@pytest.mark.parametrize("S,D,window", [(256, 32, 1), (384, 64, 0), (512, 16, 2)])
def test_attention_vs_dense_masked_softmax(S, D, window):
    rng = np.random.default_rng(9)
    b = 128
    Q, K, V = (rng.standard_normal((S, D)) for _ in range(3))
    bm = _local_block_mask(S // b, window)
    ptr = np.zeros(S // b + 1, np.int64)
    ptr[1:] = np.cumsum(bm.sum(1))
    col = np.nonzero(bm)[1]
    out, rmax, rden = ref.block_sparse_attention(Q, K, V, ptr, col, b, D**-0.5)
    dense_mask = np.kron(bm, np.ones((b, b), bool))
    np.testing.assert_allclose(out, ref.dense_masked_attention(Q, K, V, dense_mask, D**-0.5), rtol=1e-10, atol=1e-12)
    # row_max is the true max of the visible scaled scores
    sc = np.where(dense_mask, (Q @ K.T) * D**-0.5, -np.inf)
    np.testing.assert_allclose(rmax.reshape(-1), sc.max(axis=1), rtol=1e-12)
    np.testing.assert_allclose(rden.reshape(-1), np.exp(sc - sc.max(axis=1, keepdims=True)).sum(axis=1), rtol=1e-12)


def test_attention_full_mask_is_dense_and_empty_rows_zero():
    rng = np.random.default_rng(10)
    S, D, b = 256, 32, 128
    Q, K, V = (rng.standard_normal((S, D)) for _ in range(3))
    ptr = np.array([0, 2, 4])
    col = np.array([0, 1, 0, 1])
    sc = (Q @ K.T) / math.sqrt(D)
    p = np.exp(sc - sc.max(1, keepdims=True))
    dense = (p / p.sum(1, keepdims=True)) @ V
    out, _, _ = ref.block_sparse_attention(Q, K, V, ptr, col, b, D**-0.5)
    np.testing.assert_allclose(out, dense, rtol=1e-10, atol=1e-12)
    ptr = np.array([0, 0, 1])
    col = np.array([1])
    out, rmax, rden = ref.block_sparse_attention(Q, K, V, ptr, col, b, D**-0.5)
    assert not out[:128].any() and not rmax[0].any() and np.all(rden[0] == 1e-12)


def _torch_masked_attention(Q, K, V, visible, scale):
    """Dense masked softmax attention; rows with no visible key give zero."""
    sc = torch.where(visible, (Q @ K.T) * scale, torch.tensor(-math.inf, dtype=Q.dtype))
    has = visible.any(dim=1, keepdim=True)
    p = torch.softmax(torch.where(has, sc, torch.zeros_like(sc)), dim=1)
    return torch.where(has, p @ V, torch.zeros_like(Q))


@pytest.mark.parametrize(
    "S,D,b,mask",
    [
        (256, 32, 128, [[1, 1], [1, 1]]),                      # full mask
        (48, 8, 8, [[1, 1, 0, 0, 0, 1], [1, 1, 1, 0, 0, 0], [0, 1, 1, 1, 0, 0],
                    [0, 0, 1, 1, 1, 0], [1, 0, 0, 1, 1, 1], [0, 0, 0, 0, 1, 1]]),
        # ragged S (Mt = 5, block column 5 holds keys 40..43 only, block row 5
        # has no queries), an empty block row (1)
        (44, 6, 8, [[1, 0, 0, 0, 0, 1], [0, 0, 0, 0, 0, 0], [0, 1, 1, 0, 0, 0],
                    [1, 0, 0, 1, 0, 1], [0, 0, 1, 1, 1, 1], [1, 1, 1, 1, 1, 1]]),
    ],
)
def test_attention_backward_vs_dense_autograd(S, D, b, mask):
    """dQ, dK, dV equal torch float64 autograd through dense masked softmax
    attention on the same visibility (query q < (S // b) b sees key k < S
    when block (q // b, k // b) is stored)."""
    rng = np.random.default_rng(11)
    Q, K, V, dO = (rng.standard_normal((S, D)) for _ in range(4))
    bm = np.array(mask, bool)
    ptr = np.zeros(bm.shape[0] + 1, np.int64)
    ptr[1:] = np.cumsum(bm.sum(1))
    col = np.nonzero(bm)[1].astype(np.int64)
    scale = D**-0.5
    O, _, _ = ref.block_sparse_attention(Q, K, V, ptr, col, b, scale)
    dQ, dK, dV = ref.block_sparse_attention_backward(Q, K, V, O, dO, ptr, col, b, scale)
    Mt = S // b
    qi, ki = np.arange(S), np.arange(S)
    visible = (qi[:, None] < Mt * b) & bm[np.minimum(qi // b, bm.shape[0] - 1)][:, ki // b]
    Qt, Kt, Vt = (torch.tensor(t, requires_grad=True) for t in (Q, K, V))
    out = _torch_masked_attention(Qt, Kt, Vt, torch.tensor(visible), scale)
    np.testing.assert_allclose(out.detach().numpy(), O, rtol=1e-10, atol=1e-12)
    out.backward(torch.tensor(dO))
    for got, t in ((dQ, Qt), (dK, Kt), (dV, Vt)):
        np.testing.assert_allclose(got, t.grad.numpy(), rtol=1e-9, atol=1e-11)
    aQ, aK, aV = ref.block_sparse_attention_backward(Q, K, V, O, dO, ptr, col, b, scale, absolute=True)
    assert (aQ >= np.abs(dQ) - 1e-12).all() and (aK >= np.abs(dK) - 1e-12).all() and (aV >= np.abs(dV) - 1e-12).all()
    # restricting to some block rows / columns keeps exactly those contributions
    rQ, _, _ = ref.block_sparse_attention_backward(Q, K, V, O, dO, ptr, col, b, scale, rows=[0], cols=[])
    np.testing.assert_array_equal(rQ[:b], dQ[:b])
    assert not rQ[b:].any()
    _, cK, cV = ref.block_sparse_attention_backward(Q, K, V, O, dO, ptr, col, b, scale, rows=[], cols=[1])
    np.testing.assert_allclose(cK[b : 2 * b], dK[b : 2 * b], rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(cV[b : 2 * b], dV[b : 2 * b], rtol=1e-12, atol=1e-14)
    assert not cK[:b].any() and not cV[2 * b :].any()


def _cheb_U(K, t):
    """Chebyshev polynomial of the second kind U_K(t), closed forms:
    sin((K+1) th) / sin th for t = cos th, sinh((K+1) th) / sinh th for
    t = cosh th, U_K(-t) = (-1)^K U_K(t)."""
    t = np.asarray(t, dtype=np.float64)
    a = np.abs(t)
    out = np.empty_like(a)
    inside = a < 1
    th = np.arccos(a[inside])
    out[inside] = np.sin((K + 1) * th) / np.sin(th)
    th = np.arccosh(np.maximum(a[~inside], 1.0))
    out[~inside] = np.where(th > 0, np.sinh((K + 1) * th) / np.where(th > 0, np.sinh(th), 1.0), K + 1.0)
    return out * np.where(t < 0, (-1.0) ** K, 1.0)


@pytest.mark.parametrize("lo,hi,K", [(1.0, 10.0, 12), (0.5, 2.0, 30), (3.0, 3.5, 5)])
def test_chebyshev_coeffs_closed_form(lo, hi, K):
    """The reference's recurrence (alpha_0 = 1/d, then the generic step from
    k = 1) has rho_k = c alpha_k / 2 = U_k(s) / U_{k+1}(s), s = d / c, so
    alpha_k = (2/c) U_k(s)/U_{k+1}(s), beta_k = U_{k-1}(s)/U_{k+1}(s), and the
    scalar error recurrence e_{k+1} = (1 - alpha_k lam) e_k + beta_k (e_k -
    e_{k-1}), e_0 = 1, ends at U_K((d - lam)/c) / U_K(s): a Chebyshev
    polynomial of the second kind."""
    alpha, beta = ref.chebyshev_coeffs(lo, hi, K, dtype=np.float64)
    c, d = (hi - lo) / 2, (hi + lo) / 2
    s_ = d / c
    k = np.arange(K)
    np.testing.assert_allclose(alpha, (2 / c) * np.array([_cheb_U(int(i), s_)[()] / _cheb_U(int(i) + 1, s_)[()]
                                                         for i in k]), rtol=1e-12)
    np.testing.assert_allclose(beta[1:], [_cheb_U(int(i) - 1, s_)[()] / _cheb_U(int(i) + 1, s_)[()] for i in k[1:]],
                               rtol=1e-12)
    assert beta[0] == 0
    lam = np.linspace(lo, hi, 17)
    e_prev = e = np.ones_like(lam)
    for i in range(K):
        e_new = (1 - alpha[i] * lam) * e + (beta[i] * (e - e_prev) if i else 0.0)
        e_prev, e = e, e_new
    np.testing.assert_allclose(e, _cheb_U(K, (d - lam) / c) / _cheb_U(K, s_), rtol=1e-9, atol=1e-13)
    a32, b32 = ref.chebyshev_coeffs(lo, hi, K)
    assert a32.dtype == np.float32 and np.array_equal(a32, alpha.astype(np.float32))


def test_solvers_on_diagonal_matrices_closed_form():
    lam = np.array([1.0, 2.5, 4.0, 7.0])
    b = np.array([1.0, -2.0, 0.5, 3.0])
    mv = lambda x: lam * x
    omega, K = 0.2, 9
    np.testing.assert_allclose(ref.richardson(mv, b, omega, K), (1 - (1 - omega * lam) ** K) * b / lam, rtol=1e-12)
    lo, hi, K = 1.0, 7.0, 6
    alpha, beta = ref.chebyshev_coeffs(lo, hi, K, dtype=np.float64)
    c, d = (hi - lo) / 2, (hi + lo) / 2
    p = _cheb_U(K, (d - lam) / c) / _cheb_U(K, d / c)  # residual polynomial from x0 = 0
    np.testing.assert_allclose(ref.chebyshev(mv, b, alpha, beta, K), (1 - p) * b / lam, rtol=1e-10)


def test_package_solvers_match_oracle_on_cpu():
    """The torch loops (CPU, pytorch backend) follow the reference's
    statements; the coefficients agree bit for bit."""
    import trnsparse_amd as ts
    from trnsparse_amd import workloads as W

    A, lo, hi = W.spd_bsr(nb=6, b=8, band=1, n_pairs=2, dtype=torch.float64)
    a_t, b_t = ts.chebyshev_coeffs(lo, hi, 20)
    a_o, b_o = ref.chebyshev_coeffs(lo, hi, 20)
    assert np.array_equal(a_t.numpy(), a_o) and np.array_equal(b_t.numpy(), b_o)
    mv = ref.bsr_matvec(A.blocks.numpy(), A.block_col_indices.numpy(), A.block_row_ptrs.numpy(), A.shape, 8)
    rhs = torch.randn(48, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    prev = ts.get_backend()
    ts.set_backend("pytorch")
    try:
        x, K, rel = ts.richardson_bsr(A, rhs, 2.0 / (lo + hi), K=40)
        np.testing.assert_allclose(x.numpy(), ref.richardson(mv, rhs.numpy(), 2.0 / (lo + hi), 40), rtol=1e-10)
        x, K, rel = ts.chebyshev_bsr(A, rhs, lo, hi, K=20)
        np.testing.assert_allclose(x.numpy(), ref.chebyshev(mv, rhs.numpy(), a_o, b_o, 20), rtol=1e-10)
        assert K == 20 and rel < 1e-6
    finally:
        ts.set_backend(prev)


def test_error_metrics():
    ref_ = np.array([1.0, -2.0, 0.0])
    got = np.array([1.0, -2.0 + 1e-3, 1e-6])
    scale = np.array([1.0, 10.0, 1.0])
    assert ref.scaled_error(got, ref_, scale) == pytest.approx(1e-4)
    assert ref.rel_max_error(got, ref_) == pytest.approx(5e-4)
