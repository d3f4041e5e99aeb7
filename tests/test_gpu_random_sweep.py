"""Seeded random sweep of shapes through the public API on the hip backend,
against the float64 oracle (oracle/ref.py restates trnsparse/ops.py).

Each case draws its sizes so that tile edges, block edges and odd widths
come up (dimensions that are not multiples of the kernels' tiles, N not a
multiple of the vector width, head_dims the kernels pad, sequences that end
inside a block), the block size from the small-block and the 128-block
kernels' set and others that run the generic kernels. Bars as in the other
parity tests: fp32 1e-4 and bf16 2e-2 of the per-element error scale
(|A|.|B|, softmax weights applied to |V|).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import trnsparse_amd as ts
from oracle import ref
from trnsparse_amd import workloads as W

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float64: 1e-12}


def _err(got, exact, scale):
    return ref.scaled_error(got, exact, np.maximum(scale, 1e-30))


@pytest.mark.parametrize("seed", range(24))
def test_sweep_bsr_spmm(hip_backend, seed):
    rng = np.random.default_rng(1000 + seed)
    b = int(rng.choice([8, 16, 24, 32, 64, 128]))
    m, k = int(rng.integers(1, 7 * b)), int(rng.integers(1, 7 * b))
    N = int(rng.choice([1, 3, 8, 17, 64, 100, 129, 256]))
    dt = [torch.float32, torch.bfloat16, torch.float64][seed % 3]
    mb, kb = -(-m // b), -(-k // b)
    mask = torch.from_numpy(rng.random((mb, kb)) < rng.uniform(0.1, 0.9))
    g = torch.Generator().manual_seed(seed)
    dense = torch.randn(m, k, generator=g, dtype=torch.float64)
    dense *= mask.repeat_interleave(b, 0).repeat_interleave(b, 1)[:m, :k]
    A = ts.BSRMatrix.from_dense(dense.to(dt).cuda(), block_size=b)
    B = torch.randn(k, N, generator=g, dtype=torch.float64).to(dt)
    got = ts.bsr_spmm(A, B.cuda()).cpu()
    assert got.shape == (m, N) and got.dtype == dt
    blocks = A.blocks.cpu().double().numpy()
    col, ptr = A.block_col_indices.cpu().numpy(), A.block_row_ptrs.cpu().numpy()
    Bn = B.double().numpy()
    exact = ref.bsr_spmm(blocks, col, ptr, (m, k), b, Bn)
    scale = ref.bsr_spmm(blocks, col, ptr, (m, k), b, Bn, absolute=True)
    assert _err(got.double().numpy(), exact, scale) <= TOL[dt], (b, m, k, N, dt)


@pytest.mark.parametrize("seed", range(16))
def test_sweep_csr(hip_backend, seed):
    rng = np.random.default_rng(2000 + seed)
    m, n = int(rng.integers(1, 40000)), int(rng.integers(1, 40000))
    lens = np.minimum(rng.poisson(rng.uniform(0.5, 30), m), n)
    if seed % 4 == 0:
        lens[rng.integers(0, m)] = min(n, 9000)           # one long row
    v, c, p = W.random_csr(lens, n, rng)
    dt = torch.float64 if seed % 5 == 0 else torch.float32
    v = v.astype(np.float64 if dt == torch.float64 else np.float32)
    ci = c.astype(np.int32) if seed % 2 else c
    A = W.csr_matrix_from_arrays(v, ci, p.astype(ci.dtype), (m, n), device="cuda")
    x = rng.standard_normal(n).astype(v.dtype)
    y = rng.standard_normal(m).astype(v.dtype)
    for _ in range(2):                                    # the second call may use the plan
        got = ts.spmv(A, torch.from_numpy(x).cuda(), alpha=-0.5, y=torch.from_numpy(y).cuda(), beta=1.5)
        exact = ref.csr_spmv(v, c, p, (m, n), x, -0.5, y, 1.5)
        scale = ref.csr_spmv(v, c, p, (m, n), x, -0.5, y, 1.5, absolute=True)
        assert _err(got.cpu().numpy(), exact, scale) <= TOL[dt], (m, n, dt)
    N = int(rng.choice([2, 5, 8, 33]))
    B = rng.standard_normal((n, N)).astype(v.dtype)
    got = ts.spmm(A, torch.from_numpy(B).cuda())
    exact = ref.csr_spmm(v, c, p, (m, n), B)
    scale = ref.csr_spmm(v, c, p, (m, n), B, absolute=True)
    assert _err(got.cpu().numpy(), exact, scale) <= TOL[dt], (m, n, N, dt)


@pytest.mark.parametrize("seed", range(16))
def test_sweep_attention(hip_backend, seed):
    rng = np.random.default_rng(3000 + seed)
    S = int(rng.integers(1, 9)) * 128 + int(rng.choice([0, 0, 37, 100]))
    d = int(rng.choice([16, 64, 100, 128, 200, 256, 320, 512]))
    dt = torch.bfloat16 if seed % 2 else torch.float32
    nb = -(-S // 128)
    mask = torch.from_numpy(rng.random((nb, nb)) < 0.5)
    if nb > 1:
        mask[rng.integers(0, nb), :] = False              # an empty block row
    mask_bsr = W.bsr_from_block_mask(mask, 128)
    H = int(rng.integers(1, 4))
    g = torch.Generator().manual_seed(seed)
    Q, K, V = (torch.randn(H, S, d, generator=g).to(dt) for _ in range(3))
    scale = float(rng.uniform(0.02, 0.2))
    got = ts.block_sparse_attention_tiled(Q.cuda(), K.cuda(), V.cuda(), mask_bsr, scale=scale).cpu()
    assert got.shape == Q.shape and got.dtype == dt
    ptr, col = mask_bsr.block_row_ptrs.numpy(), mask_bsr.block_col_indices.numpy()
    for h in range(H):
        q, k, v = (t[h].float().numpy() for t in (Q, K, V))
        out, _, _ = ref.block_sparse_attention(q, k, v, ptr, col, 128, scale)
        sc, _, _ = ref.block_sparse_attention(q, k, np.abs(v), ptr, col, 128, scale)
        assert _err(got[h].float().numpy(), out, sc) <= TOL[dt], (S, d, dt, H)


@pytest.mark.parametrize("seed", range(8))
def test_sweep_screened(hip_backend, seed):
    rng = np.random.default_rng(4000 + seed)
    n, N = int(rng.integers(1, 700)), int(rng.integers(1, 300))
    dt = torch.float64 if seed % 4 == 3 else torch.float32
    A = rng.standard_normal((n, n))
    diag = 10.0 ** rng.uniform(-12, 0, n)
    B = rng.standard_normal((n, N))
    thr = float(10.0 ** rng.uniform(-10, -4))
    got = ts.screened_spmm(torch.from_numpy(A).to(dt).cuda(), torch.from_numpy(diag).to(dt).cuda(),
                           torch.from_numpy(B).to(dt).cuda(), thr).cpu()
    An, Bn = (torch.from_numpy(t).to(dt).double().numpy() for t in (A, B))
    dn = torch.from_numpy(diag).to(dt).numpy()            # the mask is formed in diag's precision
    exact = ref.screened_spmm(An, dn, Bn, thr)
    scale = ref.screened_spmm(An, dn, Bn, thr, absolute=True)
    assert _err(got.double().numpy(), exact, scale) <= TOL[dt], (n, N, dt)


@pytest.mark.parametrize("seed", range(12))
def test_sweep_bsr_spmm_backward(hip_backend, seed):
    rng = np.random.default_rng(5000 + seed)
    b = int(rng.choice([8, 16, 32, 64, 128, 24]))
    m, k = int(rng.integers(1, 6 * b)), int(rng.integers(1, 6 * b))
    N = int(rng.choice([1, 8, 33, 128, 200]))
    dt = [torch.float32, torch.bfloat16][seed % 2]
    mb, kb = -(-m // b), -(-k // b)
    mask = torch.from_numpy(rng.random((mb, kb)) < rng.uniform(0.2, 0.9))
    g = torch.Generator().manual_seed(seed)
    dense = torch.randn(m, k, generator=g) * mask.repeat_interleave(b, 0).repeat_interleave(b, 1)[:m, :k]
    A0 = ts.BSRMatrix.from_dense(dense.to(dt).cuda(), block_size=b)
    blocks = A0.blocks.clone().requires_grad_(True)
    A = ts.BSRMatrix(blocks=blocks, block_col_indices=A0.block_col_indices, block_row_ptrs=A0.block_row_ptrs,
                     shape=A0.shape, block_size=b)
    B = torch.randn(k, N, generator=g).to(dt).cuda().requires_grad_(True)
    G = torch.randn(m, N, generator=g).to(dt)
    ts.bsr_spmm(A, B).backward(G.cuda())
    args = (A0.blocks.cpu().double().numpy(), A0.block_col_indices.cpu().numpy(), A0.block_row_ptrs.cpu().numpy(),
            (m, k), b, B.detach().cpu().double().numpy(), G.double().numpy())
    exact = ref.bsr_spmm_backward(*args)
    scale = ref.bsr_spmm_backward(*args, absolute=True)
    for got, e, sc in zip((blocks.grad, B.grad), exact, scale):
        assert _err(got.cpu().double().numpy(), e, sc) <= TOL[dt], (b, m, k, N, dt)


@pytest.mark.parametrize("seed", range(12))
def test_sweep_attention_backward(hip_backend, seed):
    rng = np.random.default_rng(6000 + seed)
    S = int(rng.integers(1, 6)) * 128 + int(rng.choice([0, 0, 60]))
    d = int(rng.choice([32, 64, 96, 128, 256, 320, 512]))
    dt = torch.bfloat16 if seed % 2 else torch.float32
    nb = -(-S // 128)
    mask = torch.from_numpy(rng.random((nb, nb)) < 0.6)
    mask_bsr = W.bsr_from_block_mask(mask, 128)
    g = torch.Generator().manual_seed(seed)
    Q, K, V, dO = (torch.randn(S, d, generator=g).to(dt) for _ in range(4))
    scale = float(rng.uniform(0.03, 0.15))
    q, kk, v = (t.cuda().requires_grad_(True) for t in (Q, K, V))
    O = ts.block_sparse_attention_tiled(q, kk, v, mask_bsr, scale=scale)
    O.backward(dO.cuda())
    ptr, col = mask_bsr.block_row_ptrs.numpy(), mask_bsr.block_col_indices.numpy()
    args = tuple(t.float().double().numpy() for t in (Q, K, V, O.detach().cpu(), dO)) + (ptr, col, 128, scale)
    exact = ref.block_sparse_attention_backward(*args)
    bound = ref.block_sparse_attention_backward(*args, absolute=True)
    for got, e, a in zip((q.grad, kk.grad, v.grad), exact, bound):
        assert _err(got.cpu().double().numpy(), e, a) <= TOL[dt], (S, d, dt)


@pytest.mark.parametrize("seed", range(12))
def test_sweep_formats_and_csr_ops(hip_backend, seed):
    """Structure bit-exact (indices, pointers, value order) and values exact
    for the device format builders and CSR structure ops on random shapes."""
    rng = np.random.default_rng(7000 + seed)
    m, n = int(rng.integers(1, 3000)), int(rng.integers(1, 3000))
    b = int(rng.choice([8, 16, 32, 64, 128, 40]))
    thr = float(rng.choice([0.0, 0.5]))
    dense = rng.standard_normal((m, n)).astype(np.float32)
    dense[rng.random((m, n)) < rng.uniform(0.5, 0.99)] = 0.0
    if seed % 3 == 0:
        dense[: m // 3] = 0.0                                  # empty rows / block rows
    Dg = torch.from_numpy(dense).cuda()
    # BSR from_dense / to_dense
    Ab = ts.BSRMatrix.from_dense(Dg, block_size=b, threshold=thr)
    eb, ec, ep, _ = ref.bsr_from_dense(dense, b, thr)
    assert np.array_equal(Ab.block_row_ptrs.cpu().numpy(), ep) and np.array_equal(Ab.block_col_indices.cpu().numpy(), ec)
    assert np.array_equal(Ab.blocks.cpu().numpy(), eb)
    assert torch.equal(Ab.to_dense().cpu(), torch.from_numpy(ref.bsr_to_dense(eb, ec, ep, (m, n), b)))
    # CSR from_dense
    Ac = ts.from_dense(Dg, threshold=thr)
    ev, ecol, eptr = ref.csr_from_dense(dense, thr)
    assert np.array_equal(Ac.row_ptrs.cpu().numpy(), eptr) and np.array_equal(Ac.col_indices.cpu().numpy(), ecol)
    assert np.array_equal(Ac.values.cpu().numpy(), ev)
    # COO with duplicates, entries shuffled -> CSR (stable order of equal keys)
    nnz = len(ev)
    rows = np.repeat(np.arange(m), np.diff(eptr))
    perm = rng.permutation(nnz)
    dup = rng.integers(0, max(nnz, 1), size=nnz // 4) if nnz else np.zeros(0, np.int64)
    r = np.concatenate([rows[perm], rows[dup]]).astype(np.int64)
    c = np.concatenate([ecol[perm], ecol[dup]]).astype(np.int64)
    v = np.concatenate([ev[perm], ev[dup] * 0.5]).astype(np.float32)
    coo = ts.COOMatrix(values=torch.from_numpy(v).cuda(), row_indices=torch.from_numpy(r).cuda(),
                       col_indices=torch.from_numpy(c).cuda(), shape=(m, n))
    C = coo.to_csr()
    wv, wc, wp = ref.coo_to_csr(v, r, c, (m, n))
    assert np.array_equal(C.row_ptrs.cpu().numpy(), wp) and np.array_equal(C.col_indices.cpu().numpy(), wc)
    assert np.array_equal(C.values.cpu().numpy(), wv)
    # transpose and add
    T = ts.sparse_transpose(Ac)
    tv, tc, tp = ref.csr_transpose(ev, ecol, eptr, (m, n))
    assert np.array_equal(T.row_ptrs.cpu().numpy(), tp) and np.array_equal(T.col_indices.cpu().numpy(), tc)
    assert np.array_equal(T.values.cpu().numpy(), tv)
    if m == n:
        S = ts.sparse_add(Ac, T, alpha=0.5, beta=2.0)
        sv, sc, sp = ref.sparse_add((ev, ecol, eptr, (m, n)), (tv, tc, tp, (m, n)), 0.5, 2.0)
        assert np.array_equal(S.row_ptrs.cpu().numpy(), sp) and np.array_equal(S.col_indices.cpu().numpy(), sc)
        np.testing.assert_allclose(S.values.cpu().numpy(), sv, rtol=1e-6, atol=0)
