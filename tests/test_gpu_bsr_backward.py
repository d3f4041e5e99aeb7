"""GPU parity of the bsr_spmm backward (tsp_bsr_sddmm for dA on the stored
pattern, tsp_bsr_spmm_t for dB = A^T dC) against the CPU oracle
(oracle.ref.bsr_spmm_backward, pinned to dense autograd on the CPU).

Tolerances follow the forward: fp32 max error <= 1e-4 and bf16 <= 2e-2
relative to the dot-product scale of each gradient element (|G|.|B| for dA,
|A|^T.|G| for dB); fp64 <= 1e-10.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import trnsparse_amd as ts
from oracle import ref
from trnsparse_amd import workloads as W

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float64: 1e-10}


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy() if t.dtype == torch.bfloat16 else t.detach().cpu().numpy()


def _grads(A: ts.BSRMatrix, B: torch.Tensor, G: torch.Tensor):
    blocks = A.blocks.detach().clone().cuda().requires_grad_(True)
    Bd = B.detach().clone().cuda().requires_grad_(True)
    Ad = ts.BSRMatrix(blocks, A.block_col_indices, A.block_row_ptrs, A.shape, A.block_size)
    C = ts.bsr_spmm(Ad, Bd)
    C.backward(G.cuda().to(C.dtype))
    return blocks.grad, Bd.grad


def _check(A: ts.BSRMatrix, B: torch.Tensor, G: torch.Tensor, tol: float):
    db, dB = _grads(A, B, G)
    assert db.dtype == A.dtype and dB.dtype == B.dtype and dB.shape == B.shape
    args = (_np(A.blocks), A.block_col_indices.numpy(), A.block_row_ptrs.numpy(), A.shape, A.block_size, _np(B), _np(G))
    exact_b, exact_B = ref.bsr_spmm_backward(*args)
    scale_b, scale_B = ref.bsr_spmm_backward(*args, absolute=True)
    assert ref.scaled_error(_np(db), exact_b, scale_b) <= tol
    assert ref.scaled_error(_np(dB), exact_B, scale_B) <= tol


@pytest.mark.parametrize(
    "shape,b,N,density,dtype",
    [
        ((256, 384), 128, 64, 0.5, torch.float32),     # MFMA kernels
        ((512, 512), 128, 256, 0.3, torch.float32),
        ((384, 256), 128, 200, 0.6, torch.float32),    # N % 64 != 0: zero-filled k tail
        ((300, 260), 128, 12, 1.0, torch.float32),     # unaligned m, n (padded blocks)
        ((300, 260), 128, 10, 1.0, torch.float32),     # N % 4 != 0: generic kernels
        ((40, 40), 8, 12, 0.4, torch.float64),         # fp64 at block size 8: generic kernels
        ((256, 384), 128, 64, 0.5, torch.float64),     # fp64 MFMA kernels
        ((384, 256), 128, 200, 0.6, torch.float64),    # N % 32 != 0: zero-filled k tail
        ((300, 260), 128, 12, 1.0, torch.float64),     # unaligned m, n
        ((300, 260), 128, 11, 1.0, torch.float64),     # odd N: generic kernels
        ((256, 256), 128, 64, 0.5, torch.bfloat16),    # bf16 MFMA kernels
        ((512, 384), 128, 256, 0.4, torch.bfloat16),
        ((384, 256), 128, 200, 0.6, torch.bfloat16),   # N % 64 != 0: zero-filled k tail
        ((300, 260), 128, 24, 1.0, torch.bfloat16),    # unaligned m, n
        ((300, 260), 128, 12, 1.0, torch.bfloat16),    # N % 8 != 0: generic kernels
        # small blocks (bsr_sddmm_small, bsr_spmm_small over the column view)
        ((64, 64), 8, 16, 0.5, torch.float32),
        ((200, 150), 8, 37, 0.5, torch.float32),       # ragged m, n; N % 4 != 0 (element-wise reads)
        ((256, 512), 8, 512, 0.3, torch.float32),      # 16-byte reads, four 128-column tiles
        ((520, 24), 8, 130, 1.0, torch.float32),       # block columns of 65 stored blocks
        ((64, 72), 8, 2100, 0.5, torch.float32),       # N past the LDS-staged dA kernel: 4x4x1 k-split form
        ((64, 72), 8, 2100, 0.5, torch.bfloat16),
        ((256, 256), 16, 130, 0.4, torch.float32),
        ((200, 150), 16, 64, 0.5, torch.float32),      # ragged m, n
        ((320, 200), 32, 96, 0.5, torch.float32),
        ((256, 512), 64, 200, 0.3, torch.float32),
        ((330, 260), 64, 12, 0.6, torch.float32),      # ragged, narrow N
        ((256, 512), 8, 512, 0.3, torch.bfloat16),
        ((200, 150), 16, 37, 0.5, torch.bfloat16),
        ((256, 256), 32, 128, 0.5, torch.bfloat16),
        ((300, 260), 64, 24, 0.8, torch.bfloat16),
    ],
)
def test_backward_matches_oracle(hip_backend, shape, b, N, density, dtype):
    g = torch.Generator().manual_seed(31)
    A = torch.randn(*shape, generator=g, dtype=torch.float64) * (torch.rand(*shape, generator=g) < density)
    bsr = ts.BSRMatrix.from_dense(A.to(dtype), block_size=b)
    B = torch.randn(shape[1], N, generator=g, dtype=torch.float64).to(dtype)
    G = torch.randn(shape[0], N, generator=g, dtype=torch.float64).to(dtype)
    _check(bsr, B, G, TOL[dtype])


def test_backward_empty_rows_and_columns(hip_backend):
    """Block rows and block columns without stored blocks: zero gradient rows
    of dB, and dA only on the stored blocks."""
    mask = torch.tensor([[True, False, False, True], [False, False, False, False], [True, False, True, False]])
    bsr = W.bsr_from_block_mask(mask, 128)
    g = torch.Generator().manual_seed(2)
    bsr = ts.BSRMatrix(torch.randn(bsr.n_blocks, 128, 128, generator=g), bsr.block_col_indices, bsr.block_row_ptrs,
                       bsr.shape, 128)
    B = torch.randn(bsr.shape[1], 128, generator=g)
    G = torch.randn(bsr.shape[0], 128, generator=g)
    _check(bsr, B, G, TOL[torch.float32])
    _, dB = _grads(bsr, B, G)
    assert torch.count_nonzero(dB[128:256]).item() == 0  # block column 1 holds no blocks


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float64])
def test_backward_long_block_column(hip_backend, dtype):
    """A block column with 65 stored blocks (the dB kernels read a column's
    block ids 64 at a time)."""
    g = torch.Generator().manual_seed(7)
    A = torch.randn(65 * 128, 128, generator=g, dtype=torch.float64)
    bsr = ts.BSRMatrix.from_dense(A.to(dtype), block_size=128)
    assert bsr.n_blocks == 65
    B = torch.randn(128, 64, generator=g, dtype=torch.float64).to(dtype)
    G = torch.randn(65 * 128, 64, generator=g, dtype=torch.float64).to(dtype)
    _check(bsr, B, G, TOL[dtype])


def test_backward_deterministic(hip_backend):
    A, B = W.cfg3_bsr(nb=16, ncols=128, density=0.3)
    G = torch.randn(A.shape[0], 128, generator=torch.Generator().manual_seed(5))
    d1 = _grads(A, B, G)
    d2 = _grads(A, B, G)
    assert torch.equal(d1[0], d2[0]) and torch.equal(d1[1], d2[1])


def test_cfg3a_backward_full_size(hip_backend):
    """cfg3a (1638 blocks, N = 512): dA on a sample of blocks against the
    closed form in float64, and dB through the size-independent identity
    1^T dB 1 = (A 1) . (G 1) plus a sample of dB rows."""
    A, B = W.cfg3_bsr(dtype=torch.float32)
    G = torch.randn(A.shape[0], B.shape[1], generator=torch.Generator().manual_seed(9))
    db, dB = _grads(A, B, G)
    Gn, Bn = G.double().numpy(), B.double().numpy()
    ptr, col = A.block_row_ptrs.numpy(), A.block_col_indices.numpy()
    brow = np.repeat(np.arange(len(ptr) - 1), np.diff(ptr))
    for k in (0, 1, 700, 1637):
        i, j = brow[k], col[k]
        exact = Gn[i * 128 : (i + 1) * 128] @ Bn[j * 128 : (j + 1) * 128].T
        scale = np.abs(Gn[i * 128 : (i + 1) * 128]) @ np.abs(Bn[j * 128 : (j + 1) * 128]).T
        assert ref.scaled_error(db[k].cpu().numpy(), exact, scale) <= TOL[torch.float32]
    blocks = A.blocks.double().numpy()
    rowsum_A = np.zeros(A.shape[0])
    for k in range(len(col)):
        rowsum_A[brow[k] * 128 : (brow[k] + 1) * 128] += blocks[k].sum(axis=1)
    expect = rowsum_A @ Gn.sum(axis=1)
    got = dB.double().sum().item()
    bound = (np.abs(blocks).sum() * np.abs(Gn).max() * B.shape[1]) * 1e-6
    assert abs(got - expect) <= bound
    # a sample of dB rows: rows of block column j are sum_k A_k^T G_i
    for j in (0, 64, 127):
        ks = np.nonzero(col == j)[0]
        exact = sum(blocks[k].T @ Gn[brow[k] * 128 : (brow[k] + 1) * 128] for k in ks)
        scale = sum(np.abs(blocks[k]).T @ np.abs(Gn[brow[k] * 128 : (brow[k] + 1) * 128]) for k in ks)
        assert ref.scaled_error(dB[j * 128 : (j + 1) * 128].cpu().numpy(), exact, scale) <= TOL[torch.float32]


def test_cfg3b_backward_full_size(hip_backend):
    """cfg3b (bf16, 1638 blocks, N = 512, the bf16 MFMA kernels): dA on a
    sample of blocks and dB on a sample of block columns against float64."""
    A, B = W.cfg3_bsr(dtype=torch.bfloat16)
    G = torch.randn(A.shape[0], B.shape[1], generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    db, dB = _grads(A, B, G)
    assert db.dtype == torch.bfloat16 and dB.dtype == torch.bfloat16
    Gn, Bn = G.double().numpy(), B.double().numpy()
    ptr, col = A.block_row_ptrs.numpy(), A.block_col_indices.numpy()
    brow = np.repeat(np.arange(len(ptr) - 1), np.diff(ptr))
    for k in (0, 1, 700, 1637):
        i, j = brow[k], col[k]
        exact = Gn[i * 128 : (i + 1) * 128] @ Bn[j * 128 : (j + 1) * 128].T
        scale = np.abs(Gn[i * 128 : (i + 1) * 128]) @ np.abs(Bn[j * 128 : (j + 1) * 128]).T
        assert ref.scaled_error(db[k].double().cpu().numpy(), exact, scale) <= TOL[torch.bfloat16]
    blocks = A.blocks.double().numpy()
    for j in (0, 64, 127):
        ks = np.nonzero(col == j)[0]
        exact = sum(blocks[k].T @ Gn[brow[k] * 128 : (brow[k] + 1) * 128] for k in ks)
        scale = sum(np.abs(blocks[k]).T @ np.abs(Gn[brow[k] * 128 : (brow[k] + 1) * 128]) for k in ks)
        assert ref.scaled_error(dB[j * 128 : (j + 1) * 128].double().cpu().numpy(), exact, scale) <= TOL[torch.bfloat16]

@pytest.mark.gpu
@pytest.mark.parametrize("mb,nbc,p", [(1, 1, 1.0), (7, 300, 0.2), (40, 3, 0.9), (5, 5, 0.0)])
def test_block_column_view(mb, nbc, p):
    """tsp_bsr_col_view against a stable numpy sort of the blocks by column."""
    from trnsparse_amd.hip import dispatch as D

    g = torch.Generator().manual_seed(mb * 1000 + nbc)
    mask = torch.rand(mb, nbc, generator=g) < p
    A = W.bsr_from_block_mask(mask, 128)
    rp_h = A.block_row_ptrs.numpy()
    ci_h = A.block_col_indices.numpy()
    dev = torch.device("cuda")
    brow, cp, cbid, crow, corder = D._bsr_bwd_plan(A.block_row_ptrs.to(dev), A.block_col_indices.to(dev), mb, nbc, dev)
    want_brow = np.repeat(np.arange(mb), np.diff(rp_h))
    order = np.argsort(ci_h, kind="stable")
    want_cp = np.zeros(nbc + 1, dtype=np.int64)
    want_cp[1:] = np.cumsum(np.bincount(ci_h, minlength=nbc))
    assert np.array_equal(brow.cpu().numpy(), want_brow)
    assert np.array_equal(cp.cpu().numpy(), want_cp)
    assert np.array_equal(cbid.cpu().numpy(), order)
    assert np.array_equal(crow.cpu().numpy(), want_brow[order])
    assert sorted(corder.cpu().numpy().tolist()[:nbc]) == list(range(nbc))


@pytest.mark.parametrize("b", [8, 16, 64, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sddmm_blocks_in_any_order(hip_backend, b, dtype):
    """tsp_bsr_sddmm takes (block row, block column) per stored block in any
    order (the b = 8 kernel stages the dC rows of a chunk's first block row
    and reads the others from memory): shuffled blocks give the same blocks
    as CSR order, and each matches float64."""
    from trnsparse_amd.hip import _lib

    g = torch.Generator().manual_seed(b)
    nb_r, nb_c, N = 24, 20, 96
    mask = torch.rand(nb_r, nb_c, generator=g) < 0.4
    A = W.bsr_from_block_mask(mask, b)
    dev = torch.device("cuda")
    ptr = A.block_row_ptrs.numpy()
    brow = np.repeat(np.arange(nb_r), np.diff(ptr))
    col = A.block_col_indices.numpy()
    perm = torch.randperm(len(col), generator=g).numpy()
    G = torch.randn(nb_r * b, N, generator=g).to(dtype)
    B = torch.randn(nb_c * b, N, generator=g).to(dtype)
    Gd, Bd = G.to(dev), B.to(dev)
    outs = []
    for order in (np.arange(len(col)), perm):
        br = torch.from_numpy(brow[order].copy()).to(dev)
        cc = torch.from_numpy(col[order].copy()).to(dev)
        out = torch.full((len(col), b, b), float("nan"), dtype=dtype, device=dev)
        _lib.call("tsp_bsr_sddmm", Gd.data_ptr(), N, nb_r * b, Bd.data_ptr(), N, nb_c * b, N, br.data_ptr(),
                  cc.data_ptr(), len(col), b, _lib.dtype_code(dtype), out.data_ptr(), _lib.stream_handle(dev))
        outs.append(out.cpu())
    assert torch.equal(outs[1], outs[0][torch.from_numpy(perm)])
    Gn, Bn = G.double().numpy(), B.double().numpy()
    for k in range(len(col)):
        i, j = brow[k], col[k]
        exact = Gn[i * b:(i + 1) * b] @ Bn[j * b:(j + 1) * b].T
        scale = np.abs(Gn[i * b:(i + 1) * b]) @ np.abs(Bn[j * b:(j + 1) * b]).T
        assert ref.scaled_error(outs[0][k].double().numpy(), exact, scale) <= TOL[dtype]


@pytest.mark.parametrize("b", [8, 16, 64])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_small_blocks_at_scale(hip_backend, b, dtype):
    """Small-block forward and backward at 4096^2 with cfg3's 10 % block
    density (banded plus uniform), N = 96: every element of C, dA and dB
    against float64 (scipy BSR products), at the fp32 / bf16 bars."""
    import scipy.sparse as sp

    n, N = 4096, 96
    g = torch.Generator().manual_seed(40 + b)
    mask = W.cfg3_block_mask(n // b, half_band=3 * 128 // b, density=0.10, seed=41)
    A = W.bsr_from_block_mask(mask, b, blocks=torch.randn(int(mask.sum()), b, b, generator=g).to(dtype))
    B = torch.randn(n, N, generator=g).to(dtype)
    G = torch.randn(n, N, generator=g).to(dtype)
    blocks = A.blocks.detach().clone().cuda().requires_grad_(True)
    Bd = B.cuda().requires_grad_(True)
    Ad = ts.BSRMatrix(blocks, A.block_col_indices, A.block_row_ptrs, A.shape, b)
    C = ts.bsr_spmm(Ad, Bd)
    C.backward(G.cuda().to(C.dtype))
    blk = A.blocks.double().numpy()
    ind, ptr = A.block_col_indices.numpy(), A.block_row_ptrs.numpy()
    S = sp.bsr_matrix((blk, ind, ptr), shape=(n, n))
    Sa = sp.bsr_matrix((np.abs(blk), ind, ptr), shape=(n, n))
    Bn, Gn = B.double().numpy(), G.double().numpy()
    tol = TOL[dtype]
    assert ref.scaled_error(_np(C), S @ Bn, Sa @ np.abs(Bn)) <= tol
    assert ref.scaled_error(_np(Bd.grad), S.T @ Gn, Sa.T @ np.abs(Gn)) <= tol
    # dA block k = G[rows of i] @ B[rows of j]^T, in chunks of blocks
    brow = np.repeat(np.arange(len(ptr) - 1), np.diff(ptr))
    dA = _np(blocks.grad)
    for s0 in range(0, len(ind), 4096):
        i, j = brow[s0:s0 + 4096], ind[s0:s0 + 4096]
        Gi = Gn.reshape(-1, b, N)[i]
        Bj = Bn.reshape(-1, b, N)[j]
        exact = Gi @ Bj.transpose(0, 2, 1)
        scale = np.abs(Gi) @ np.abs(Bj).transpose(0, 2, 1)
        assert ref.scaled_error(dA[s0:s0 + 4096], exact, scale) <= tol
