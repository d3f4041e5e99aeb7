"""GPU parity of BSR times one vector (tsp_bsr_spmv: bsr_spmm with N = 1 and
the fused solver update) and of the fixed-step solvers built on it, against
the CPU oracle (oracle.ref.bsr_spmm / richardson / chebyshev, float64).

Tolerances: fp32 <= 1e-4 and bf16 <= 2e-2 relative to the dot-product
scale |A|.|x| per entry (as the SpMM tests); fp64 <= 1e-10. Solvers: the
fp32 iterate within 1e-4 of the float64 oracle iterate, relative to its
largest entry.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import trnsparse_amd as ts
from oracle import ref
from trnsparse_amd import workloads as W
from trnsparse_amd.hip import _lib
from trnsparse_amd.hip.dispatch import hip_bsr_matvec_update

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float64: 1e-10}


def _np(t):
    return t.detach().double().cpu().numpy()


def _oracle(A: ts.BSRMatrix, x, absolute=False):
    return ref.bsr_spmm(_np(A.blocks), A.block_col_indices.numpy(), A.block_row_ptrs.numpy(), A.shape, A.block_size,
                        _np(x)[:, None], absolute=absolute)[:, 0]


@pytest.mark.parametrize(
    "shape,b,density,dtype",
    [
        ((1024, 1024), 128, 0.3, torch.float32),   # b = 128 kernel
        ((1000, 900), 128, 0.4, torch.float32),    # ragged: x read as zero past n, rows past m skipped
        ((512, 768), 128, 0.5, torch.float64),
        ((512, 512), 128, 0.5, torch.bfloat16),
        ((200, 150), 16, 0.3, torch.float32),      # other block sizes: thread per row
        ((64, 64), 8, 0.5, torch.float64),
    ],
)
def test_bsr_spmm_one_column_matches_oracle(hip_backend, shape, b, density, dtype):
    g = torch.Generator().manual_seed(shape[0] + b)
    A = torch.randn(*shape, generator=g, dtype=torch.float64) * (torch.rand(*shape, generator=g) < density)
    bsr = ts.BSRMatrix.from_dense(A.to(dtype), block_size=b)
    x = torch.randn(shape[1], 1, generator=g, dtype=torch.float64).to(dtype)
    y = ts.bsr_spmm(bsr, x.cuda())
    assert y.shape == (shape[0], 1) and y.dtype == dtype
    exact, scale = _oracle(bsr, x[:, 0]), _oracle(bsr, x[:, 0], absolute=True)
    assert ref.scaled_error(_np(y[:, 0]), exact, scale) <= TOL[dtype]


def test_bsr_spmm_one_column_empty_rows(hip_backend):
    mask = torch.tensor([[True, False], [False, False], [False, True]])
    bsr = W.bsr_from_block_mask(mask, 128)
    bsr = ts.BSRMatrix(torch.randn(bsr.n_blocks, 128, 128), bsr.block_col_indices, bsr.block_row_ptrs, bsr.shape, 128)
    x = torch.randn(256, 1)
    y = ts.bsr_spmm(bsr, x.cuda()).cpu()
    assert torch.count_nonzero(y[128:256]).item() == 0
    assert ref.scaled_error(y[:, 0].numpy(), _oracle(bsr, x[:, 0]), _oracle(bsr, x[:, 0], True)) <= TOL[torch.float32]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_fused_update_terms(hip_backend, dtype):
    """out = alpha A x + beta u + gamma v + delta w, and out may be u / w."""
    A, _, _ = W.spd_bsr(nb=6, b=128, band=1, n_pairs=2, dtype=dtype)
    n = A.shape[0]
    g = torch.Generator().manual_seed(4)
    x, u, v, w = (torch.randn(n, generator=g, dtype=torch.float64).to(dtype).cuda() for _ in range(4))
    Ax = _oracle(A, x)
    want = -0.7 * Ax + 1.3 * _np(u) + 0.25 * _np(v) - 0.5 * _np(w)
    scale = 0.7 * _oracle(A, x, True) + 1.3 * np.abs(_np(u)) + 0.25 * np.abs(_np(v)) + 0.5 * np.abs(_np(w))
    out = hip_bsr_matvec_update(A, x, -0.7, torch.empty_like(x), u=u, beta=1.3, v=v, gamma=0.25, w=w, delta=-0.5)
    assert ref.scaled_error(_np(out), want, scale) <= TOL[dtype]
    ww = w.clone()
    hip_bsr_matvec_update(A, x, -0.7, ww, u=u, beta=1.3, v=v, gamma=0.25, w=ww, delta=-0.5)  # out aliases w
    assert torch.equal(ww, out)
    with pytest.raises(RuntimeError, match="alias"):
        hip_bsr_matvec_update(A, x, 1.0, x)


@pytest.mark.parametrize("nb,band,pairs", [(8, 1, 3), (32, 2, 40)])
def test_richardson_and_chebyshev_match_oracle(hip_backend, nb, band, pairs):
    A, lo, hi = W.spd_bsr(nb=nb, b=128, band=band, n_pairs=pairs)
    n = A.shape[0]
    rhs = torch.randn(n, generator=torch.Generator().manual_seed(nb))
    Ad = ts.BSRMatrix(A.blocks.cuda(), A.block_col_indices.cuda(), A.block_row_ptrs.cuda(), A.shape, 128)
    mv = ref.bsr_matvec(_np(A.blocks), A.block_col_indices.numpy(), A.block_row_ptrs.numpy(), A.shape, 128)
    omega = 2.0 / (lo + hi)
    x, K, rel = ts.richardson_bsr(Ad, rhs.cuda(), omega, K=30)
    want = ref.richardson(mv, rhs.double().numpy(), omega, 30)
    assert x.is_cuda and K == 30
    assert np.abs(_np(x) - want).max() <= 1e-4 * np.abs(want).max()
    r = rhs.double().numpy() - mv(want)
    assert abs(rel - np.linalg.norm(r) / np.linalg.norm(rhs.double().numpy())) <= 1e-4
    x, K, rel = ts.chebyshev_bsr(Ad, rhs.cuda(), lo, hi, K=25)
    alpha, beta = ref.chebyshev_coeffs(lo, hi, 25)
    want = ref.chebyshev(mv, rhs.double().numpy(), alpha, beta, 25)
    assert np.abs(_np(x) - want).max() <= 1e-4 * np.abs(want).max()
    assert rel < 1e-3  # converges on SPD A with valid bounds


def test_spmv_entry_point_rejects_bad_sizes(hip_backend):
    lib = _lib.load()
    assert lib.tsp_bsr_spmv(None, 0, None, None, 0, 0, 1, 1, None, 1.0, None, 0.0, None, 0.0, None, 0.0, None, None,
                            None) == -1
    assert lib.tsp_bsr_spmv(None, 9, None, None, 0, 128, 1, 1, None, 1.0, None, 0.0, None, 0.0, None, 0.0, None, None,
                            None) == -2
