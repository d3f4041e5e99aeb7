"""CPU tests of the host logic: the explicit "pytorch" backend (the
reference's torch semantics) against the oracle, the reference's known
answers, and the backend switch — including that the HIP backend fails
loudly instead of falling back."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import trnsparse_amd as ts
from oracle import ref
from trnsparse_amd import backend
from trnsparse_amd import workloads as W


@pytest.fixture(autouse=True)
def _pytorch(pytorch_backend):
    yield


def test_spmv_spmm_known_answers():
    csr = ts.from_dense(torch.tensor([[2.0, 0.0], [0.0, 3.0]]))
    out = ts.spmv(csr, torch.ones(2), alpha=2.0, y=torch.tensor([10.0, 20.0]), beta=0.5)
    np.testing.assert_allclose(out.numpy(), [9.0, 16.0])
    out = ts.spmm(ts.from_dense(torch.eye(2)), torch.ones(2, 3), alpha=2.0, C=torch.ones(2, 3) * 10, beta=0.5)
    np.testing.assert_allclose(out.numpy(), np.full((2, 3), 7.0))
    with pytest.raises(AssertionError):
        ts.spmv(csr, torch.ones(3))


def test_spmv_symmetric_add_scale():
    A = torch.tensor([[4.0, 1.0, 0.0], [1.0, 3.0, 2.0], [0.0, 2.0, 5.0]])
    x = torch.tensor([1.0, 2.0, 3.0])
    np.testing.assert_allclose(ts.spmv_symmetric(ts.from_dense(torch.triu(A)), x).numpy(), (A @ x).numpy(), atol=1e-6)
    C = ts.sparse_add(ts.from_dense(torch.tensor([[1.0, 0.0], [0.0, 2.0]])), ts.from_dense(torch.tensor([[0.0, 3.0], [4.0, 0.0]])))
    np.testing.assert_allclose(C.to_dense().numpy(), [[1.0, 3.0], [4.0, 2.0]])
    np.testing.assert_allclose(ts.sparse_scale(ts.from_dense(torch.eye(2)), 3.0).to_dense().numpy(), 3 * np.eye(2))


@pytest.mark.parametrize("shape,b,density", [((24, 24), 8, 0.5), ((20, 14), 8, 1.0), ((256, 384), 128, 0.5)])
def test_bsr_spmm_vs_oracle(shape, b, density):
    g = torch.Generator().manual_seed(5)
    A = torch.randn(*shape, generator=g) * (torch.rand(*shape, generator=g) < density)
    bsr = ts.BSRMatrix.from_dense(A, block_size=b)
    B = torch.randn(shape[1], 12, generator=g)
    got = ts.bsr_spmm(bsr, B)
    args = (bsr.blocks.numpy(), bsr.block_col_indices.numpy(), bsr.block_row_ptrs.numpy(), bsr.shape, b)
    exact, scale = ref.bsr_spmm(*args, B.numpy()), ref.bsr_spmm(*args, B.numpy(), absolute=True)
    assert ref.scaled_error(got.numpy(), exact, scale) <= 1e-5
    empty = ts.BSRMatrix.from_dense(torch.zeros(16, 16), block_size=8)
    assert torch.count_nonzero(ts.bsr_spmm(empty, torch.randn(16, 8))).item() == 0


def test_bsr_spmm_out_dtype_bf16():
    A, B = W.cfg3_bsr(nb=4, ncols=16, dtype=torch.bfloat16, density=0.5)
    got = ts.bsr_spmm(A, B, out_dtype=torch.float32)
    assert got.dtype == torch.float32
    args = (A.blocks.float().numpy(), A.block_col_indices.numpy(), A.block_row_ptrs.numpy(), A.shape, 128)
    exact = ref.bsr_spmm(*args, B.float().numpy())
    scale = ref.bsr_spmm(*args, B.float().numpy(), absolute=True)
    assert ref.scaled_error(got.numpy(), exact, scale) <= 1e-5


def test_screened_vs_oracle_and_known_cases():
    torch.manual_seed(2)
    n = 64
    A = torch.randn(n, n)
    diag = torch.abs(torch.randn(n)) * 4.0
    B = torch.randn(n, 16)
    for thr in (0.0, 0.5, 1e30):
        got = ts.screened_spmm(A, diag, B, threshold=thr)
        exact = ref.screened_spmm(A.numpy(), diag.numpy(), B.numpy(), thr)
        scale = ref.screened_spmm(A.numpy(), diag.numpy(), B.numpy(), thr, absolute=True)
        assert ref.scaled_error(got.numpy(), exact, scale) <= 1e-5
    assert torch.count_nonzero(ts.screened_spmm(A, diag, B, threshold=1e30)).item() == 0
    with pytest.raises(AssertionError):
        ts.screened_spmm(A, diag[:10], B, 0.5)
    assert np.array_equal(ts.screened_mask(diag, 0.5).numpy(), ref.screened_mask(diag.numpy(), 0.5))


def test_attention_tiled_vs_oracle_and_stats():
    torch.manual_seed(10)
    S, D = 384, 32
    Q, K, V = (torch.randn(S, D) for _ in range(3))
    mask = torch.tensor([[1, 1, 0], [0, 0, 0], [1, 0, 1]], dtype=torch.bool)
    mbsr = W.bsr_from_block_mask(mask, 128)
    got = ts.block_sparse_attention_tiled(Q, K, V, mbsr)
    out, rmax, rden = ref.block_sparse_attention(Q.numpy(), K.numpy(), V.numpy(), mbsr.block_row_ptrs.numpy(),
                                                 mbsr.block_col_indices.numpy(), 128, D**-0.5)
    np.testing.assert_allclose(got.numpy(), out, atol=1e-5, rtol=1e-4)
    from trnsparse_amd.ops import _block_sparse_attn_pytorch

    _, rm, rd = _block_sparse_attn_pytorch(Q, K, V, mbsr, D**-0.5, return_stats=True)
    np.testing.assert_allclose(rm.numpy(), rmax, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(rd.numpy(), rden, rtol=1e-5)


def test_attention_gradcheck_pytorch_backend():
    torch.manual_seed(40)
    mbsr = W.bsr_from_block_mask(torch.tensor([[True, True, False], [False, True, False], [True, False, True]]), 8)
    Q, K, V = (torch.randn(24, 4, dtype=torch.float64, requires_grad=True) for _ in range(3))
    assert torch.autograd.gradcheck(lambda q, k, v: ts.block_sparse_attention_tiled(q, k, v, mbsr), (Q, K, V),
                                    eps=1e-4, atol=1e-3, rtol=1e-3)


def test_attention_batched_equals_per_head():
    torch.manual_seed(3)
    Q, K, V = (torch.randn(3, 256, 16) for _ in range(3))
    mbsr = W.bsr_from_block_mask(torch.ones(2, 2, dtype=torch.bool), 128)
    got = ts.block_sparse_attention_tiled(Q, K, V, mbsr)
    for h in range(3):
        torch.testing.assert_close(got[h], ts.block_sparse_attention_tiled(Q[h], K[h], V[h], mbsr))


# ------------------------------------------------------------ backend switch


def test_backend_names_and_errors():
    assert ts.get_backend() == "pytorch"
    with pytest.raises(AssertionError):
        ts.set_backend("cuda")
    with pytest.raises(RuntimeError):
        ts.set_backend("nki")
    assert ts.HAS_NKI is False


@pytest.mark.skipif(torch.cuda.is_available(), reason="CPU-only check")
def test_hip_backend_without_gpu_raises():
    with pytest.raises(RuntimeError):
        ts.set_backend("hip")
    ts.set_backend("auto")
    assert backend._use_hip() is False  # auto resolves to the torch path without a GPU
    assert ts.has_hip() is False


def test_hip_path_never_falls_back(monkeypatch):
    """With the HIP backend forced, a missing library raises instead of
    quietly computing with torch."""
    from trnsparse_amd.hip import _lib

    monkeypatch.setattr(backend, "_backend", "hip")
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", _lib.LIB_PATH.with_name("missing_lib.so"))
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load()
    A = ts.BSRMatrix.from_dense(torch.randn(16, 16), block_size=8)
    with pytest.raises(Exception) as exc:
        ts.bsr_spmm(A, torch.randn(16, 4))
    assert not isinstance(exc.value, AssertionError)
