"""`import trnsparse` — the reference's import name — reaches this build.

The reference's tests and callers import `trnsparse`
(reference tests/test_ops.py, test_bsr.py, test_formats.py). These CPU
tests run the reference's known answers through that name, on the
"pytorch" backend, and check that the names are the very objects of
trnsparse_amd, so the HIP routing behind them is the same.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch


def test_names_are_trnsparse_amd_objects():
    import trnsparse
    import trnsparse.formats
    import trnsparse_amd
    from trnsparse.nki import HAS_NKI, get_backend, set_backend
    from trnsparse.nki.dispatch import _use_nki
    from trnsparse.ops import spmv

    for name in trnsparse_amd.__all__:
        assert getattr(trnsparse, name) is getattr(trnsparse_amd, name), name
    assert trnsparse.formats is trnsparse_amd.formats
    assert spmv is trnsparse_amd.spmv
    assert (HAS_NKI, get_backend, set_backend) == (False, trnsparse_amd.get_backend, trnsparse_amd.set_backend)
    assert _use_nki() is False
    assert trnsparse.__version__ == trnsparse_amd.__version__


@pytest.fixture
def pytorch_via_name():
    import trnsparse

    prev = trnsparse.get_backend()
    trnsparse.set_backend("pytorch")
    yield trnsparse
    trnsparse.set_backend(prev)


def test_known_answers_through_the_reference_name(pytorch_via_name):
    trnsparse = pytorch_via_name
    # spmv: y = alpha * A x + beta * y  ->  [9, 16]
    A = trnsparse.from_dense(torch.tensor([[2.0, 0.0], [0.0, 3.0]]))
    out = trnsparse.spmv(A, torch.ones(2), alpha=2.0, y=torch.tensor([10.0, 20.0]), beta=0.5)
    np.testing.assert_allclose(out.numpy(), [9.0, 16.0])
    # spmm with C: 2 * I @ 1 + 0.5 * 10 = 7
    out = trnsparse.spmm(trnsparse.from_dense(torch.eye(2)), torch.ones(2, 3), alpha=2.0, C=torch.ones(2, 3) * 10,
                         beta=0.5)
    np.testing.assert_allclose(out.numpy(), np.full((2, 3), 7.0))
    # identity SpMV returns x
    x = torch.tensor([1.5, -2.0, 3.25])
    np.testing.assert_allclose(trnsparse.spmv(trnsparse.eye_sparse(3), x).numpy(), x.numpy())
    with pytest.raises(AssertionError):
        trnsparse.spmv(A, torch.ones(3))
    # bsr_spmm equals the dense product; an empty pattern gives exact zeros
    g = torch.Generator().manual_seed(0)
    D = torch.randn(32, 24, generator=g) * (torch.rand(32, 24, generator=g) < 0.5)
    bsr = trnsparse.BSRMatrix.from_dense(D, block_size=8)
    B = torch.randn(24, 5, generator=g)
    torch.testing.assert_close(trnsparse.bsr_spmm(bsr, B), D @ B, rtol=1e-5, atol=1e-5)
    empty = trnsparse.BSRMatrix.from_dense(torch.zeros(16, 16), block_size=8)
    assert torch.count_nonzero(trnsparse.bsr_spmm(empty, torch.randn(16, 4))).item() == 0
    # screened_spmm: threshold 0 keeps everything, a huge one screens everything
    A2, d2, B2 = torch.randn(16, 16, generator=g), torch.rand(16, generator=g) + 0.1, torch.randn(16, 4, generator=g)
    torch.testing.assert_close(trnsparse.screened_spmm(A2, d2, B2, 0.0), A2 @ B2, rtol=1e-5, atol=1e-5)
    assert torch.count_nonzero(trnsparse.screened_spmm(A2, d2, B2, 1e30)).item() == 0
    # a full mask makes block-sparse attention dense attention
    S, Dh = 32, 8
    Q, K, V = (torch.randn(S, Dh, generator=g) for _ in range(3))
    mask = trnsparse.BSRMatrix.from_dense(torch.ones(S, S), block_size=16)
    want = torch.softmax((Q @ K.T) * Dh**-0.5, dim=-1) @ V
    torch.testing.assert_close(trnsparse.block_sparse_attention_tiled(Q, K, V, mask), want, rtol=1e-5, atol=1e-5)


def test_set_backend_through_nki_module():
    import trnsparse
    from trnsparse.nki import get_backend, set_backend

    prev = get_backend()
    try:
        set_backend("pytorch")
        assert trnsparse.get_backend() == "pytorch"
        with pytest.raises(AssertionError):
            set_backend("cuda")
        with pytest.raises(RuntimeError):
            set_backend("nki")
    finally:
        set_backend(prev)
