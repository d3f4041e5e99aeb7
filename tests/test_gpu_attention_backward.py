"""GPU parity of the block-sparse attention backward (tsp_bsa_bwd through
autograd of block_sparse_attention_tiled) against the CPU oracle
(oracle.ref.block_sparse_attention_backward, pinned to float64 torch
autograd through dense masked attention).

The oracle takes the same Q, K, V, dO and the GPU forward's O (an input of
the backward: D = rowsum(dO * O)) and its own float64 row stats. Error
measure per gradient element: |g - g_exact| / g_abs, with g_abs the oracle's
absolute form (|dS| replaced by P (|dO V^T| + |D|), operands by their
magnitudes). fp32 <= 1e-4, bf16 <= 2e-2, fp64 <= 1e-10. fp32 with b = 128
and d in {64, 128, 256} runs the fp32 MFMA kernels (16-row tiles at
d = 256), bf16 with d <= 128 the bf16 MFMA kernels of d = 128 (d below 128
zero-padded to 128), bf16 with d = 256 and fp32 / bf16 with d > 256
block products over the mask stacked over heads (SDDMM, elementwise softmax
gradient, BSR SpMMs) when S is a whole number of blocks, other d below 256
zero-padded to 64, 128 or 256 first; everything else (fp64, ragged S at
large d, other block sizes) the generic kernels.
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


def local_mask(nb, window):
    i = torch.arange(nb)
    return (i[:, None] - i[None, :]).abs() <= window


def global_mask(nb, window, n_global):
    m = local_mask(nb, window)
    m[:n_global, :] = True
    m[:, :n_global] = True
    return m


def _np(t):
    return t.detach().double().cpu().numpy()


def _run(Q, K, V, dO, mask_bsr, scale=None):
    """Forward + backward on the GPU; returns (O, dQ, dK, dV) on the host."""
    q, k, v = (t.cuda().requires_grad_(True) for t in (Q, K, V))
    out = ts.block_sparse_attention_tiled(q, k, v, mask_bsr, scale=scale)
    out.backward(dO.cuda())
    return out.detach().cpu(), q.grad.cpu(), k.grad.cpu(), v.grad.cpu()


def _check_head(Q, K, V, dO, O, grads, mask_bsr, scale, tol, rows=None, cols=None, sel_q=None, sel_k=None):
    args = (_np(Q), _np(K), _np(V), _np(O), _np(dO), mask_bsr.block_row_ptrs.numpy(),
            mask_bsr.block_col_indices.numpy(), mask_bsr.block_size, scale)
    exact = ref.block_sparse_attention_backward(*args, rows=rows, cols=cols)
    bound = ref.block_sparse_attention_backward(*args, absolute=True, rows=rows, cols=cols)
    for i, (g, e, a) in enumerate(zip(grads, exact, bound)):
        sel = (sel_q if i == 0 else sel_k)
        g, e, a = _np(g), e, a
        if sel is not None:
            g, e, a = g[sel], e[sel], a[sel]
        err = ref.scaled_error(g, e, np.maximum(a, 1e-30))
        assert err <= tol, f"{'dQ dK dV'.split()[i]}: scaled error {err:.3g} > {tol}"


@pytest.mark.parametrize(
    "S,D,mask,dtype",
    [
        (256, 32, local_mask(2, 1), torch.float32),
        (384, 64, global_mask(3, 0, 1), torch.float32),
        (300, 16, local_mask(3, 1), torch.float64),       # ragged S: 2 query block rows, 3 key block columns
        (512, 128, local_mask(4, 1), torch.bfloat16),     # MFMA kernels
        (512, 128, global_mask(4, 1, 1), torch.bfloat16),
        (300, 128, local_mask(3, 2), torch.bfloat16),     # MFMA, last key block crosses S
        (1024, 128, global_mask(8, 1, 1), torch.bfloat16),  # MFMA, global column split into 2 segments
        (256, 64, local_mask(2, 1), torch.bfloat16),      # bf16 d = 64: zero-padded to 128, bf16 MFMA kernels
        (640, 64, W.cfg5_block_mask(5), torch.bfloat16),
        (256, 32, local_mask(2, 1), torch.bfloat16),      # head_dim zero-padded to 128
        (300, 96, local_mask(3, 1), torch.bfloat16),      # zero-padded to 128, last key block crosses S
        (256, 100, global_mask(2, 0, 1), torch.float32),  # head_dim zero-padded to 128
        (256, 160, local_mask(2, 1), torch.bfloat16),     # head_dim zero-padded to 256: block products
        (256, 320, local_mask(2, 1), torch.bfloat16),     # block products (head_dim over 256)
        (300, 320, local_mask(3, 1), torch.bfloat16),     # generic bf16 (S not whole blocks)
        (512, 512, local_mask(4, 2), torch.float32),      # block products, fp32
        (640, 512, W.cfg5_block_mask(5), torch.bfloat16),  # block products, bf16
        (512, 384, global_mask(4, 1, 1), torch.float32),
        (512, 256, local_mask(4, 2), torch.float32),      # fp32 MFMA d = 256
        (700, 256, global_mask(6, 1, 1), torch.float32),  # d = 256, ragged S, global column split
        (640, 256, W.cfg5_block_mask(5), torch.float32),
        (300, 200, local_mask(3, 2), torch.float32),      # zero-padded to 256, last key block crosses S
        (512, 256, local_mask(4, 1), torch.bfloat16),     # bf16 d = 256: block products on bf16 MFMA
        (512, 128, local_mask(4, 1), torch.float32),      # fp32 MFMA kernels
        (1024, 128, global_mask(8, 1, 1), torch.float32),  # fp32 MFMA, global column split into 2 segments
        (300, 128, local_mask(3, 2), torch.float32),      # fp32 MFMA, last key block crosses S
        (640, 64, W.cfg5_block_mask(5), torch.float32),   # fp32 MFMA d = 64, global columns split
        (700, 64, torch.ones(6, 6, dtype=torch.bool), torch.float32),
    ],
)
def test_backward_matches_oracle(hip_backend, S, D, mask, dtype):
    g = torch.Generator().manual_seed(S + D)
    mask_bsr = W.bsr_from_block_mask(mask, 128)
    Q, K, V, dO = (torch.randn(S, D, generator=g, dtype=torch.float64).to(dtype) for _ in range(4))
    O, dQ, dK, dV = _run(Q, K, V, dO, mask_bsr)
    assert dQ.dtype == dtype and dK.shape == K.shape
    _check_head(Q, K, V, dO, O, (dQ, dK, dV), mask_bsr, D**-0.5, TOL[dtype])


@pytest.mark.parametrize("dtype,D", [(torch.float32, 128), (torch.bfloat16, 128), (torch.float32, 256)])
def test_backward_empty_rows_and_ragged(hip_backend, dtype, D):
    """Block row 1 stores nothing, block column 2 is never stored, rows past
    (S // b) b have no block row: their gradients are exactly zero."""
    S = 440
    mask = torch.tensor([[True, False, False, True], [False, False, False, False],
                         [True, True, False, False], [False, False, False, True]])
    mask_bsr = W.bsr_from_block_mask(mask, 128)
    g = torch.Generator().manual_seed(3)
    Q, K, V, dO = (torch.randn(S, D, generator=g, dtype=torch.float64).to(dtype) for _ in range(4))
    O, dQ, dK, dV = _run(Q, K, V, dO, mask_bsr, scale=0.1)
    assert torch.count_nonzero(dQ[128:256]).item() == 0
    assert torch.count_nonzero(dQ[384:]).item() == 0
    assert torch.count_nonzero(dK[256:384]).item() == 0 and torch.count_nonzero(dV[256:384]).item() == 0
    _check_head(Q, K, V, dO, O, (dQ, dK, dV), mask_bsr, 0.1, TOL[dtype])


@pytest.mark.parametrize("D", [128, 64])
def test_backward_batched_heads_bf16(hip_backend, D):
    """Leading (batch, head) dims; at D = 64 the operands are zero-padded to
    128 and the gradients cut back to 64 columns."""
    torch.manual_seed(12)
    S = 512
    mask_bsr = W.bsr_from_block_mask(global_mask(4, 1, 1), 128)
    Q, K, V, dO = (torch.randn(2, 2, S, D).to(torch.bfloat16) for _ in range(4))
    O, dQ, dK, dV = _run(Q, K, V, dO, mask_bsr)
    assert dQ.shape == Q.shape
    for i in range(Q.shape[0]):
        for hh in range(Q.shape[1]):
            _check_head(Q[i, hh], K[i, hh], V[i, hh], dO[i, hh], O[i, hh], (dQ[i, hh], dK[i, hh], dV[i, hh]), mask_bsr,
                        D**-0.5, TOL[torch.bfloat16])


@pytest.mark.parametrize("D", [64, 256])
def test_backward_batched_heads_f32(hip_backend, D):
    """fp32 MFMA kernels over 3 heads: the column pass's (item, head) grid."""
    torch.manual_seed(15)
    S = 512
    mask_bsr = W.bsr_from_block_mask(global_mask(4, 1, 1), 128)
    Q, K, V, dO = (torch.randn(3, S, D) for _ in range(4))
    O, dQ, dK, dV = _run(Q, K, V, dO, mask_bsr)
    for hh in range(3):
        _check_head(Q[hh], K[hh], V[hh], dO[hh], O[hh], (dQ[hh], dK[hh], dV[hh]), mask_bsr, D**-0.5,
                    TOL[torch.float32])


def test_backward_f32_long_row(hip_backend):
    """A query block row with more than 64 stored blocks (the row pass reads
    the row's block columns 64 at a time)."""
    nb, D = 67, 64
    S = nb * 128
    mask = local_mask(nb, 0)
    mask[1, :] = True
    mask_bsr = W.bsr_from_block_mask(mask, 128)
    g = torch.Generator().manual_seed(16)
    Q, K, V, dO = (torch.randn(S, D, generator=g) for _ in range(4))
    O, dQ, dK, dV = _run(Q, K, V, dO, mask_bsr)
    rows, cols = [1, 2], [0, 1, 66]
    sel_q = np.concatenate([np.arange(r * 128, (r + 1) * 128) for r in rows])
    sel_k = np.concatenate([np.arange(c * 128, (c + 1) * 128) for c in cols])
    _check_head(Q, K, V, dO, O, (dQ, dK, dV), mask_bsr, D**-0.5, TOL[torch.float32], rows=rows, cols=cols,
                sel_q=sel_q, sel_k=sel_k)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_backward_deterministic(hip_backend, dtype):
    torch.manual_seed(13)
    mask_bsr = W.bsr_from_block_mask(global_mask(4, 1, 1), 128)
    Q, K, V, dO = (torch.randn(2, 512, 128).to(dtype) for _ in range(4))
    a = _run(Q, K, V, dO, mask_bsr)
    b = _run(Q, K, V, dO, mask_bsr)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_cfg5_backward_full_size(hip_backend):
    """cfg5 (32 heads, S 8192, d 128, 370 mask blocks): on every head, sampled
    block rows of dQ and block columns of dK / dV against the oracle, and the identity
    sum_k dV[k] = sum over queries of non-empty block rows of dO[q] (each
    softmax row sums to one) on every head."""
    Q, K, V, mask_bsr = W.cfg5_attention()
    dO = torch.randn(Q.shape, generator=torch.Generator().manual_seed(14)).to(torch.bfloat16)
    O, dQ, dK, dV = _run(Q, K, V, dO, mask_bsr)
    ptr = mask_bsr.block_row_ptrs.numpy()
    rows, cols = [0, 1, 5, 63], [0, 2, 40, 63]
    sel_q = np.concatenate([np.arange(r * 128, (r + 1) * 128) for r in rows])
    sel_k = np.concatenate([np.arange(c * 128, (c + 1) * 128) for c in cols])
    for hh in range(Q.shape[0]):  # all 32 heads
        _check_head(Q[hh], K[hh], V[hh], dO[hh], O[hh], (dQ[hh], dK[hh], dV[hh]), mask_bsr, 128**-0.5,
                    TOL[torch.bfloat16], rows=rows, cols=cols, sel_q=sel_q, sel_k=sel_k)
    live = np.repeat(np.diff(ptr)[: 8192 // 128] > 0, 128)
    dOd = dO.double().numpy()
    got = dV.double().sum(dim=1).numpy()                 # (H, D)
    expect = dOd[:, live].sum(axis=1)
    bound = np.abs(dOd[:, live]).sum(axis=1) * 2e-2 / 8  # bf16 P and dV rounding, summed magnitudes
    assert (np.abs(got - expect) <= bound + 1e-3).all()


def test_cfg5_backward_full_size_f32(hip_backend):
    """cfg5's shapes and mask with fp32 Q, K, V, dO (the fp32 MFMA kernels):
    on every head, sampled block rows of dQ and block columns of dK / dV
    against the oracle."""
    Q, K, V, mask_bsr = W.cfg5_attention()
    Q, K, V = Q.float(), K.float(), V.float()
    dO = torch.randn(Q.shape, generator=torch.Generator().manual_seed(14))
    O, dQ, dK, dV = _run(Q, K, V, dO, mask_bsr)
    rows, cols = [0, 1, 5, 63], [0, 1, 2, 40, 63]
    sel_q = np.concatenate([np.arange(r * 128, (r + 1) * 128) for r in rows])
    sel_k = np.concatenate([np.arange(c * 128, (c + 1) * 128) for c in cols])
    for hh in range(Q.shape[0]):  # all 32 heads
        _check_head(Q[hh], K[hh], V[hh], dO[hh], O[hh], (dQ[hh], dK[hh], dV[hh]), mask_bsr, 128**-0.5,
                    TOL[torch.float32], rows=rows, cols=cols, sel_q=sel_q, sel_k=sel_k)


@pytest.mark.parametrize("D,dtype", [(256, torch.bfloat16), (512, torch.float32), (512, torch.bfloat16)])
def test_backward_block_products_batched_heads(hip_backend, D, dtype):
    """Block-product backward over 4 heads (the stacked pattern), with an
    empty block row: every head's gradients against the oracle."""
    torch.manual_seed(70)
    H, S = 4, 512
    mask = global_mask(4, 1, 1)
    mask[2, :] = False
    mask_bsr = W.bsr_from_block_mask(mask, 128)
    Q, K, V, dO = (torch.randn(H, S, D).to(dtype) for _ in range(4))
    O, dQ, dK, dV = _run(Q, K, V, dO, mask_bsr)
    assert torch.count_nonzero(dQ[:, 256:384]).item() == 0
    for hh in range(H):
        _check_head(Q[hh], K[hh], V[hh], dO[hh], O[hh], (dQ[hh], dK[hh], dV[hh]), mask_bsr, D**-0.5, TOL[dtype])
