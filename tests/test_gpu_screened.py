"""GPU parity of screened_spmm (fused mask + fp32 MFMA GEMM) against the oracle.

The mask is checked bit-exactly (A = ones, B = identity makes C the mask
itself), including Q_i*Q_j landing exactly on fl32(sqrt(threshold)); values
are checked against the float64 oracle with the dot-product error scale
(fp32 tolerance 1e-4), plus the reference's own cases
(tests/test_screening.py:76-133 and tests/test_nki_screened_spmm.py:33-55).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import trnsparse_amd as ts
from oracle import ref
from trnsparse_amd import workloads as W

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _check(A, diag, B, thr, got, rows=None):
    An, dn, Bn = A.cpu().numpy(), diag.cpu().numpy(), B.cpu().numpy()
    mask = ref.screened_mask(dn, thr)
    if rows is not None:
        mask, An, got = mask[rows], An[rows], got[rows]
    Am = np.where(mask, An.astype(np.float64), 0.0)
    exact = Am @ Bn.astype(np.float64)
    scale = np.abs(Am) @ np.abs(Bn.astype(np.float64))
    err = ref.scaled_error(got.cpu().numpy() if isinstance(got, torch.Tensor) else got, exact, scale)
    assert err <= TOL, err


def test_threshold_zero_equals_matmul(hip_backend):
    torch.manual_seed(0)
    n = 64
    A = torch.randn(n, n)
    diag = torch.abs(torch.randn(n)) + 0.1
    B = torch.randn(n, 16)
    got = ts.screened_spmm(A, diag, B.cuda(), threshold=0.0).cpu()
    torch.testing.assert_close(got, A @ B, atol=1e-5, rtol=1e-5)


def test_huge_threshold_exact_zeros(hip_backend):
    torch.manual_seed(1)
    n = 64
    got = ts.screened_spmm(torch.randn(n, n), torch.abs(torch.randn(n)), torch.randn(n, 16).cuda(), threshold=1e30)
    torch.testing.assert_close(got.cpu(), torch.zeros(n, 16), atol=0, rtol=0)


def test_parity_vs_explicit_mask(hip_backend):
    torch.manual_seed(2)
    n = 64
    A = torch.randn(n, n)
    diag = torch.abs(torch.randn(n)) * 4.0
    B = torch.randn(n, 16)
    got = ts.screened_spmm(A, diag, B.cuda(), threshold=0.5).cpu()
    Q = torch.sqrt(torch.abs(diag))
    mask = (Q.unsqueeze(-1) * Q.unsqueeze(0)) > math.sqrt(0.5)
    torch.testing.assert_close(got, (A * mask.to(A.dtype)) @ B, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("n,N,threshold", [(128, 128, 0.0), (128, 128, 0.5), (256, 128, 0.5), (256, 256, 0.1),
                                           (200, 64, 0.3), (300, 130, 0.2)])
def test_reference_hardware_grid(hip_backend, n, N, threshold):
    torch.manual_seed(42)
    A = torch.randn(n, n)
    diag = torch.abs(torch.randn(n)) * 4.0 + 0.01
    B = torch.randn(n, N)
    got = ts.screened_spmm(A, diag, B.cuda(), threshold=threshold).cpu()
    Q = torch.sqrt(torch.abs(diag))
    mask = (Q.unsqueeze(-1) * Q.unsqueeze(0)) > math.sqrt(max(threshold, 0.0))
    torch.testing.assert_close(got, (A * mask.to(A.dtype)) @ B, atol=1e-3, rtol=1e-4)
    _check(A, diag, B, threshold, got)


@pytest.mark.parametrize("diag_dtype", [torch.float32, torch.float64])
def test_mask_bit_exact_at_threshold(hip_backend, diag_dtype):
    """C = (ones * mask) @ I = mask; Q values put some products exactly on
    the rounded threshold (not kept: strict >) and one ulp above (kept)."""
    n = 384
    rng = np.random.default_rng(5)
    npdt = np.float32 if diag_dtype == torch.float32 else np.float64
    t = npdt(math.sqrt(1e-20))  # threshold rounded to diag's precision
    Q = (10.0 ** rng.uniform(-12, 0, n)).astype(npdt)
    Q[0] = npdt(1.0)
    Q[1] = t  # Q0*Q1 == t exactly
    Q[2] = np.nextafter(t, npdt(1))  # one ulp above
    Q[3] = np.nextafter(t, npdt(0))
    diag = torch.from_numpy((Q.astype(np.float64) ** 2).astype(npdt))
    Qr = np.sqrt(np.abs(diag.numpy())).astype(npdt)
    A = torch.ones(n, n)
    Bm = torch.eye(n)
    got = ts.screened_spmm(A, diag, Bm.cuda(), threshold=1e-20).cpu().numpy()
    expect = ref.screened_mask(diag.numpy(), 1e-20).astype(np.float32)
    assert np.array_equal(got, expect)
    if Qr[0] * Qr[1] == t:  # the square/sqrt round trip kept the value
        assert got[0, 1] == 0.0


def test_tile_skip_structured(hip_backend):
    """Rows/cols 128..255 have tiny Q: every tile pair touching them is fully
    masked and skipped; the result still equals the oracle."""
    n = 512
    g = torch.Generator().manual_seed(6)
    diag = torch.rand(n, generator=g) + 0.5
    diag[128:256] = 1e-30
    A = torch.randn(n, n, generator=g)
    B = torch.randn(n, 96, generator=g)
    got = ts.screened_spmm(A, diag, B.cuda(), threshold=1e-12).cpu()
    assert torch.count_nonzero(got[128:256]).item() == 0
    _check(A, diag, B, 1e-12, got)


@pytest.mark.parametrize("n,N,threshold,diag_dtype", [
    (256, 64, 0.3, torch.float64), (300, 200, 1e-6, torch.float64), (512, 128, 1e-12, torch.float32),
    (128, 8, 0.0, torch.float64),
])
def test_f64_mfma(hip_backend, n, N, threshold, diag_dtype):
    """fp64 A and B (even n) run screened_f64_dma: against the float64 oracle
    at 1e-12 of the dot-product scale; rows 128..255 (when present) have tiny
    Q, so their tile pairs are skipped."""
    g = torch.Generator().manual_seed(n + N)
    diag = (torch.rand(n, generator=g, dtype=torch.float64) + 0.1).to(diag_dtype)
    if n >= 256:
        diag[128:256] = 1e-30
    A = torch.randn(n, n, generator=g, dtype=torch.float64)
    B = torch.randn(n, N, generator=g, dtype=torch.float64)
    got = ts.screened_spmm(A.cuda(), diag.cuda(), B.cuda(), threshold=threshold).cpu()
    assert got.dtype == torch.float64
    mask = ref.screened_mask(diag.numpy(), threshold)
    Am = np.where(mask, A.numpy(), 0.0)
    err = ref.scaled_error(got.numpy(), Am @ B.numpy(), np.abs(Am) @ np.abs(B.numpy()))
    assert err <= 1e-12, err


def test_f64_mfma_mask_exact(hip_backend):
    """(ones * mask) @ I in fp64 reproduces the mask exactly."""
    n = 256
    rng = np.random.default_rng(8)
    diag = torch.from_numpy(10.0 ** rng.uniform(-16, 0, n))
    got = ts.screened_spmm(torch.ones(n, n, dtype=torch.float64).cuda(), diag.cuda(),
                           torch.eye(n, dtype=torch.float64).cuda(), threshold=1e-10).cpu().numpy()
    assert np.array_equal(got, ref.screened_mask(diag.numpy(), 1e-10).astype(np.float64))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_16bit_operands(hip_backend, dtype):
    """bf16 / fp16 A and B (fp32 diag): C in A's dtype within the 16-bit
    tolerance of the dot-product scale; the mask is the fp32 one."""
    n, N = 384, 96
    g = torch.Generator().manual_seed(9)
    diag = torch.rand(n, generator=g) + 0.05
    diag[128:256] = 1e-30
    A = torch.randn(n, n, generator=g).to(dtype)
    B = torch.randn(n, N, generator=g).to(dtype)
    got = ts.screened_spmm(A.cuda(), diag.cuda(), B.cuda(), threshold=1e-8).cpu()
    assert got.dtype == dtype
    mask = ref.screened_mask(diag.numpy(), 1e-8)
    Am = np.where(mask, A.double().numpy(), 0.0)
    Bn = B.double().numpy()
    err = ref.scaled_error(got.double().numpy(), Am @ Bn, np.abs(Am) @ np.abs(Bn))
    assert err <= 2e-2, err
    assert torch.count_nonzero(got[128:256]).item() == 0


def test_f64_generic_and_gradcheck(hip_backend):
    torch.manual_seed(7)
    n = 41  # odd: the generic kernel
    A = torch.randn(n, n, dtype=torch.float64, device="cuda", requires_grad=True)
    diag = (torch.abs(torch.randn(n, dtype=torch.float64)) * 4.0 + 0.01).cuda()
    B = torch.randn(n, 5, dtype=torch.float64, device="cuda", requires_grad=True)
    got = ts.screened_spmm(A, diag, B, threshold=0.5)
    Q = torch.sqrt(torch.abs(diag))
    mask = ((Q.unsqueeze(-1) * Q.unsqueeze(0)) > math.sqrt(0.5)).double()
    torch.testing.assert_close(got, (A * mask) @ B, rtol=1e-12, atol=1e-12)
    assert torch.autograd.gradcheck(lambda a, b: ts.screened_spmm(a, diag, b, threshold=0.5), (A, B), eps=1e-6, atol=1e-6)


def test_cfg4_full_size(hip_backend):
    A, diag, B, thr = W.cfg4_screened()
    got = ts.screened_spmm(A.cuda(), diag.cuda(), B.cuda(), threshold=thr).cpu()
    rows = np.r_[0:128, 1000:1040, 2048:2176, 3968:4096]
    _check(A, diag, B, thr, got, rows=rows)
    # every row: (A*mask) @ B and its |.| scale in float64 on the CPU, the
    # mask from the oracle's rule
    Am = A.double() * torch.from_numpy(ref.screened_mask(diag.numpy(), thr))
    exact = Am @ B.double()
    scale = Am.abs() @ B.double().abs()
    assert ((got.double() - exact).abs() / scale.clamp_min(1e-30)).max().item() <= TOL
    del Am, exact, scale
    # linearity at full size: C @ 1 = (A*mask) @ (B @ 1)
    ones = torch.ones(B.shape[1], 1, dtype=torch.float64)
    lhs = got.double() @ ones
    rhs = ts.screened_spmm(A.cuda(), diag.cuda(), (B.double() @ ones).float().cuda(), threshold=thr).cpu().double()
    mask = torch.from_numpy(ref.screened_mask(diag.numpy(), thr))
    sc = (A.abs().double() * mask) @ (B.abs().double() @ ones)
    assert ((lhs - rhs).abs() / sc).max().item() <= TOL


# ------------------------------------------------------------------ backward


def _check_backward(A, diag, B, thr, G, dA, dB, tol, rows=None):
    """dA, dB against ref.screened_spmm_backward with the |.| error scale;
    `rows` restricts the dA check and the dB check to those rows."""
    An, Bn, Gn = (t.double().cpu().numpy() for t in (A, B, G))
    dn = diag.cpu().numpy()
    if rows is None:
        eA, eB = ref.screened_spmm_backward(An, dn, Bn, thr, Gn)
        sA, sB = ref.screened_spmm_backward(An, dn, Bn, thr, Gn, absolute=True)
    else:
        mask = ref.screened_mask(dn, thr)
        eA = np.where(mask[rows], Gn[rows] @ Bn.T, 0.0)
        sA = np.where(mask[rows], np.abs(Gn[rows]) @ np.abs(Bn).T, 0.0)
        eB = np.where(mask[:, rows], An[:, rows], 0.0).T @ Gn
        sB = np.where(mask[:, rows], np.abs(An[:, rows]), 0.0).T @ np.abs(Gn)
    if dA is not None:
        gA = dA.double().cpu().numpy()
        gA = gA if rows is None else gA[rows]
        assert ref.scaled_error(gA, eA, np.maximum(sA, 1e-300)) <= tol
        # masked pairs are exact zeros
        assert (gA[sA == 0] == 0).all()
    if dB is not None:
        gB = dB.double().cpu().numpy()
        gB = gB if rows is None else gB[rows]
        assert ref.scaled_error(gB, eB, np.maximum(sB, 1e-300)) <= tol


@pytest.mark.parametrize("n,N,thr", [
    (200, 70, 1e-6),      # partial tiles on both sides, some tile pairs skipped
    (384, 128, 1e-3),     # whole tiles
    (257, 1, 1e-9),       # one column
    (128, 300, 0.0),      # nothing masked
    (150, 20, 1e30),      # everything masked: exact zeros
])
def test_backward_f32_vs_oracle(hip_backend, n, N, thr):
    g = torch.Generator().manual_seed(n + N)
    diag = torch.pow(10.0, torch.empty(n).uniform_(-8.0, 0.0, generator=g))
    diag[: n // 3] *= 1e-6                               # rows whose tiles drop out
    A = torch.randn(n, n, generator=g)
    B = torch.randn(n, N, generator=g)
    G = torch.randn(n, N, generator=g)
    Ad, Bd = A.cuda().requires_grad_(True), B.cuda().requires_grad_(True)
    out = ts.screened_spmm(Ad, diag.cuda(), Bd, threshold=thr)
    out.backward(G.cuda())
    assert Ad.grad.dtype == torch.float32 and Bd.grad.shape == B.shape
    _check_backward(A, diag, B, thr, G, Ad.grad, Bd.grad, TOL)


def test_backward_one_input_grad(hip_backend):
    """Only A (then only B) requires grad: the other product is not run."""
    g = torch.Generator().manual_seed(4)
    n, N, thr = 160, 33, 1e-5
    diag = torch.pow(10.0, torch.empty(n).uniform_(-8.0, 0.0, generator=g))
    A, B, G = torch.randn(n, n, generator=g), torch.randn(n, N, generator=g), torch.randn(n, N, generator=g)
    Ad = A.cuda().requires_grad_(True)
    ts.screened_spmm(Ad, diag.cuda(), B.cuda(), threshold=thr).backward(G.cuda())
    _check_backward(A, diag, B, thr, G, Ad.grad, None, TOL)
    Bd = B.cuda().requires_grad_(True)
    ts.screened_spmm(A.cuda(), diag.cuda(), Bd, threshold=thr).backward(G.cuda())
    _check_backward(A, diag, B, thr, G, None, Bd.grad, TOL)


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-12), (torch.bfloat16, 2e-2)])
def test_backward_f64_and_bf16(hip_backend, dtype, tol):
    """fp64 runs the generic backward kernels (f64 diag too), bf16 the fp32
    MFMA kernels on widened operands with one rounding of the gradients."""
    g = torch.Generator().manual_seed(5)
    n, N, thr = 140, 24, 1e-6
    diag = torch.pow(10.0, torch.empty(n, dtype=torch.float64).uniform_(-8.0, 0.0, generator=g))
    if dtype != torch.float64:
        diag = diag.float()
    A, B, G = (torch.randn(n, k, generator=g, dtype=torch.float64).to(dtype) for k in (n, N, N))
    Ad, Bd = A.cuda().requires_grad_(True), B.cuda().requires_grad_(True)
    ts.screened_spmm(Ad, diag.cuda(), Bd, threshold=thr).backward(G.cuda())
    assert Ad.grad.dtype == dtype and Bd.grad.dtype == dtype
    _check_backward(A, diag, B, thr, G, Ad.grad, Bd.grad, tol)


def test_backward_cfg4_full_size(hip_backend):
    """cfg4 (4096 x 4096, N = 4096): sampled rows of dA and dB against the
    oracle, and at full size dA @ 1 = ((dC B^T) * mask) @ 1 checked through
    the forward kernel: the row sums of dA equal screened_spmm of dC B^T
    with a ones vector (both apply the same mask)."""
    A, diag, B, thr = W.cfg4_screened()
    g = torch.Generator().manual_seed(6)
    G = torch.randn(B.shape, generator=g)
    Ad, Bd = A.cuda().requires_grad_(True), B.cuda().requires_grad_(True)
    ts.screened_spmm(Ad, diag.cuda(), Bd, threshold=thr).backward(G.cuda())
    rows = np.r_[0:64, 2000:2048, 4032:4096]
    _check_backward(A, diag, B, thr, G, Ad.grad, Bd.grad, TOL, rows=rows)
    # full size: dA @ 1 == (X * mask) @ 1 with X = dC B^T, via the forward kernel
    X = (G.cuda().double() @ B.cuda().double().T).float()
    ones = torch.ones(A.shape[0], 1, device="cuda")
    lhs = (Ad.grad.double() @ ones.double()).cpu()
    rhs = ts.screened_spmm(X, diag.cuda(), ones, threshold=thr).double().cpu()
    mask = torch.from_numpy(ref.screened_mask(diag.numpy(), thr)).cuda()
    sc = ((X.abs().double() * mask) @ ones.double()).cpu() + 1e-30
    assert ((lhs - rhs).abs() / sc).max().item() <= 1e-4
    # dB column sums: 1^T dB = 1^T (A * mask)^T dC = ((A * mask) @ 1)^T dC
    am1 = ts.screened_spmm(A.cuda(), diag.cuda(), torch.ones(A.shape[0], 1, device="cuda"), threshold=thr)
    lhs = Bd.grad.double().sum(0).cpu()
    rhs = (am1.double().T @ G.cuda().double()).squeeze(0).cpu()
    scb = (ts.screened_spmm(A.abs().cuda(), diag.cuda(), torch.ones(A.shape[0], 1, device="cuda"),
                            threshold=thr).double().T @ G.abs().cuda().double()).squeeze(0).cpu() + 1e-30
    assert ((lhs - rhs).abs() / scb).max().item() <= 1e-4
