"""Fixed-step solvers over BSR matrices (reference trnsparse/iterative.py).

Only the fixed-iteration-count solvers — the ones whose loop body is a
matvec plus elementwise updates — are part of this build: `richardson_bsr`
(reference iterative.py:256-295) and `chebyshev_bsr` (:200-253) with its
coefficients `chebyshev_coeffs` (:148-197). On the HIP backend, with the
right-hand side on the GPU, each step is one fused pass over A
(`tsp_bsr_spmv`: out = alpha·A·x + beta·u + gamma·v + delta·w), so A is read
once per iteration and the update costs no extra pass; a matrix that fits
the 256 MB last-level cache (MALL) stays resident across the iterations.
Elsewhere the steps run as the reference writes them, with `bsr_spmm` as
the matvec.
"""

from __future__ import annotations

import torch

from .backend import _use_hip
from .formats import BSRMatrix
from .ops import bsr_spmm

_FUSED_DTYPES = (torch.float32, torch.float64, torch.bfloat16)


def chebyshev_coeffs(lam_min: float, lam_max: float, K: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Step coefficients (alpha, beta), float32 of length K, for
    x_{k+1} = x_k + alpha_k r_k + beta_k (x_k - x_{k-1}) (reference
    iterative.py:148-197).

    The recurrence of the Chebyshev iteration in Barrett et al., Templates
    for the Solution of Linear Systems (1994), Algorithm 2.1, in momentum
    form, as the reference applies it: with the centre d and half-width c of
    [lam_min, lam_max], alpha_0 = 1/d, beta_0 = 0 and, from k = 1,
    t = (c alpha_{k-1} / 2)^2, alpha_k = 1 / (d - t / alpha_{k-1}),
    beta_k = alpha_k t / alpha_{k-1}. With that start the residual
    polynomial after K steps is U_K((d - lam)/c) / U_K(d/c) (Chebyshev
    polynomials of the second kind). Computed in float64, returned as
    float32 as the reference returns them.
    """
    c = (lam_max - lam_min) / 2.0
    d = (lam_max + lam_min) / 2.0
    alpha = torch.zeros(K, dtype=torch.float64)
    beta = torch.zeros(K, dtype=torch.float64)
    if K == 0:
        return alpha.float(), beta.float()
    prev = 1.0 / d
    alpha[0] = prev
    for k in range(1, K):
        t = (c * prev / 2.0) ** 2
        a = 1.0 / (d - t / prev)
        alpha[k] = a
        beta[k] = a * t / prev
        prev = a
    return alpha.float(), beta.float()


def _fused(A: BSRMatrix, b: torch.Tensor) -> bool:
    return _use_hip() and b.is_cuda and b.dtype == A.dtype and b.dtype in _FUSED_DTYPES and b.dim() == 1


def _matvec(A: BSRMatrix, x: torch.Tensor) -> torch.Tensor:
    return bsr_spmm(A, x.unsqueeze(1)).squeeze(1)


def _residual(A: BSRMatrix, b: torch.Tensor, x: torch.Tensor, b_norm: float) -> float:
    if _fused(A, b):
        from .hip.dispatch import hip_bsr_matvec_update

        r = hip_bsr_matvec_update(A, x, -1.0, torch.empty_like(x), u=b, beta=1.0)  # r = b - A x
    else:
        r = b - _matvec(A, x)
    return torch.linalg.norm(r).item() / max(b_norm, 1e-15)


def richardson_bsr(A: BSRMatrix, b: torch.Tensor, omega: float, K: int = 100,
                   x0: torch.Tensor | None = None) -> tuple[torch.Tensor, int, float]:
    """K steps of x <- x + omega (b - A x) (reference iterative.py:256-295).

    Returns (x, K, ||b - A x|| / ||b||).
    """
    n = b.shape[0]
    x = x0.clone() if x0 is not None else torch.zeros(n, dtype=b.dtype, device=b.device)
    b_norm = torch.linalg.norm(b).item()
    if _fused(A, b):
        from .hip.dispatch import hip_bsr_matvec_update

        y = torch.empty_like(x)
        for _ in range(K):
            # y = -omega A x + x + omega b
            hip_bsr_matvec_update(A, x, -omega, y, u=x, beta=1.0, v=b, gamma=omega)
            x, y = y, x
    else:
        for _ in range(K):
            r = b - _matvec(A, x)
            x = x + omega * r
    return x, K, _residual(A, b, x, b_norm)


def chebyshev_bsr(A: BSRMatrix, b: torch.Tensor, lam_min: float, lam_max: float, K: int = 50,
                  x0: torch.Tensor | None = None) -> tuple[torch.Tensor, int, float]:
    """K Chebyshev steps for SPD A with spectrum in [lam_min, lam_max]
    (reference iterative.py:200-253). Returns (x, K, ||b - A x|| / ||b||)."""
    n = b.shape[0]
    x = x0.clone() if x0 is not None else torch.zeros(n, dtype=b.dtype, device=b.device)
    b_norm = torch.linalg.norm(b).item()
    alpha, beta = chebyshev_coeffs(lam_min, lam_max, K)
    if _fused(A, b):
        from .hip.dispatch import hip_bsr_matvec_update

        xp = x.clone()
        for k in range(K):
            a, be = alpha[k].item(), beta[k].item()
            # x_{k+1} = -a A x + (1 + be) x + a b - be x_{k-1}, written over x_{k-1}
            hip_bsr_matvec_update(A, x, -a, xp, u=x, beta=1.0 + be, v=b, gamma=a, w=xp if k > 0 else None,
                                  delta=-be)
            x, xp = xp, x
    else:
        x_prev = x.clone()
        for k in range(K):
            r = b - _matvec(A, x)
            x_new = x + alpha[k].item() * r
            if k > 0:
                x_new = x_new + beta[k].item() * (x - x_prev)
            x_prev = x
            x = x_new
    return x, K, _residual(A, b, x, b_norm)
