"""The reference's CPU torch path restated op for op — CPU baseline only.

Test infrastructure: `bench.py` times these on the GPU box's host cores to
report `cpu_baseline`; they are never part of the product path. Each
follows the reference's torch code for the op (loop order, dtype of the
accumulators, the third-party call it makes):

- bsr_spmm:  trnsparse/ops.py:162-192 — Python loop over block rows and
             stored blocks, one torch (MKL) matmul per block, `+=` into an
             output of A's dtype.
- spmv:      trnsparse/ops.py:30-48 — torch.sparse_csr_tensor @ x.
- screened:  trnsparse/ops.py:262-277 — materialised mask, A*mask, dense @.
- attention: trnsparse/ops.py:280-357 — pass 1 tile stats, row reduction,
             pass 2 weighted accumulation, one head at a time.
- attention_backward: trnsparse/ops.py:360-473 — D = rowsum(dO * O), then
             per stored block P, dS and the three `+=` products, one head.
- bsr_from_dense: trnsparse/formats.py:183-221 — pad, block-grid view
             copy, amax of |v|, nonzero, boolean gather.
"""

from __future__ import annotations

import math
import os
import time

import torch


def threads() -> int:
    """Threads the CPU baselines run on: the CPUs this process may use (its
    affinity mask, else the machine's count), capped by OMP_NUM_THREADS."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        n = min(n, int(env))
    return max(1, n)


def bsr_spmm(blocks, col_idx, row_ptrs, shape, b, B):
    m, n = shape
    k = B.shape[1]
    mb = (m + b - 1) // b
    ptrs = row_ptrs.tolist()
    cols = col_idx.tolist()
    out = torch.zeros(mb * b, k, dtype=blocks.dtype)
    for i in range(mb):
        for idx in range(ptrs[i], ptrs[i + 1]):
            j = cols[idx]
            out[i * b : (i + 1) * b] += blocks[idx] @ B[j * b : (j + 1) * b]
    return out[:m]


def spmv(values, col_idx, row_ptrs, shape, x, alpha=1.0):
    A = torch.sparse_csr_tensor(row_ptrs, col_idx, values, size=shape)
    return alpha * (A @ x)


def screened_spmm(A, diag, B, threshold):
    Q = torch.sqrt(torch.abs(diag))
    mask = (Q.unsqueeze(-1) * Q.unsqueeze(0)) > math.sqrt(threshold)
    return (A * mask.to(A.dtype)) @ B


def attention_head(Q, K, V, row_ptrs, col_idx, b, scale):
    seq, d = Q.shape
    Mt = seq // b
    ptrs = row_ptrs.tolist()
    cols = col_idx.tolist()
    nb = len(cols)
    tmax = torch.full((nb, b), float("-inf"), dtype=Q.dtype)
    tsum = torch.zeros((nb, b), dtype=Q.dtype)
    for m in range(Mt):
        qb = Q[m * b : (m + 1) * b]
        for idx in range(ptrs[m], ptrs[m + 1]):
            c = cols[idx]
            s = (qb @ K[c * b : (c + 1) * b].T) * scale
            tmax[idx] = s.max(dim=1).values
            tsum[idx] = torch.exp(s - tmax[idx].unsqueeze(1)).sum(dim=1)
    rmax = torch.zeros(seq, dtype=Q.dtype)
    rden = torch.zeros(seq, dtype=Q.dtype)
    for m in range(Mt):
        s0, e0 = ptrs[m], ptrs[m + 1]
        if s0 == e0:
            continue
        rmax[m * b : (m + 1) * b] = tmax[s0:e0].max(dim=0).values
        for idx in range(s0, e0):
            rden[m * b : (m + 1) * b] += tsum[idx] * torch.exp(tmax[idx] - rmax[m * b : (m + 1) * b])
    rden = rden.clamp(min=1e-12)
    out = torch.zeros(seq, d, dtype=Q.dtype)
    for m in range(Mt):
        qb = Q[m * b : (m + 1) * b]
        rm = rmax[m * b : (m + 1) * b].unsqueeze(1)
        rd = rden[m * b : (m + 1) * b].unsqueeze(1)
        for idx in range(ptrs[m], ptrs[m + 1]):
            c = cols[idx]
            s = (qb @ K[c * b : (c + 1) * b].T) * scale
            out[m * b : (m + 1) * b] += (torch.exp(s - rm) / rd) @ V[c * b : (c + 1) * b]
    return out


def attention_backward_head(Q, K, V, O, dO, row_ptrs, col_idx, b, scale, rmax, rden):
    seq, d = Q.shape
    Mt = seq // b
    ptrs = row_ptrs.tolist()
    cols = col_idx.tolist()
    D = (dO * O).sum(dim=-1)
    dQ, dK, dV = torch.zeros_like(Q), torch.zeros_like(K), torch.zeros_like(V)
    for m in range(Mt):
        s0, e0 = ptrs[m], ptrs[m + 1]
        if s0 == e0:
            continue
        qs = slice(m * b, (m + 1) * b)
        rm, rd, dd = rmax[qs].unsqueeze(1), rden[qs].unsqueeze(1), D[qs].unsqueeze(1)
        for idx in range(s0, e0):
            c = cols[idx]
            ks = slice(c * b, (c + 1) * b)
            P = torch.exp((Q[qs] @ K[ks].T) * scale - rm) / rd
            dS = P * (dO[qs] @ V[ks].T - dd)
            dQ[qs] += dS @ K[ks] * scale
            dK[ks] += dS.T @ Q[qs] * scale
            dV[ks] += P.T @ dO[qs]
    return dQ, dK, dV


def bsr_from_dense(A, b, threshold=0.0):
    m, n = A.shape
    mp, np_ = -(-m // b) * b, -(-n // b) * b
    if (mp, np_) != (m, n):
        P = torch.zeros(mp, np_, dtype=A.dtype)
        P[:m, :n] = A
        A = P
    mb, nbc = mp // b, np_ // b
    grid = A.reshape(mb, b, nbc, b).permute(0, 2, 1, 3).contiguous()
    keep = grid.abs().amax(dim=(-2, -1)) > threshold
    ptrs = torch.zeros(mb + 1, dtype=torch.long)
    ptrs[1:] = keep.sum(dim=1).cumsum(dim=0)
    cols = keep.nonzero(as_tuple=False)[:, 1].to(torch.long)
    return grid[keep].contiguous(), cols, ptrs


def time_call(fn, reps: int = 5, budget_s: float = 30.0) -> tuple[float, int]:
    """(median wall time in s, number of timed reps) of `fn()` after one
    untimed warmup call; the rep count is cut so the reps fit `budget_s`."""
    t0 = time.perf_counter()
    fn()
    first = time.perf_counter() - t0
    reps = max(1, min(reps, int(budget_s / max(first, 1e-6))))
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2], reps
