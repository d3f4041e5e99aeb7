"""Sparse operations: the public API of the compute path.

Signatures, defaults, error behaviour and results follow the reference
(trnsparse/ops.py). Each hot op checks `_use_hip()` exactly where the
reference checked `_use_nki()` (ops.py:67-73, 204-209, 255-260, 500-505,
535-540, 618-623) and then calls the HIP dispatch layer
(`trnsparse_amd.hip.dispatch`), which drives the gfx950 kernels through
the C ABI. With the "pytorch" backend selected the in-file torch code runs:
it restates the reference's torch path operation for operation (same loop
order and accumulation dtype), so both backends answer the same question.

`spmv` also crosses the seam here; in the reference it is always
`torch.sparse_csr_tensor @ x` (ops.py:30-48).
"""

from __future__ import annotations

import math

import torch

from .backend import _use_hip
from .formats import BSRMatrix, COOMatrix, CSRMatrix


def _as_torch_csr(A: CSRMatrix) -> torch.Tensor:
    """torch.sparse_csr_tensor view of a CSRMatrix (reference ops.py:25-27)."""
    return torch.sparse_csr_tensor(A.row_ptrs, A.col_indices, A.values, size=A.shape)


# --------------------------------------------------------------------- CSR


def spmv(
    A: CSRMatrix,
    x: torch.Tensor,
    alpha: float = 1.0,
    y: torch.Tensor | None = None,
    beta: float = 0.0,
) -> torch.Tensor:
    """y = alpha * A @ x + beta * y  (reference ops.py:30-48).

    alpha scales the product after the row sums; `y` is read only when it is
    given and beta != 0, and is never modified (a new tensor is returned).
    """
    m, n = A.shape
    assert x.shape[0] == n, f"Dimension mismatch: A is {A.shape}, x is {x.shape}"
    if _use_hip():
        from .hip.dispatch import hip_spmv

        return hip_spmv(A, x, alpha, y, beta)
    result = alpha * (_as_torch_csr(A) @ x)
    if y is not None and beta != 0.0:
        result = result + beta * y
    return result


def spmm(
    A: CSRMatrix,
    B: torch.Tensor,
    alpha: float = 1.0,
    C: torch.Tensor | None = None,
    beta: float = 0.0,
) -> torch.Tensor:
    """C = alpha * A @ B + beta * C  (reference ops.py:51-78)."""
    m, n = A.shape
    assert B.shape[0] == n, f"Dimension mismatch: A is {A.shape}, B is {B.shape}"
    if _use_hip():
        from .hip.dispatch import hip_spmm

        return hip_spmm(A, B, alpha, C, beta)
    result = alpha * (_as_torch_csr(A) @ B)
    if C is not None and beta != 0.0:
        result = result + beta * C
    return result


def spmv_symmetric(A: CSRMatrix, x: torch.Tensor, alpha: float = 1.0, uplo: str = "upper") -> torch.Tensor:
    """Symmetric SpMV from one stored triangle (reference ops.py:81-104):
    alpha * (A @ x + S^T @ x) with S the entries off the diagonal (duplicates
    summed); `uplo` is accepted and unused, as there. On the HIP backend with
    A on the GPU: S^T is built once on the device (transpose by a stable sort
    of (col, row), cached on A) and the two products run as CSR SpMVs, the
    second accumulating into the first."""
    m, n = A.shape
    assert m == n, "Matrix must be square for symmetric SpMV"
    if _use_hip() and A.values.is_cuda:
        from .hip.dispatch import hip_spmv

        St = _strict_transpose(A)
        y = hip_spmv(A, x, alpha)
        return hip_spmv(St, x, alpha, y, 1.0)
    counts = A.row_ptrs[1:] - A.row_ptrs[:-1]
    rows = torch.repeat_interleave(torch.arange(m, device=counts.device), counts)
    cols = A.col_indices
    strict = rows != cols
    strict_t = torch.sparse_coo_tensor(
        torch.stack([rows[strict], cols[strict]]), A.values[strict], size=A.shape
    ).coalesce()
    return alpha * (_as_torch_csr(A) @ x + strict_t.t() @ x)


def _strict_transpose(A: CSRMatrix) -> CSRMatrix:
    """CSR of the transpose of A's off-diagonal entries (duplicates summed),
    on A's device; cached on A keyed by the identity and version of its
    tensors."""
    key = tuple((t.data_ptr(), t._version) for t in (A.values, A.col_indices, A.row_ptrs))
    hit = getattr(A, "_strict_t", None)
    if hit is not None and hit[0] == key:
        return hit[1]
    from .hip import formats as hf

    coo = A.to_coo()
    keep = coo.row_indices != coo.col_indices
    vals, cols, rp = hf.coo_sum_to_csr(coo.values[keep], coo.col_indices[keep], coo.row_indices[keep],
                                       (A.shape[1], A.shape[0]))
    St = CSRMatrix(values=vals, col_indices=cols, row_ptrs=rp, shape=(A.shape[1], A.shape[0]))
    try:
        # the source tensors ride along, so a new tensor cannot take a freed
        # one's address (and key) while this entry lives
        A._strict_t = (key, St, (A.values, A.col_indices, A.row_ptrs))
    except AttributeError:
        pass
    return St


def sparse_add(A: CSRMatrix, B: CSRMatrix, alpha: float = 1.0, beta: float = 1.0) -> CSRMatrix:
    """C = alpha*A + beta*B on the union pattern (reference ops.py:107-132).

    Entries sorted by (row, col), one per distinct coordinate with its
    duplicates summed (explicit zeros kept). On the HIP backend with A and
    B on the GPU the coalesce runs on the device (`tsp_csr_sum`: each row's
    entries of A then B, stably sorted by column, runs summed); the values
    are scaled by torch first, as in the reference."""
    assert A.shape == B.shape, f"Shape mismatch: {A.shape} vs {B.shape}"
    if _use_hip() and A.values.is_cuda and B.values.is_cuda and A.values.dtype == B.values.dtype:
        from .hip import formats as hf

        if A.values.dtype in hf.DEVICE_DTYPES:
            # (x * 1.0 is x bit for bit, so a unit factor is not applied)
            av = A.values if alpha == 1.0 else alpha * A.values
            bv = B.values if beta == 1.0 else beta * B.values
            vals, cols, rp = hf.csr_sum(av, A.col_indices, A.row_ptrs, bv, B.col_indices, B.row_ptrs, A.shape)
            return CSRMatrix(values=vals, col_indices=cols, row_ptrs=rp, shape=A.shape)
    ca, cb = A.to_coo(), B.to_coo()
    idx = torch.stack(
        [torch.cat([ca.row_indices, cb.row_indices]), torch.cat([ca.col_indices, cb.col_indices])]
    )
    vals = torch.cat([alpha * ca.values, beta * cb.values])
    csr = torch.sparse_coo_tensor(idx, vals, size=A.shape).coalesce().to_sparse_csr()
    return CSRMatrix(values=csr.values(), col_indices=csr.col_indices(), row_ptrs=csr.crow_indices(), shape=A.shape)


def sparse_scale(A: CSRMatrix, alpha: float) -> CSRMatrix:
    """B = alpha * A (reference ops.py:135-142)."""
    return CSRMatrix(
        values=alpha * A.values,
        col_indices=A.col_indices.clone(),
        row_ptrs=A.row_ptrs.clone(),
        shape=A.shape,
    )


def sparse_transpose(A: CSRMatrix) -> CSRMatrix:
    """CSR of A^T (reference ops.py:145-154). On the HIP backend with A on
    the GPU: a stable device sort of the entries by column with the rows
    carried along (`tsp_csr_transpose`), the same order as the reference's
    sort by (col, row)."""
    if _use_hip() and A.values.is_cuda:
        from .hip import formats as hf

        if A.values.dtype in hf.DEVICE_DTYPES:
            vals, cols, rp = hf.csr_transpose(A.values, A.col_indices, A.row_ptrs, A.shape)
            return CSRMatrix(values=vals, col_indices=cols, row_ptrs=rp, shape=(A.shape[1], A.shape[0]))
    coo = A.to_coo()
    return COOMatrix(
        values=coo.values, row_indices=coo.col_indices, col_indices=coo.row_indices, shape=(A.shape[1], A.shape[0])
    ).to_csr()


def nnz_per_row(A: CSRMatrix) -> torch.Tensor:
    """Stored entries per row (reference ops.py:157-159)."""
    return A.row_ptrs[1:] - A.row_ptrs[:-1]


# --------------------------------------------------------------------- BSR


def _bsr_spmm_pytorch(A: BSRMatrix, B: torch.Tensor, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Torch semantics of bsr_spmm (reference ops.py:162-192).

    For each block row i and stored block idx (indptr order), with column
    block j: out[i*b:(i+1)*b] += blocks[idx] @ B[j*b:(j+1)*b]. `out` has
    A's dtype unless `out_dtype` asks otherwise, in which case the block
    products are formed in `out_dtype` from upcast operands.
    """
    m, n = A.shape
    _, k = B.shape
    b = A.block_size
    m_pad = ((m + b - 1) // b) * b
    n_pad = ((n + b - 1) // b) * b
    mb = m_pad // b
    if B.shape[0] != n:
        raise AssertionError(f"Dimension mismatch: A is {A.shape}, B is {B.shape}")
    if n_pad != n:
        B_p = torch.zeros(n_pad, k, dtype=B.dtype, device=B.device)
        B_p[:n, :] = B
        B = B_p
    odt = out_dtype or A.dtype
    blocks = A.blocks if odt == A.dtype else A.blocks.to(odt)
    if odt != B.dtype and out_dtype is not None:
        B = B.to(odt)
    out = torch.zeros(m_pad, k, dtype=odt, device=B.device)
    ptrs = A.block_row_ptrs.tolist()
    cols = A.block_col_indices.tolist()
    for i in range(mb):
        for idx in range(ptrs[i], ptrs[i + 1]):
            j = cols[idx]
            out[i * b : (i + 1) * b] += blocks[idx] @ B[j * b : (j + 1) * b]
    return out[:m]


def bsr_spmm(A: BSRMatrix, B: torch.Tensor, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Block-sparse x dense: C = A @ B  (reference ops.py:195-210).

    `out_dtype` (an addition; default A.dtype as in the reference) lets bf16
    operands produce an fp32 result, accumulated in fp32.
    """
    if B.shape[0] != A.shape[1]:
        raise AssertionError(f"Dimension mismatch: A is {A.shape}, B is {B.shape}")
    if _use_hip():
        from .hip.dispatch import hip_bsr_spmm

        return hip_bsr_spmm(A, B, out_dtype=out_dtype)
    return _bsr_spmm_pytorch(A, B, out_dtype=out_dtype)


# ---------------------------------------------------------------- screened


def screened_mask(diag_integrals: torch.Tensor, threshold: float) -> torch.Tensor:
    """mask[i, j] = Q_i*Q_j > sqrt(threshold), Q = sqrt(|diag|) (reference ops.py:273-276).

    The product and the compare run in diag's dtype: torch casts the Python
    float sqrt(threshold) to that dtype before comparing.
    """
    Q = torch.sqrt(torch.abs(diag_integrals))
    return (Q.unsqueeze(-1) * Q.unsqueeze(0)) > math.sqrt(threshold)


def screened_spmm(
    A: torch.Tensor,
    diag_integrals: torch.Tensor,
    B: torch.Tensor,
    threshold: float,
) -> torch.Tensor:
    """Schwarz-screened dense matmul C = (A * mask) @ B  (reference ops.py:213-277).

    mask[i, j] = sqrt(|d_i|) * sqrt(|d_j|) > sqrt(threshold). On the HIP
    backend the mask is applied while A tiles are staged (no mask tensor)
    and 128x128 tiles whose bound cannot pass are skipped.
    """
    assert diag_integrals.dim() == 1, f"diag_integrals must be 1-D; got shape {diag_integrals.shape}"
    M, K = A.shape
    assert diag_integrals.shape[0] == M == K, (
        "screened_spmm requires square A with diag_integrals of matching length; "
        f"got A shape {A.shape}, diag_integrals shape {diag_integrals.shape}"
    )
    if _use_hip():
        from .hip.dispatch import hip_screened_spmm

        return hip_screened_spmm(A, diag_integrals, B, threshold)
    mask = screened_mask(diag_integrals, threshold)
    return (A * mask.to(A.dtype)) @ B


# --------------------------------------------------------------- attention


def _block_sparse_attn_pytorch(Q, K, V, mask_bsr, scale: float, return_stats: bool = False):
    """Two-pass block-sparse attention, torch semantics (reference ops.py:280-357).

    Pass 1 stores per stored block the row max and stable exp-sum of
    score = (Q_m @ K_j^T) * scale; they are reduced to row_max / row_denom
    (row_denom clamped at 1e-12; empty block rows get row_max 0 and zero
    output); pass 2 accumulates exp(score - row_max) / row_denom @ V_j.
    Stats and output are in Q's dtype, as in the reference.
    """
    seq_len, head_dim = Q.shape
    b = mask_bsr.block_size
    M_tiles = seq_len // b
    ptrs = mask_bsr.block_row_ptrs.tolist()
    cols = mask_bsr.block_col_indices.tolist()
    n_blocks = len(cols)
    dev = Q.device

    tile_max = torch.full((n_blocks, b), float("-inf"), dtype=Q.dtype, device=dev)
    tile_sumexp = torch.zeros((n_blocks, b), dtype=Q.dtype, device=dev)
    for m in range(M_tiles):
        q_block = Q[m * b : (m + 1) * b]
        for idx in range(ptrs[m], ptrs[m + 1]):
            c = cols[idx]
            score = (q_block @ K[c * b : (c + 1) * b].T) * scale
            tile_max[idx] = score.max(dim=1).values
            tile_sumexp[idx] = torch.exp(score - tile_max[idx].unsqueeze(1)).sum(dim=1)

    row_max = torch.full((seq_len,), float("-inf"), dtype=Q.dtype, device=dev)
    row_denom = torch.zeros(seq_len, dtype=Q.dtype, device=dev)
    for m in range(M_tiles):
        s, e = ptrs[m], ptrs[m + 1]
        if s == e:
            row_max[m * b : (m + 1) * b] = 0.0
            continue
        row_max[m * b : (m + 1) * b] = tile_max[s:e].max(dim=0).values
        rm = row_max[m * b : (m + 1) * b]
        for idx in range(s, e):
            row_denom[m * b : (m + 1) * b] += tile_sumexp[idx] * torch.exp(tile_max[idx] - rm)
    row_denom = row_denom.clamp(min=1e-12)

    out = torch.zeros(seq_len, head_dim, dtype=Q.dtype, device=dev)
    for m in range(M_tiles):
        s, e = ptrs[m], ptrs[m + 1]
        if s == e:
            continue
        q_block = Q[m * b : (m + 1) * b]
        rm = row_max[m * b : (m + 1) * b].unsqueeze(1)
        rd = row_denom[m * b : (m + 1) * b].unsqueeze(1)
        for idx in range(s, e):
            c = cols[idx]
            score = (q_block @ K[c * b : (c + 1) * b].T) * scale
            out[m * b : (m + 1) * b] += (torch.exp(score - rm) / rd) @ V[c * b : (c + 1) * b]

    if return_stats:
        return out, row_max[: M_tiles * b].view(M_tiles, b), row_denom[: M_tiles * b].view(M_tiles, b)
    return out


def _block_sparse_attn_backward(Q, K, V, O, dO, mask_bsr, scale, row_max=None, row_denom=None):
    """Tiled softmax-attention backward (reference ops.py:360-473).

    D = rowsum(dO * O); per stored block P = exp(score - row_max)/row_denom,
    dS = P * (dO @ V_j^T - D); dQ += dS @ K_j * scale, dK_j += dS^T @ Q *
    scale, dV_j += P^T @ dO. Stats are recomputed when not supplied.
    """
    seq_len, head_dim = Q.shape
    b = mask_bsr.block_size
    M_tiles = seq_len // b
    ptrs = mask_bsr.block_row_ptrs.tolist()
    cols = mask_bsr.block_col_indices.tolist()
    dev = Q.device
    D = (dO * O).sum(dim=-1)

    if row_max is not None and row_denom is not None:
        rmax = row_max.reshape(-1)
        rden = row_denom.reshape(-1)
    else:
        rmax = torch.full((seq_len,), float("-inf"), dtype=Q.dtype, device=dev)
        rden = torch.zeros(seq_len, dtype=Q.dtype, device=dev)
        for m in range(M_tiles):
            s, e = ptrs[m], ptrs[m + 1]
            if s == e:
                rmax[m * b : (m + 1) * b] = 0.0
                continue
            q_block = Q[m * b : (m + 1) * b]
            rm = rmax[m * b : (m + 1) * b]
            for idx in range(s, e):
                c = cols[idx]
                score = (q_block @ K[c * b : (c + 1) * b].T) * scale
                rm = torch.maximum(rm, score.max(dim=1).values)
            rmax[m * b : (m + 1) * b] = rm
        for m in range(M_tiles):
            s, e = ptrs[m], ptrs[m + 1]
            if s == e:
                continue
            q_block = Q[m * b : (m + 1) * b]
            rm = rmax[m * b : (m + 1) * b]
            for idx in range(s, e):
                c = cols[idx]
                score = (q_block @ K[c * b : (c + 1) * b].T) * scale
                rden[m * b : (m + 1) * b] += torch.exp(score - rm.unsqueeze(1)).sum(dim=1)
        rden = rden.clamp(min=1e-12)

    dQ = torch.zeros_like(Q)
    dK = torch.zeros_like(K)
    dV = torch.zeros_like(V)
    for m in range(M_tiles):
        s, e = ptrs[m], ptrs[m + 1]
        if s == e:
            continue
        q_block = Q[m * b : (m + 1) * b]
        do_block = dO[m * b : (m + 1) * b]
        d_block = D[m * b : (m + 1) * b]
        rm = rmax[m * b : (m + 1) * b].unsqueeze(1)
        rd = rden[m * b : (m + 1) * b].unsqueeze(1)
        for idx in range(s, e):
            c = cols[idx]
            k_block = K[c * b : (c + 1) * b]
            v_block = V[c * b : (c + 1) * b]
            score = (q_block @ k_block.T) * scale
            P = torch.exp(score - rm) / rd
            dS = P * (do_block @ v_block.T - d_block.unsqueeze(1))
            dQ[m * b : (m + 1) * b] += dS @ k_block * scale
            dK[c * b : (c + 1) * b] += dS.T @ q_block * scale
            dV[c * b : (c + 1) * b] += P.T @ do_block
    return dQ, dK, dV


class _AttnTiledFunction(torch.autograd.Function):
    """Autograd wrapper of tiled attention (reference ops.py:476-546).

    Forward runs the HIP kernel (or the torch two-pass spec) and saves
    Q, K, V, O and the row stats; backward runs the HIP backward kernels (or
    the tiled torch backward on the "pytorch" backend).
    Q/K/V are (seq, d) or batched (..., seq, d) sharing one mask. The mask
    itself is passed (not its tensors, as the reference's pattern stand-in
    at ops.py:488-498 does): the device copies of its pattern and the row
    order are cached on it, so repeated calls copy nothing to the device and
    a HIP graph can capture a forward + backward step.
    """

    @staticmethod
    def forward(ctx, Q, K, V, mask_bsr, scale):
        handle = mask_bsr
        if _use_hip():
            from .hip.dispatch import hip_block_sparse_attention

            out, row_max, row_denom = hip_block_sparse_attention(Q, K, V, handle, scale, return_stats=True)
        else:
            out, row_max, row_denom = _attn_pytorch_batched(Q, K, V, handle, scale, return_stats=True)
        ctx.save_for_backward(Q, K, V, out, row_max, row_denom)
        ctx.handle = handle
        ctx.scale = scale
        return out

    @staticmethod
    def backward(ctx, dO):
        Q, K, V, O, row_max, row_denom = ctx.saved_tensors
        if _use_hip():
            from .hip.dispatch import hip_block_sparse_attention_backward

            dQ, dK, dV = hip_block_sparse_attention_backward(
                Q, K, V, O, dO.contiguous(), ctx.handle, ctx.scale, row_max, row_denom
            )
            return dQ, dK, dV, None, None
        lead = Q.shape[:-2]
        S, D = Q.shape[-2:]
        q, k, v, o, do = (t.reshape(math.prod(lead), S, D) for t in (Q, K, V, O, dO))
        rm = row_max.reshape(q.shape[0], -1).to(Q.dtype)
        rd = row_denom.reshape(q.shape[0], -1).to(Q.dtype)
        grads = [
            _block_sparse_attn_backward(q[h], k[h], v[h], o[h], do[h], ctx.handle, ctx.scale, rm[h], rd[h])
            for h in range(q.shape[0])
        ]
        dQ, dK, dV = (torch.stack([g[i] for g in grads]).reshape(*lead, S, D) for i in range(3))
        return dQ, dK, dV, None, None


def _attn_pytorch_batched(Q, K, V, mask_bsr, scale, return_stats=False):
    if Q.dim() == 2:
        return _block_sparse_attn_pytorch(Q, K, V, mask_bsr, scale, return_stats=return_stats)
    lead = Q.shape[:-2]
    S, D = Q.shape[-2:]
    q, k, v = (t.reshape(math.prod(lead), S, D) for t in (Q, K, V))
    res = [_block_sparse_attn_pytorch(q[h], k[h], v[h], mask_bsr, scale, return_stats=return_stats) for h in range(q.shape[0])]
    if not return_stats:
        return torch.stack(res).reshape(*lead, S, D)
    out = torch.stack([r[0] for r in res]).reshape(*lead, S, D)
    rmax = torch.stack([r[1] for r in res]).reshape(*lead, *res[0][1].shape)
    rden = torch.stack([r[2] for r in res]).reshape(*lead, *res[0][2].shape)
    return out, rmax, rden


def block_sparse_attention_tiled(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    mask_bsr: BSRMatrix,
    scale: float | None = None,
) -> torch.Tensor:
    """Block-sparse softmax attention over the stored blocks of `mask_bsr`
    (reference ops.py:549-625).

    Q, K, V: (seq_len, head_dim), or (..., seq_len, head_dim) with leading
    batch/head dims sharing one mask (an addition; each head is the 2-D
    op). Only the mask's pattern is used. `scale` defaults to
    head_dim**-0.5. Rows of an empty block row produce zeros. When any input
    requires grad the call goes through `_AttnTiledFunction`.
    """
    head_dim = Q.shape[-1]
    if scale is None:
        scale = head_dim**-0.5
    if torch.is_grad_enabled() and (Q.requires_grad or K.requires_grad or V.requires_grad):
        return _AttnTiledFunction.apply(Q, K, V, mask_bsr, scale)
    if _use_hip():
        from .hip.dispatch import hip_block_sparse_attention

        return hip_block_sparse_attention(Q, K, V, mask_bsr, scale)
    return _attn_pytorch_batched(Q, K, V, mask_bsr, scale)
