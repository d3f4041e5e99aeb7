"""Deterministic synthetic inputs for the five benchmark configurations.

Shared by `bench.py`, the tests and the smoke check so that every leg sees
the same seeded data. Generators run on the CPU (numpy / torch CPU RNG), so
the data do not depend on the GPU; callers move them to the device.

  cfg1  bsr_spmm plumbing: 1024^2, 128-blocks (8x8 grid), off-diagonal
        blocks present with p=0.25, diagonal always; B 1024x256. Seed 0.
  cfg2  CSR SpMV: 1,048,576^2, row lengths Poisson(16) clipped to [1,64]
        (or Zipf(1.5) clipped to [1,4096]), columns uniform without
        replacement and sorted per row, values and x N(0,1). Seed 1.
  cfg3  bsr_spmm at scale: 16384^2 in 128-blocks, band |i-j|<=3 plus
        uniform off-band blocks to 10% block density, B 16384x512. Seed 2.
  cfg4  screened_spmm: n=4096, diag log-uniform in [1e-14, 1],
        |A_ij| = exp(-|i-j|/256)*U(0.5,1) with random sign, B N(0,1),
        threshold 1e-20 (mask Q_iQ_j > 1e-10). Seed 3.
  cfg5  block-sparse attention: 32 heads x 8192 x 128 bf16, 128-blocks;
        block row m attends to blocks max(0,m-3)..m and {0, 1}. Seed 4.
"""

from __future__ import annotations

import numpy as np
import torch

from .formats import BSRMatrix, CSRMatrix

# --------------------------------------------------------------- helpers


def bsr_from_block_mask(block_mask: torch.Tensor, block_size: int, blocks: torch.Tensor | None = None,
                        dtype: torch.dtype = torch.float32) -> BSRMatrix:
    """BSRMatrix with the pattern of a boolean (mb, nbc) block mask.

    The structure is what `BSRMatrix.from_dense` produces for a dense matrix
    whose nonzero blocks are exactly the True entries: row-major block order,
    int64 `block_row_ptrs` (CPU) and `block_col_indices`. `blocks` defaults
    to all-ones blocks (an attention mask's values are never read).
    """
    block_mask = block_mask.to(torch.bool).cpu()
    mb, nbc = block_mask.shape
    row_ptrs = torch.zeros(mb + 1, dtype=torch.long)
    row_ptrs[1:] = block_mask.sum(dim=1).cumsum(dim=0)
    col_idx = block_mask.nonzero(as_tuple=False)[:, 1].to(torch.long)
    nnzb = col_idx.numel()
    if blocks is None:
        blocks = torch.ones(nnzb, block_size, block_size, dtype=dtype)
    assert blocks.shape == (nnzb, block_size, block_size)
    return BSRMatrix(blocks=blocks, block_col_indices=col_idx, block_row_ptrs=row_ptrs,
                     shape=(mb * block_size, nbc * block_size), block_size=block_size)


# ------------------------------------------------------------------ cfg1


def cfg1_bsr_plumbing():
    """(A_bsr, B, A_dense): seed 0; mask = rand(8,8) < 0.25 | eye; blocks
    randn(128,128) in row-major block order; B randn(1024, 256)."""
    torch.manual_seed(0)
    nb, b = 8, 128
    mask = (torch.rand(nb, nb) < 0.25) | torch.eye(nb, dtype=torch.bool)
    A = torch.zeros(nb * b, nb * b)
    for i in range(nb):
        for j in range(nb):
            if mask[i, j]:
                A[i * b : (i + 1) * b, j * b : (j + 1) * b] = torch.randn(b, b)
    B = torch.randn(nb * b, 256)
    return BSRMatrix.from_dense(A, block_size=b), B, A


# ------------------------------------------------------------------ cfg2


def cfg2_csr(m: int = 1 << 20, n: int | None = None, dist: str = "poisson", seed: int = 1,
             index_dtype=np.int64):
    """(values f32, col_idx, row_ptrs, x f32, shape) for the SpMV config.

    dist "poisson": lengths clip(Poisson(16), 1, 64); "zipf": clip(Zipf(1.5),
    1, 4096) (clipping, not resampling, is the recorded choice). Columns in a
    row are distinct and sorted: drawn uniformly, then rows holding a
    duplicate are redrawn without replacement.
    """
    n = m if n is None else n
    rng = np.random.default_rng(seed)
    if dist == "poisson":
        lens = np.clip(rng.poisson(16, size=m), 1, 64)
    elif dist == "zipf":
        lens = np.clip(rng.zipf(1.5, size=m), 1, 4096)
    else:
        raise ValueError(dist)
    values, cols, row_ptrs = random_csr(lens, n, rng)
    x = rng.standard_normal(n, dtype=np.float32)
    return values, cols.astype(index_dtype), row_ptrs.astype(index_dtype), x, (m, n)


def random_csr(lens, n: int, rng: np.random.Generator):
    """(values f32, col_idx int64, row_ptrs int64) with the given row lengths;
    columns of a row distinct, sorted, uniform over [0, n); values N(0,1)."""
    lens = np.minimum(np.asarray(lens, dtype=np.int64), n)
    m = lens.shape[0]
    row_ptrs = np.zeros(m + 1, dtype=np.int64)
    np.cumsum(lens, out=row_ptrs[1:])
    nnz = int(row_ptrs[-1])
    rows = np.repeat(np.arange(m, dtype=np.int64), lens)
    keys = rows * n + rng.integers(0, n, size=nnz, dtype=np.int64)
    keys.sort()
    cols = keys - rows * n
    dup = np.zeros(nnz, dtype=bool)
    dup[1:] = keys[1:] == keys[:-1]
    for r in np.unique(rows[dup]):
        s, e = row_ptrs[r], row_ptrs[r + 1]
        cols[s:e] = np.sort(rng.choice(n, size=e - s, replace=False))
    values = rng.standard_normal(nnz, dtype=np.float32)
    return values, cols, row_ptrs


def csr_matrix_from_arrays(values, cols, row_ptrs, shape, device="cpu") -> CSRMatrix:
    return CSRMatrix(
        values=torch.from_numpy(values).to(device),
        col_indices=torch.from_numpy(cols).to(device),
        row_ptrs=torch.from_numpy(row_ptrs).to(device),
        shape=tuple(shape),
    )


# ------------------------------------------------------------------ cfg3


def cfg3_block_mask(nb: int = 128, half_band: int = 3, density: float = 0.10, seed: int = 2) -> torch.Tensor:
    """Band |i-j| <= half_band plus uniform off-band blocks up to `density`."""
    g = torch.Generator().manual_seed(seed)
    i = torch.arange(nb)
    band = (i[:, None] - i[None, :]).abs() <= half_band
    target = int(round(density * nb * nb))
    off = (~band).flatten().nonzero().flatten()
    extra = max(0, target - int(band.sum()))
    pick = off[torch.randperm(off.numel(), generator=g)[:extra]]
    mask = band.flatten().clone()
    mask[pick] = True
    return mask.view(nb, nb)


def cfg3_bsr(nb: int = 128, ncols: int = 512, dtype: torch.dtype = torch.float32, seed: int = 2,
             density: float = 0.10):
    """(A_bsr, B) for the bsr_spmm-at-scale config (block values and B N(0,1))."""
    mask = cfg3_block_mask(nb, density=density, seed=seed)
    g = torch.Generator().manual_seed(seed + 1000)
    nnzb = int(mask.sum())
    blocks = torch.randn(nnzb, 128, 128, generator=g).to(dtype)
    B = torch.randn(nb * 128, ncols, generator=g).to(dtype)
    return bsr_from_block_mask(mask, 128, blocks=blocks), B


# ------------------------------------------------------------------ cfg4


def cfg4_screened(n: int = 4096, ncols: int | None = None, seed: int = 3):
    """(A, diag, B, threshold) for the Fock-like screened SpMM config."""
    ncols = n if ncols is None else ncols
    g = torch.Generator().manual_seed(seed)
    diag = torch.pow(10.0, torch.empty(n, dtype=torch.float64).uniform_(-14.0, 0.0, generator=g)).float()
    i = torch.arange(n, dtype=torch.float32)
    decay = torch.exp(-(i[:, None] - i[None, :]).abs() / 256.0)
    mag = torch.empty(n, n).uniform_(0.5, 1.0, generator=g)
    sign = torch.where(torch.rand(n, n, generator=g) < 0.5, -1.0, 1.0)
    A = (decay * mag * sign).contiguous()
    B = torch.randn(n, ncols, generator=g)
    return A, diag, B, 1e-20


# ------------------------------------------------------------------ cfg5


def cfg5_block_mask(n_blocks: int = 64, window: int = 4, n_global: int = 2) -> torch.Tensor:
    """Block row m attends to max(0, m-window+1)..m and to blocks 0..n_global-1."""
    mask = torch.zeros(n_blocks, n_blocks, dtype=torch.bool)
    for m in range(n_blocks):
        mask[m, max(0, m - window + 1) : m + 1] = True
    mask[:, :n_global] = True
    return mask


def cfg5_attention(heads: int = 32, seq: int = 8192, d: int = 128, dtype=torch.bfloat16, seed: int = 4):
    """(Q, K, V, mask_bsr) with Q/K/V (heads, seq, d) N(0,1) cast to `dtype`."""
    g = torch.Generator().manual_seed(seed)
    Q = torch.randn(heads, seq, d, generator=g).to(dtype)
    K = torch.randn(heads, seq, d, generator=g).to(dtype)
    V = torch.randn(heads, seq, d, generator=g).to(dtype)
    mask = cfg5_block_mask(seq // 128)
    return Q, K, V, bsr_from_block_mask(mask, 128)


def spd_bsr(nb: int = 128, b: int = 128, band: int = 1, n_pairs: int = 0, dtype=torch.float32, seed: int = 6):
    """(A, lam_min, lam_max): a symmetric positive definite BSR matrix for
    the fixed-step solvers, nb x nb blocks of b x b, with its Gershgorin
    eigenvalue bounds. Pattern: the block band |i - j| <= band plus n_pairs
    random symmetric off-band pairs; off-diagonal values N(0,1)/sqrt(b)
    (block (j, i) = block (i, j)^T), diagonal blocks symmetric N(0,1)/sqrt(b)
    plus s I with s = 1.5 x the largest off-diagonal absolute row sum, so the
    spectrum lies in [s - R, s + R] with R <= s / 1.5 (the bounds returned)."""
    g = torch.Generator().manual_seed(seed)
    pairs = {(i, j) for i in range(nb) for j in range(i + 1, min(nb, i + band + 1))}
    while len(pairs) < nb * band - band * (band + 1) // 2 + n_pairs:
        i, j = sorted(torch.randint(0, nb, (2,), generator=g).tolist())
        if i != j:
            pairs.add((i, j))
    blocks = {}
    for i, j in sorted(pairs):
        Bij = torch.randn(b, b, generator=g, dtype=torch.float64) / b**0.5
        blocks[(i, j)] = Bij
        blocks[(j, i)] = Bij.T.contiguous()
    for i in range(nb):
        Bii = torch.randn(b, b, generator=g, dtype=torch.float64) / b**0.5
        blocks[(i, i)] = (Bii + Bii.T) / 2
    rowsum = torch.zeros(nb * b, dtype=torch.float64)
    for (i, j), Bij in blocks.items():
        a = Bij.abs().sum(dim=1)
        if i == j:
            a = a - Bij.diagonal().abs()
        rowsum[i * b : (i + 1) * b] += a
    R = float(rowsum.max())
    shift = 1.5 * R
    for i in range(nb):
        blocks[(i, i)] = blocks[(i, i)] + shift * torch.eye(b, dtype=torch.float64)
    diag_min = min(float(blocks[(i, i)].diagonal().min()) for i in range(nb))
    diag_max = max(float(blocks[(i, i)].diagonal().max()) for i in range(nb))
    keys = sorted(blocks)
    ptrs = torch.zeros(nb + 1, dtype=torch.long)
    for i, _ in keys:
        ptrs[i + 1] += 1
    ptrs = torch.cumsum(ptrs, 0)
    A = BSRMatrix(torch.stack([blocks[k] for k in keys]).to(dtype), torch.tensor([j for _, j in keys]), ptrs,
                  (nb * b, nb * b), b)
    return A, diag_min - R, diag_max + R
