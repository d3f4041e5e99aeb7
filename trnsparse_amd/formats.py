"""Sparse matrix formats: CSR, COO and BSR.

Same dataclasses, fields, defaults and structure rules as the reference
(trnsparse/formats.py). Structure tensors are int64 (torch.long) as there.
On the HIP backend, conversions whose input lives on the GPU (float32,
float64, bfloat16 values) run as device kernels (`hip/formats.py`,
`csrc/formats.hip`) and return device tensors; otherwise the helpers are
vectorised torch ops. Both produce exactly the structure the reference
produces:

- `BSRMatrix.from_dense` (reference formats.py:183-221): pad to a block
  multiple, keep a block iff max|v| > threshold, row-major block order,
  block columns sorted within a row, `shape` = the unpadded shape.
- `COOMatrix.to_csr` (reference formats.py:104-124): entries sorted by the
  key row*n+col, `row_ptrs` = cumulative row counts.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .backend import _use_hip


def _device_formats(t: torch.Tensor):
    """The device conversion module when `t` is a GPU tensor of a dtype the
    kernels serve and the HIP backend is in effect, else None."""
    if not (isinstance(t, torch.Tensor) and t.is_cuda and _use_hip()):
        return None
    from .hip import formats as hf

    return hf if t.dtype in hf.DEVICE_DTYPES else None


@dataclass
class CSRMatrix:
    """Compressed Sparse Row matrix (reference formats.py:21-69).

    values:      (nnz,)  non-zero values
    col_indices: (nnz,)  column of each value
    row_ptrs:    (m+1,)  row i spans row_ptrs[i]:row_ptrs[i+1]
    shape:       (m, n)
    """

    values: torch.Tensor
    col_indices: torch.Tensor
    row_ptrs: torch.Tensor
    shape: tuple[int, int]

    @property
    def nnz(self) -> int:
        return self.values.shape[0]

    @property
    def dtype(self) -> torch.dtype:
        return self.values.dtype

    @property
    def density(self) -> float:
        return self.nnz / (self.shape[0] * self.shape[1])

    def to_dense(self) -> torch.Tensor:
        hf = _device_formats(self.values)
        if hf is not None:
            return hf.csr_to_dense(self.values, self.col_indices, self.row_ptrs, self.shape)
        t = torch.sparse_csr_tensor(self.row_ptrs, self.col_indices, self.values, size=self.shape)
        return t.to_dense()

    def to_coo(self) -> COOMatrix:
        """COO view with row indices expanded from `row_ptrs` (reference :54-65)."""
        hf = _device_formats(self.values)
        if hf is not None:
            rows = hf.csr_row_indices(self.row_ptrs, self.shape[0], self.nnz, self.values.device)
            return COOMatrix(values=self.values.clone(), row_indices=rows, col_indices=self.col_indices.clone(),
                             shape=self.shape)
        counts = (self.row_ptrs[1:] - self.row_ptrs[:-1]).to("cpu")
        rows = torch.repeat_interleave(torch.arange(self.shape[0], dtype=torch.long), counts)
        return COOMatrix(
            values=self.values.clone(),
            row_indices=rows,
            col_indices=self.col_indices.clone(),
            shape=self.shape,
        )

    def __repr__(self) -> str:
        return f"CSRMatrix(shape={self.shape}, nnz={self.nnz}, density={self.density:.4f})"


@dataclass
class COOMatrix:
    """Coordinate (triplet) matrix (reference formats.py:71-127)."""

    values: torch.Tensor
    row_indices: torch.Tensor
    col_indices: torch.Tensor
    shape: tuple[int, int]

    @property
    def nnz(self) -> int:
        return self.values.shape[0]

    @property
    def dtype(self) -> torch.dtype:
        return self.values.dtype

    @property
    def density(self) -> float:
        return self.nnz / (self.shape[0] * self.shape[1])

    def to_dense(self) -> torch.Tensor:
        m, n = self.shape
        dense = torch.zeros(m, n, dtype=self.dtype, device=self.values.device)
        dense[self.row_indices, self.col_indices] = self.values
        return dense

    def to_csr(self) -> CSRMatrix:
        """Sort by (row, col) and build row pointers (reference :104-124)."""
        m, n = self.shape
        hf = _device_formats(self.values)
        if hf is not None:
            vals, cols, rp = hf.coo_to_csr(self.values, self.row_indices, self.col_indices, self.shape)
            return CSRMatrix(values=vals, col_indices=cols, row_ptrs=rp, shape=self.shape)
        order = torch.argsort(self.row_indices * n + self.col_indices, stable=True)
        rows = self.row_indices[order]
        counts = torch.bincount(rows.to("cpu"), minlength=m)
        row_ptrs = torch.zeros(m + 1, dtype=torch.long)
        row_ptrs[1:] = torch.cumsum(counts, dim=0)
        return CSRMatrix(
            values=self.values[order],
            col_indices=self.col_indices[order],
            row_ptrs=row_ptrs,
            shape=self.shape,
        )

    def __repr__(self) -> str:
        return f"COOMatrix(shape={self.shape}, nnz={self.nnz}, density={self.density:.4f})"


def _round_up(v: int, b: int) -> int:
    return ((v + b - 1) // b) * b


@dataclass
class BSRMatrix:
    """Block-Sparse Row matrix (reference formats.py:130-263).

    blocks:            (n_blocks, b, b)  stored dense blocks, row-major
    block_col_indices: (n_blocks,)       column-block index of each block
    block_row_ptrs:    (ceil(M/b)+1,)    block row i spans [ptr[i], ptr[i+1])
    shape:             (M, N)            element shape (unpadded)
    block_size:        b, default 128 (one MFMA-friendly 128x128 tile)
    """

    blocks: torch.Tensor
    block_col_indices: torch.Tensor
    block_row_ptrs: torch.Tensor
    shape: tuple[int, int]
    block_size: int = 128

    @property
    def n_blocks(self) -> int:
        return self.blocks.shape[0]

    @property
    def nnz(self) -> int:
        """Stored elements = n_blocks * b^2 (zeros inside stored blocks count)."""
        return self.n_blocks * self.block_size * self.block_size

    @property
    def dtype(self) -> torch.dtype:
        return self.blocks.dtype

    @property
    def density(self) -> float:
        """Fraction of blocks stored (block density, not element density)."""
        m, n = self.shape
        total = (m // self.block_size) * (n // self.block_size)
        return self.n_blocks / total if total else 0.0

    @classmethod
    def from_dense(cls, A: torch.Tensor, block_size: int = 128, threshold: float = 0.0) -> BSRMatrix:
        """Keep a block iff some element has |v| > threshold (reference :183-221)."""
        m, n = A.shape
        b = block_size
        hf = _device_formats(A)
        if hf is not None:
            blocks, col_idx, row_ptrs = hf.bsr_from_dense(A, b, threshold)
            return cls(blocks=blocks, block_col_indices=col_idx, block_row_ptrs=row_ptrs, shape=(m, n), block_size=b)
        m_pad, n_pad = _round_up(m, b), _round_up(n, b)
        if (m_pad, n_pad) != (m, n):
            padded = torch.zeros(m_pad, n_pad, dtype=A.dtype, device=A.device)
            padded[:m, :n] = A
            A = padded
        mb, nbc = m_pad // b, n_pad // b
        grid = A.reshape(mb, b, nbc, b).permute(0, 2, 1, 3).contiguous()
        keep = grid.abs().amax(dim=(-2, -1)) > threshold  # (mb, nbc)
        row_ptrs = torch.zeros(mb + 1, dtype=torch.long)
        row_ptrs[1:] = keep.sum(dim=1).cumsum(dim=0)
        col_idx = keep.nonzero(as_tuple=False)[:, 1].to(torch.long)
        return cls(
            blocks=grid[keep].contiguous(),
            block_col_indices=col_idx,
            block_row_ptrs=row_ptrs,
            shape=(m, n),
            block_size=b,
        )

    @classmethod
    def from_csr(cls, csr: CSRMatrix, block_size: int = 128, threshold: float = 0.0) -> BSRMatrix:
        """CSR -> BSR through the dense intermediate (reference :223-231)."""
        return cls.from_dense(csr.to_dense(), block_size=block_size, threshold=threshold)

    def block_rows(self) -> torch.Tensor:
        """Block-row index of every stored block (expanded `block_row_ptrs`)."""
        counts = (self.block_row_ptrs[1:] - self.block_row_ptrs[:-1]).to("cpu")
        mb = counts.shape[0]
        return torch.repeat_interleave(torch.arange(mb, dtype=torch.long), counts)

    def to_dense(self) -> torch.Tensor:
        """Scatter the stored blocks into a dense (M, N) tensor (reference :233-251)."""
        m, n = self.shape
        b = self.block_size
        hf = _device_formats(self.blocks)
        if hf is not None:
            return hf.bsr_to_dense(self.blocks, self.block_row_ptrs, self.block_col_indices, self.shape, b)
        m_pad, n_pad = _round_up(m, b), _round_up(n, b)
        mb, nbc = m_pad // b, n_pad // b
        dev = self.blocks.device
        grid = torch.zeros(mb, nbc, b, b, dtype=self.dtype, device=dev)
        if self.n_blocks:
            rows = self.block_rows().to(dev)
            grid[rows, self.block_col_indices.to(dev)] = self.blocks
        dense = grid.permute(0, 2, 1, 3).reshape(m_pad, n_pad)
        return dense[:m, :n].contiguous()

    def to_csr(self) -> CSRMatrix:
        """BSR -> CSR through the dense intermediate (reference :253-257)."""
        return from_dense(self.to_dense(), threshold=0.0)

    def __repr__(self) -> str:
        return (
            f"BSRMatrix(shape={self.shape}, block_size={self.block_size}, "
            f"n_blocks={self.n_blocks}, block_density={self.density:.4f})"
        )


def from_dense(A: torch.Tensor, threshold: float = 0.0) -> CSRMatrix:
    """Dense -> CSR keeping |v| > threshold (reference formats.py:269-278)."""
    m, n = A.shape
    hf = _device_formats(A)
    if hf is not None:
        vals, cols, rp = hf.csr_from_dense(A, threshold)
        return CSRMatrix(values=vals, col_indices=cols, row_ptrs=rp, shape=(m, n))
    mask = torch.abs(A) > threshold
    rows, cols = torch.where(mask)
    coo = COOMatrix(values=A[mask], row_indices=rows, col_indices=cols, shape=(m, n))
    return coo.to_csr()


def from_scipy(sp_matrix) -> CSRMatrix:
    """scipy.sparse -> CSR with float32 values (reference formats.py:281-291)."""
    import scipy.sparse as sp

    csr = sp.csr_matrix(sp_matrix)
    return CSRMatrix(
        values=torch.tensor(csr.data, dtype=torch.float32),
        col_indices=torch.tensor(csr.indices, dtype=torch.long),
        row_ptrs=torch.tensor(csr.indptr, dtype=torch.long),
        shape=csr.shape,
    )


def eye_sparse(n: int, dtype: torch.dtype = torch.float32) -> CSRMatrix:
    """Sparse identity (reference formats.py:294-301)."""
    return CSRMatrix(
        values=torch.ones(n, dtype=dtype),
        col_indices=torch.arange(n, dtype=torch.long),
        row_ptrs=torch.arange(n + 1, dtype=torch.long),
        shape=(n, n),
    )
