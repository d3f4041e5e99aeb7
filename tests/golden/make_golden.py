"""Write the golden fixtures in this directory from the CPU oracle.

The reference repository holds no golden-vector files (its tests recompute
every expectation from seeds), so these fixtures are a regression guard of
this build, not parity evidence: the oracle they come from is pinned by
tests/test_oracle.py. Each fixture stores its inputs (or, for cfg1, the
seeded generator's structure plus every 16th output row) and the oracle's
outputs (float64 accumulation, stored as float32 where a float32 copy is
far inside the 1e-4 parity bar), small enough to commit.

Usage: python tests/golden/make_golden.py   (rewrites the .npz files)
"""

from __future__ import annotations

import math
import pathlib
import sys

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import ref  # noqa: E402
from trnsparse_amd import workloads as W  # noqa: E402


def cfg1():
    A, B, _ = W.cfg1_bsr_plumbing()
    args = (A.blocks.numpy(), A.block_col_indices.numpy(), A.block_row_ptrs.numpy(), A.shape, 128)
    C = ref.bsr_spmm(*args, B.numpy())
    S = ref.bsr_spmm(*args, B.numpy(), absolute=True)
    np.savez_compressed(HERE / "cfg1_bsr.npz", block_row_ptrs=A.block_row_ptrs.numpy(),
                        block_col_indices=A.block_col_indices.numpy(), rows=np.arange(0, 1024, 16),
                        C_rows=C[::16].astype(np.float32), scale_rows=S[::16].astype(np.float32),
                        C_colsum=C.sum(axis=0))


def attention():
    g = torch.Generator().manual_seed(7)
    S, D = 384, 32
    i = torch.arange(3)
    mask = ((i[:, None] - i[None, :]).abs() <= 1)
    mask[2, 0] = True
    Q, K, V = (torch.randn(S, D, generator=g) for _ in range(3))
    bsr = W.bsr_from_block_mask(mask, 128)
    ptr, col = bsr.block_row_ptrs.numpy(), bsr.block_col_indices.numpy()
    out, rmax, rden = ref.block_sparse_attention(Q.numpy(), K.numpy(), V.numpy(), ptr, col, 128, D**-0.5)
    sc, _, _ = ref.block_sparse_attention(Q.numpy(), K.numpy(), np.abs(V.numpy()), ptr, col, 128, D**-0.5)
    np.savez_compressed(HERE / "attention_small.npz", Q=Q.numpy(), K=K.numpy(), V=V.numpy(),
                        block_mask=mask.numpy(), block_row_ptrs=ptr, block_col_indices=col, scale=D**-0.5,
                        O=out.astype(np.float32), row_max=rmax, row_denom=rden, O_scale=sc.astype(np.float32))


def screened():
    g = torch.Generator().manual_seed(8)
    n, N, thr = 160, 40, 1e-5
    A = torch.randn(n, n, generator=g)
    diag = 10.0 ** (-8 * torch.rand(n, generator=g))
    B = torch.randn(n, N, generator=g)
    C = ref.screened_spmm(A.numpy(), diag.numpy(), B.numpy(), thr)
    S = ref.screened_spmm(A.numpy(), diag.numpy(), B.numpy(), thr, absolute=True)
    mask = ref.screened_mask(diag.numpy(), thr)
    np.savez_compressed(HERE / "screened_small.npz", A=A.numpy(), diag=diag.numpy(), B=B.numpy(), threshold=thr,
                        mask=mask, C=C.astype(np.float32), scale=S.astype(np.float32))


def spmv():
    rng = np.random.default_rng(9)
    m, n = 300, 500
    lens = rng.integers(0, 30, m)
    lens[[0, 17, m - 1]] = 0
    v, c, p = W.random_csr(lens, n, rng)
    x = rng.standard_normal(n).astype(np.float32)
    y = rng.standard_normal(m).astype(np.float32)
    out = ref.csr_spmv(v, c, p, (m, n), x, alpha=-1.25, y=y, beta=0.5)
    sc = ref.csr_spmv(v, c, p, (m, n), x, alpha=-1.25, y=y, beta=0.5, absolute=True)
    np.savez_compressed(HERE / "spmv_small.npz", values=v, col_indices=c, row_ptrs=p, shape=np.array([m, n]), x=x,
                        y=y, alpha=-1.25, beta=0.5, out=out, scale=sc)


if __name__ == "__main__":
    cfg1()
    attention()
    screened()
    spmv()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)
