"""trnsparse_amd — the trnsparse sparse compute path, MI355X-native.

Drop-in for the reference's public API on the hot path (trnsparse/__init__.py):
formats (CSRMatrix, COOMatrix, BSRMatrix, from_dense, from_scipy,
eye_sparse), ops (spmv, spmm, bsr_spmm, screened_spmm,
block_sparse_attention_tiled and the small CSR helpers) and the backend
switch (set_backend / get_backend / HAS_NKI), plus the fixed-step solvers
(richardson_bsr, chebyshev_bsr, chebyshev_coeffs). The compute runs in
hand-written gfx950 HIP kernels behind the C ABI in include/trnsparse_hip.h.
"""

__version__ = "0.1.0"

from .backend import HAS_NKI, get_backend, has_hip, set_backend
from .formats import BSRMatrix, COOMatrix, CSRMatrix, eye_sparse, from_dense, from_scipy
from .iterative import chebyshev_bsr, chebyshev_coeffs, richardson_bsr
from .ops import (
    block_sparse_attention_tiled,
    bsr_spmm,
    nnz_per_row,
    screened_mask,
    screened_spmm,
    sparse_add,
    sparse_scale,
    sparse_transpose,
    spmm,
    spmv,
    spmv_symmetric,
)

__all__ = [
    "CSRMatrix",
    "COOMatrix",
    "BSRMatrix",
    "from_dense",
    "from_scipy",
    "eye_sparse",
    "spmv",
    "spmm",
    "spmv_symmetric",
    "bsr_spmm",
    "screened_spmm",
    "screened_mask",
    "block_sparse_attention_tiled",
    "sparse_add",
    "sparse_scale",
    "sparse_transpose",
    "nnz_per_row",
    "richardson_bsr",
    "chebyshev_bsr",
    "chebyshev_coeffs",
    "HAS_NKI",
    "has_hip",
    "set_backend",
    "get_backend",
]
