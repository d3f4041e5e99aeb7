"""ctypes binding of libtrnsparse_hip.so (C ABI: include/trnsparse_hip.h).

Every entry point takes device pointers, sizes, dtype codes and a HIP
stream handle; a nonzero status is turned into RuntimeError carrying
`tsp_last_error()`. Loading fails loudly when the library has not been
built: the HIP backend never falls back to another implementation.
"""

from __future__ import annotations

import ctypes
import pathlib
import threading

import torch

LIB_PATH = pathlib.Path(__file__).resolve().parent.parent / "libtrnsparse_hip.so"

TSP_F32, TSP_F64, TSP_BF16 = 0, 1, 2
TSP_I32, TSP_I64 = 0, 1

_DTYPE_CODE = {torch.float32: TSP_F32, torch.float64: TSP_F64, torch.bfloat16: TSP_BF16}
_INDEX_CODE = {torch.int32: TSP_I32, torch.int64: TSP_I64}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_DBL = ctypes.c_double

# name -> (restype, argtypes); mirrors include/trnsparse_hip.h
SIGNATURES: dict[str, tuple] = {
    "tsp_version": (_INT, []),
    "tsp_last_error": (ctypes.c_char_p, []),
    "tsp_bsr_spmm": (
        _INT,
        [_P, _INT, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _INT, _P, _P],
    ),
    "tsp_bsr_row_order": (_INT, [_P, _I64, _P, _P]),
    "tsp_bsr_col_view_workspace_size": (_I64, [_I64, _I64]),
    "tsp_bsr_col_view": (_INT, [_P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _I64, _P]),
    "tsp_bsr_spmv": (
        _INT,
        [_P, _INT, _P, _P, _I64, _I64, _I64, _I64, _P, _DBL, _P, _DBL, _P, _DBL, _P, _DBL, _P, _P, _P],
    ),
    "tsp_bsr_sddmm": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _I64, _P, _P, _I64, _I64, _INT, _P, _P]),
    "tsp_bsr_spmm_t": (_INT, [_P, _INT, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, _P]),
    "tsp_bsr_sddmm_ex": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _I64, _P, _P, _I64, _I64, _INT, _P, _INT, _P]),
    "tsp_bsa_block_softmax": (_INT, [_P, _P, _I64, _I64, _DBL, _P, _INT, _P, _P, _P]),
    "tsp_bsa_block_grad": (_INT, [_P, _P, _P, _I64, _I64, _DBL, _P, _P, _P, _P, _P, _INT, _P]),
    "tsp_bsa_rowdot": (_INT, [_P, _P, _INT, _I64, _I64, _P, _P]),
    "tsp_bsa_block_pgrad": (_INT, [_P, _P, _P, _P, _INT, _I64, _I64, _P, _P, _I64, _I64, _DBL, _P, _P, _P, _P, _P,
                                   _P]),
    "tsp_csr_plan_size": (_I64, [_I64, _I64]),
    "tsp_csr_plan": (_INT, [_P, _INT, _I64, _I64, _P, _P]),
    "tsp_csr_spmv": (_INT, [_P, _INT, _P, _P, _INT, _I64, _I64, _I64, _P, _P, _DBL, _P, _DBL, _P, _P]),
    "tsp_csr_colplan_geometry": (_INT, [_I64, _I64, _I64, _INT, _I64, _P]),
    "tsp_csr_colplan_build": (_INT, [_P, _INT, _P, _P, _INT, _I64, _I64, _I64, _P, _P, _P, _P]),
    "tsp_csr_colplan_refresh": (_INT, [_P, _INT, _P, _INT, _I64, _I64, _I64, _P, _P, _P]),
    "tsp_csr_colplan_spmv": (_INT, [_P, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _INT, _P, _DBL, _P, _DBL, _P, _P, _P]),
    "tsp_csr_spmm": (
        _INT,
        [_P, _INT, _P, _P, _INT, _I64, _I64, _I64, _P, _I64, _I64, _DBL, _P, _I64, _DBL, _P, _I64, _P],
    ),
    "tsp_csr_sddmm": (_INT, [_P, _P, _INT, _I64, _I64, _I64, _P, _I64, _P, _I64, _I64, _INT, _DBL, _P, _P]),
    "tsp_csr_bucket_plan_size": (_I64, [_I64]),
    "tsp_csr_bucket_plan": (_INT, [_P, _INT, _I64, _P, _P]),
    "tsp_csr_bucketed_spmv": (_INT, [_P, _INT, _P, _P, _INT, _I64, _I64, _I64, _P, _I64, _I64, _P, _DBL, _P, _DBL, _P,
                                     _P]),
    "tsp_screened_workspace_size": (_I64, [_I64, _INT]),
    "tsp_screened_spmm": (_INT, [_P, _INT, _I64, _P, _INT, _DBL, _I64, _P, _I64, _I64, _P, _I64, _P, _P]),
    "tsp_screened_spmm_noalloc_max_rows": (_I64, [_INT]),
    "tsp_screened_spmm_noalloc": (_INT, [_P, _INT, _I64, _P, _INT, _DBL, _I64, _P, _I64, _I64, _P, _I64, _P]),
    "tsp_screened_spmm_backward": (_INT, [_P, _INT, _I64, _P, _INT, _DBL, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _P,
                                          _I64, _P, _P]),
    "tsp_bsa_fwd": (_INT, [_P, _P, _P, _INT, _I64, _I64, _I64, _P, _P, _I64, _DBL, _P, _P, _P, _P]),
    "tsp_format_workspace_size": (_I64, [_I64]),
    "tsp_bsr_from_dense_pattern": (_INT, [_P, _INT, _I64, _I64, _I64, _I64, _DBL, _P, _P, _P, _P]),
    "tsp_bsr_from_dense_fill": (_INT, [_P, _INT, _I64, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _P]),
    "tsp_bsr_to_dense": (_INT, [_P, _INT, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _P]),
    "tsp_csr_from_dense_pattern": (_INT, [_P, _INT, _I64, _I64, _I64, _DBL, _P, _P, _P]),
    "tsp_csr_from_dense_fill": (_INT, [_P, _INT, _I64, _I64, _I64, _DBL, _P, _P, _P, _P]),
    "tsp_csr_to_dense": (_INT, [_P, _INT, _P, _P, _I64, _I64, _P, _I64, _P]),
    "tsp_csr_row_indices": (_INT, [_P, _I64, _I64, _P, _P]),
    "tsp_coo_to_csr_workspace_size": (_I64, [_I64, _I64, _I64]),
    "tsp_coo_to_csr": (_INT, [_P, _INT, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P]),
    "tsp_coo_sum_to_csr_workspace_size": (_I64, [_I64, _I64, _I64]),
    "tsp_coo_sum_to_csr": (_INT, [_P, _INT, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P]),
    "tsp_csr_transpose_workspace_size": (_I64, [_I64, _I64, _I64, _INT]),
    "tsp_csr_sum_workspace_size": (_I64, [_I64, _I64, _I64, _I64, _INT]),
    "tsp_csr_sum": (_INT, [_P, _P, _P, _I64, _P, _P, _P, _I64, _INT, _I64, _I64, _P, _P, _P, _P, _I64, _P]),
    "tsp_csr_transpose": (_INT, [_P, _INT, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P]),
    "tsp_bsa_bwd_plan": (_I64, [_P, _I64, _I64, _I64, _I64, _P, _I64]),
    "tsp_bsa_bwd_workspace_size": (_I64, [_I64, _I64, _I64, _I64]),
    "tsp_bsa_bwd": (
        _INT,
        [_P, _P, _P, _P, _P, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _I64, _DBL, _P, _P, _P, _P, _P,
         _P, _I64, _I64, _I64, _P, _P],
    ),
}

_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise RuntimeError if unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH.name} is not built; run `python -m trnsparse_amd.build_lib` "
                    "(the HIP backend has no fallback)"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


OPS_PATH = pathlib.Path(__file__).resolve().parent.parent / "libtrnsparse_torch_ops.so"
_ops = None


def ops():
    """`torch.ops.trnsparse_hip` (csrc/torch_ops.cpp) after loading the
    operator library once; raise RuntimeError if it is not built."""
    global _ops
    if _ops is not None:
        return _ops
    load()  # the operator library links against the C library
    with _lock:
        if _ops is None:
            if not OPS_PATH.exists():
                raise RuntimeError(
                    f"{OPS_PATH.name} is not built; run `python -m trnsparse_amd.build_lib` "
                    "(the HIP backend has no fallback)"
                )
            torch.ops.load_library(str(OPS_PATH))
            _ops = torch.ops.trnsparse_hip
    return _ops


def last_error() -> str:
    return load().tsp_last_error().decode(errors="replace")


def call(name: str, *args) -> None:
    """Call a status-returning entry point; raise RuntimeError on failure."""
    st = getattr(load(), name)(*args)
    if st != 0:
        raise RuntimeError(f"{name} failed with status {st}: {last_error()}")


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise RuntimeError(f"HIP backend does not support dtype {dt}") from None


def index_code(dt: torch.dtype) -> int:
    try:
        return _INDEX_CODE[dt]
    except KeyError:
        raise RuntimeError(f"HIP backend needs int32 or int64 indices, got {dt}") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
