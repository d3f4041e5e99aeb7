"""Compile the oracle's C restatement (oracle/csr_spmv.c) into
oracle/liboracle.so with gcc, and load it with ctypes. Test infrastructure only.

The reference is pure Python, so there is no reference source to build into
oracle/_ref; this library is our own restatement.
"""

from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
SRC = HERE / "csr_spmv.c"
LIB = HERE / "liboracle.so"


def build() -> pathlib.Path:
    tmp = LIB.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-fopenmp", "-fPIC", "-shared", "-o", str(tmp), str(SRC), "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stderr}")
    tmp.replace(LIB)
    return LIB


_lib = None


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        P, I64, INT, DBL, FLT = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double, ctypes.c_float
        lib.oracle_csr_spmv_f64.argtypes = [P, P, P, INT, I64, P, DBL, P, DBL, INT, P]
        lib.oracle_csr_spmv_f64.restype = None
        lib.oracle_csr_spmv_f32.argtypes = [P, P, P, INT, I64, P, FLT, P, FLT, P]
        lib.oracle_csr_spmv_f32.restype = None
        _lib = lib
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def csr_spmv_f64(values, col, row_ptrs, m, x, alpha=1.0, y=None, beta=0.0, absolute=False):
    """Float64-accumulated SpMV (and |A|.|x| scale with absolute=True)."""
    values = np.ascontiguousarray(values, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    y = None if y is None else np.ascontiguousarray(y, np.float32)
    col = np.ascontiguousarray(col)
    row_ptrs = np.ascontiguousarray(row_ptrs)
    assert col.dtype == row_ptrs.dtype and col.dtype in (np.int32, np.int64)
    out = np.empty(m, np.float64)
    load().oracle_csr_spmv_f64(_p(values), _p(col), _p(row_ptrs), int(col.dtype == np.int64), m, _p(x),
                               alpha, _p(y), beta, int(absolute), _p(out))
    return out


def csr_spmv_f32(values, col, row_ptrs, m, x, alpha=1.0, y=None, beta=0.0):
    """Float32-accumulated SpMV over OpenMP threads (CPU baseline)."""
    out = np.empty(m, np.float32)
    load().oracle_csr_spmv_f32(_p(values), _p(col), _p(row_ptrs), int(col.dtype == np.int64), m, _p(x),
                               alpha, _p(y), beta, _p(out))
    return out
