"""The allocation-free screened SpMM entry point (tsp_screened_spmm_noalloc).

Called through the C ABI and checked against tsp_screened_spmm (the entry
point that takes a caller workspace) on two calls in a row, the second with
a smaller input, bit for bit (same kernels, same arithmetic), and against
the CPU oracle at the fp32 bar. The size limit is checked on the host.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import ref
from trnsparse_amd.hip import _lib

pytestmark = pytest.mark.gpu


def _case(n, ncols, seed, dtype=torch.float32, diag_dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(n, n, generator=g, dtype=torch.float64).to(dtype)
    diag = (10.0 ** (-8 * torch.rand(n, generator=g, dtype=torch.float64))).to(diag_dtype)
    B = torch.randn(n, ncols, generator=g, dtype=torch.float64).to(dtype)
    return A, diag, B


def _run(name, A, diag, B, thr, with_ws):
    dev = torch.device("cuda")
    Ad, dd, Bd = A.to(dev), diag.to(dev), B.to(dev)
    m, ncols = A.shape[0], B.shape[1]
    C = torch.full((m, ncols), float("nan"), dtype=A.dtype, device=dev)
    dcode, code = _lib.dtype_code(dd.dtype), _lib.dtype_code(Ad.dtype)
    st = _lib.stream_handle(dev)
    if with_ws:
        ws = torch.empty(max(1, _lib.load().tsp_screened_workspace_size(m, dcode)), dtype=torch.uint8, device=dev)
        _lib.call("tsp_screened_spmm", Ad.data_ptr(), code, m, dd.data_ptr(), dcode, math.sqrt(thr), m, Bd.data_ptr(),
                  ncols, ncols, C.data_ptr(), ncols, ws.data_ptr(), st)
    else:
        _lib.call("tsp_screened_spmm_noalloc", Ad.data_ptr(), code, m, dd.data_ptr(), dcode, math.sqrt(thr), m,
                  Bd.data_ptr(), ncols, ncols, C.data_ptr(), ncols, st)
    torch.cuda.synchronize()
    return C.cpu()


@pytest.mark.parametrize("diag_dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_noalloc_matches_workspace_entry_point(dtype, diag_dtype):
    thr = 1e-6
    # two calls in a row, the second smaller: the scratch keeps the first
    # call's Q values past the second call's rows, which must not leak in
    # (an fp64 diag stores 8-byte Q entries in the scratch, a smaller row limit)
    for n, ncols, seed in ((1000, 96, 1), (300, 40, 2)):
        A, diag, B = _case(n, ncols, seed, dtype, diag_dtype)
        got = _run("noalloc", A, diag, B, thr, with_ws=False)
        want = _run("ws", A, diag, B, thr, with_ws=True)
        assert torch.equal(got, want)
        exact = ref.screened_spmm(A.numpy(), diag.numpy(), B.numpy(), thr)
        scale = ref.screened_spmm(A.numpy(), diag.numpy(), B.numpy(), thr, absolute=True)
        assert ref.scaled_error(got.numpy(), exact, scale) <= 1e-4
