"""Golden fixtures (tests/golden/, written by tests/golden/make_golden.py).

CPU: the oracle and the seeded generators still reproduce the stored
vectors (a regression guard for the checker itself). GPU: the HIP kernels,
through the public API, reproduce them at the parity bar (fp32: max error
<= 1e-4 relative to the |.|-scale stored beside each output).
"""

from __future__ import annotations

import pathlib

import numpy as np
import pytest
import torch

import trnsparse_amd as ts
from oracle import ref
from trnsparse_amd import workloads as W

G = pathlib.Path(__file__).resolve().parent / "golden"
TOL = 1e-4


def _load(name):
    with np.load(G / name, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


# ---------------------------------------------------------------- CPU


def test_cfg1_generator_and_oracle_reproduce_fixture():
    f = _load("cfg1_bsr.npz")
    A, B, _ = W.cfg1_bsr_plumbing()
    assert np.array_equal(A.block_row_ptrs.numpy(), f["block_row_ptrs"])
    assert np.array_equal(A.block_col_indices.numpy(), f["block_col_indices"])
    C = ref.bsr_spmm(A.blocks.numpy(), A.block_col_indices.numpy(), A.block_row_ptrs.numpy(), A.shape, 128, B.numpy())
    assert ref.scaled_error(C[f["rows"]], f["C_rows"], f["scale_rows"]) <= 1e-6
    np.testing.assert_allclose(C.sum(axis=0), f["C_colsum"], rtol=1e-12, atol=1e-9)


def test_small_fixtures_reproduce_on_cpu():
    a = _load("attention_small.npz")
    out, rmax, rden = ref.block_sparse_attention(a["Q"], a["K"], a["V"], a["block_row_ptrs"], a["block_col_indices"],
                                                 128, float(a["scale"]))
    assert ref.scaled_error(out, a["O"], a["O_scale"]) <= 1e-6
    np.testing.assert_allclose(rmax, a["row_max"], rtol=1e-12)
    np.testing.assert_allclose(rden, a["row_denom"], rtol=1e-12)
    s = _load("screened_small.npz")
    assert np.array_equal(ref.screened_mask(s["diag"], float(s["threshold"])), s["mask"])
    C = ref.screened_spmm(s["A"], s["diag"], s["B"], float(s["threshold"]))
    assert ref.scaled_error(C, s["C"], s["scale"]) <= 1e-6
    v = _load("spmv_small.npz")
    m, n = v["shape"]
    out = ref.csr_spmv(v["values"], v["col_indices"], v["row_ptrs"], (m, n), v["x"], float(v["alpha"]), v["y"],
                       float(v["beta"]))
    assert ref.scaled_error(out, v["out"], v["scale"]) <= 1e-12


# ---------------------------------------------------------------- GPU


@pytest.mark.gpu
def test_hip_reproduces_golden(hip_backend):
    dev = torch.device("cuda")
    f = _load("cfg1_bsr.npz")
    A, B, _ = W.cfg1_bsr_plumbing()
    C = ts.bsr_spmm(A, B.to(dev)).cpu().numpy()
    assert ref.scaled_error(C[f["rows"]], f["C_rows"], f["scale_rows"]) <= TOL

    a = _load("attention_small.npz")
    mask = W.bsr_from_block_mask(torch.from_numpy(a["block_mask"]), 128)
    Q, K, V = (torch.from_numpy(a[k]).to(dev) for k in ("Q", "K", "V"))
    O = ts.block_sparse_attention_tiled(Q, K, V, mask).cpu().numpy()
    assert ref.scaled_error(O, a["O"], np.maximum(a["O_scale"], 1e-30)) <= TOL

    s = _load("screened_small.npz")
    Cs = ts.screened_spmm(*(torch.from_numpy(s[k]).to(dev) for k in ("A", "diag")),
                          torch.from_numpy(s["B"]).to(dev), float(s["threshold"])).cpu().numpy()
    assert ref.scaled_error(Cs, s["C"], s["scale"]) <= TOL

    v = _load("spmv_small.npz")
    m, n = (int(t) for t in v["shape"])
    Acsr = W.csr_matrix_from_arrays(v["values"], v["col_indices"], v["row_ptrs"], (m, n), device=dev)
    y = ts.spmv(Acsr, torch.from_numpy(v["x"]).to(dev), alpha=float(v["alpha"]), y=torch.from_numpy(v["y"]).to(dev),
                beta=float(v["beta"])).cpu().numpy()
    assert ref.scaled_error(y, v["out"], v["scale"]) <= TOL
