"""The registered operator layer (torch.ops.trnsparse_hip, csrc/torch_ops.cpp).

CPU: the operator library loads next to the C library, every operator has
its schema, and the Meta implementations give the output shapes and dtypes
(what torch.compile traces with). GPU: operators called directly agree with
the public API, a torch.compile(fullgraph=True) region traces through them,
and a HIP graph replays them.
"""

from __future__ import annotations

import pytest
import torch

from trnsparse_amd.hip import _lib

OPS = {
    "bsr_spmm": "(Tensor blocks, Tensor block_row_ptrs, Tensor block_col_indices, Tensor? row_order, int m, int n, "
                "int block_size, Tensor B, ScalarType out_dtype) -> Tensor",
    "bsr_sddmm": "(Tensor grad_out, Tensor B, Tensor block_rows, Tensor block_col_indices, int m, int n, "
                 "int block_size) -> Tensor",
    "bsr_spmm_t": "(Tensor blocks, Tensor col_ptrs, Tensor col_block_ids, Tensor col_block_rows, Tensor col_order, "
                  "int m, int n, int block_size, Tensor grad_out) -> Tensor",
    "csr_spmv": "(Tensor values, Tensor col_indices, Tensor row_ptrs, Tensor windows, int m, int n, Tensor x, "
                "float alpha, Tensor? y, float beta) -> Tensor",
    "csr_colplan_spmv": "(Tensor plan, int[] geometry, Tensor values, Tensor col_indices, Tensor row_ptrs, int m, "
                        "int n, Tensor x, float alpha, Tensor? y, float beta) -> Tensor",
    "csr_spmm": "(Tensor values, Tensor col_indices, Tensor row_ptrs, int m, int n, Tensor X, float alpha, "
                "Tensor? Y, float beta) -> Tensor",
    "screened_spmm": "(Tensor A, Tensor diag_integrals, Tensor B, float threshold_sqrt) -> Tensor",
    "screened_spmm_backward": "(Tensor A, Tensor diag_integrals, Tensor B, float threshold_sqrt, Tensor grad_out, "
                              "bool need_a, bool need_b) -> (Tensor, Tensor)",
    "bsa_fwd": "(Tensor Q, Tensor K, Tensor V, Tensor block_row_ptrs, Tensor block_col_indices, int block_size, "
               "float scale, bool return_stats) -> (Tensor, Tensor, Tensor)",
    "bsa_bwd": "(Tensor Q, Tensor K, Tensor V, Tensor O, Tensor dO, Tensor block_row_ptrs, Tensor block_col_indices, "
               "Tensor col_ptrs, Tensor col_block_rows, int n_block_cols, int block_size, float scale, "
               "Tensor row_max, Tensor row_denom, Tensor plan, int n_items, int n_splits, int n_partials) -> "
               "(Tensor, Tensor, Tensor)",
}


def test_operator_library_in_tree_and_schemas():
    ops = _lib.ops()
    assert _lib.OPS_PATH.parent == _lib.LIB_PATH.parent  # in-tree, next to the C library
    for name, sig in OPS.items():
        assert str(getattr(ops, name).default._schema) == f"trnsparse_hip::{name}{sig}"


def _meta(*shape, dtype=torch.float32):
    return torch.empty(*shape, dtype=dtype, device="meta")


def test_meta_shapes():
    ops = _lib.ops()
    i64 = torch.int64
    rp, ci = _meta(4, dtype=i64), _meta(6, dtype=i64)
    assert ops.bsr_spmm(_meta(6, 128, 128), rp, ci, None, 300, 512, 128, _meta(512, 70), torch.float32).shape == (300, 70)
    c = ops.bsr_spmm(_meta(6, 32, 32, dtype=torch.bfloat16), rp, ci, None, 96, 96, 32,
                     _meta(96, 8, dtype=torch.bfloat16), torch.bfloat16)
    assert c.shape == (96, 8) and c.dtype == torch.bfloat16
    assert ops.bsr_sddmm(_meta(300, 70), _meta(512, 70), ci, ci, 300, 512, 128).shape == (6, 128, 128)
    assert ops.bsr_spmm_t(_meta(6, 128, 128), _meta(5, dtype=i64), ci, ci, _meta(4, dtype=torch.int32), 300, 512, 128,
                          _meta(300, 70)).shape == (512, 70)
    v, cols, ptrs = _meta(50), _meta(50, dtype=torch.int32), _meta(11, dtype=torch.int32)
    assert ops.csr_spmv(v, cols, ptrs, _meta(3, dtype=i64), 10, 20, _meta(20), 1.0, None, 0.0).shape == (10,)
    geom = [0] * 10
    assert ops.csr_colplan_spmv(_meta(100, dtype=torch.uint8), geom, v, cols, ptrs, 10, 20, _meta(20), 1.0, None,
                                0.0).shape == (10,)
    assert ops.csr_spmm(v, cols, ptrs, 10, 20, _meta(20, 3), 1.0, None, 0.0).shape == (10, 3)
    assert ops.screened_spmm(_meta(64, 64), _meta(64), _meta(64, 9), 1e-5).shape == (64, 9)
    dA, dB = ops.screened_spmm_backward(_meta(64, 64), _meta(64), _meta(64, 9), 1e-5, _meta(64, 9), True, False)
    assert dA.shape == (64, 64) and dB.numel() == 0
    Q = _meta(3, 512, 64, dtype=torch.bfloat16)
    O, rm, rd = ops.bsa_fwd(Q, Q, Q, rp, ci, 128, 0.125, True)
    assert O.shape == Q.shape and O.dtype == torch.bfloat16 and rm.shape == (3, 4, 128) and rm.dtype == torch.float32
    O, rm, _ = ops.bsa_fwd(_meta(2, 300, 32, dtype=torch.float64), _meta(2, 300, 32, dtype=torch.float64),
                           _meta(2, 300, 32, dtype=torch.float64), rp, ci, 128, 0.2, True)
    assert rm.shape == (2, 2, 128) and rm.dtype == torch.float64
    g = ops.bsa_bwd(Q, Q, Q, Q, Q, rp, ci, rp, ci, 4, 128, 0.125, _meta(3, 512), _meta(3, 512),
                    _meta(20, dtype=torch.int32), 4, 0, 0)
    assert all(t.shape == Q.shape and t.dtype == Q.dtype for t in g)


@pytest.mark.gpu
def test_ops_match_api_compile_and_graph(hip_backend):
    import trnsparse_amd as ts
    from trnsparse_amd.hip import dispatch as D

    ops = _lib.ops()
    g = torch.Generator().manual_seed(3)
    A = torch.randn(384, 256, generator=g) * (torch.rand(384, 256, generator=g) < 0.5)
    bsr = ts.BSRMatrix.from_dense(A, block_size=128)
    B = torch.randn(256, 96, generator=g).cuda()
    want = ts.bsr_spmm(bsr, B)
    rp, ci, order = D._bsr_plan(bsr.block_col_indices, bsr.block_row_ptrs, 3, B.device, holder=bsr)
    blocks = bsr.blocks.cuda()
    got = ops.bsr_spmm(blocks, rp, ci, order, 384, 256, 128, B, torch.float32)
    torch.testing.assert_close(got, want, rtol=0, atol=0)

    @torch.compile(fullgraph=True, backend="aot_eager")
    def f(blocks, rp, ci, B):
        return ops.bsr_spmm(blocks, rp, ci, None, 384, 256, 128, B * 2.0, torch.float32) + 1.0

    torch.testing.assert_close(f(blocks, rp, ci, B), 2.0 * want + 1.0, rtol=1e-6, atol=1e-5)

    # HIP graph: capture once, replay with new B contents, eager work between replays
    static_B = B.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.bsr_spmm(blocks, rp, ci, order, 384, 256, 128, static_B, torch.float32)  # warm up on the side stream
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_C = ops.bsr_spmm(blocks, rp, ci, order, 384, 256, 128, static_B, torch.float32)
    for rep in range(3):
        newB = torch.randn(256, 96, generator=torch.Generator().manual_seed(10 + rep)).cuda()
        static_B.copy_(newB)
        graph.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(static_C, ts.bsr_spmm(bsr, newB), rtol=0, atol=0)


@pytest.mark.gpu
def test_ops_reject_mismatched_arguments(hip_backend):
    """Every operator checks its tensors against the sizes and dtypes it
    passes to the kernels: a mismatched call raises before any launch."""
    import trnsparse_amd as ts
    from trnsparse_amd.hip import dispatch as D

    ops = _lib.ops()
    dev = torch.device("cuda")
    i64 = dict(dtype=torch.int64, device=dev)
    # BSR: a 256 x 256 matrix in 128-blocks, three stored blocks
    rp = torch.tensor([0, 2, 3], **i64)
    ci = torch.tensor([0, 1, 1], **i64)
    blocks = torch.randn(3, 128, 128, device=dev)
    B = torch.randn(256, 16, device=dev)
    ops.bsr_spmm(blocks, rp, ci, None, 256, 256, 128, B, torch.float32)  # the well-formed call runs
    bad_bsr = [
        lambda: ops.bsr_spmm(blocks, rp, ci, None, 256, 256, 128, B[:200], torch.float32),  # B shorter than n
        lambda: ops.bsr_spmm(blocks, rp, ci, None, 384, 256, 128, B, torch.float32),  # row_ptrs vs m
        lambda: ops.bsr_spmm(blocks, rp, ci[:2], None, 256, 256, 128, B, torch.float32),  # indices vs blocks
        lambda: ops.bsr_spmm(blocks, rp, ci, None, 256, 256, 64, B, torch.float32),  # block size vs blocks
        lambda: ops.bsr_spmm(blocks.double(), rp, ci, None, 256, 256, 128, B, torch.float32),  # dtypes differ
        lambda: ops.bsr_spmm(blocks, rp.int(), ci, None, 256, 256, 128, B, torch.float32),  # int32 pointers
        lambda: ops.bsr_spmm(blocks, rp, ci, torch.zeros(1, dtype=torch.int32, device=dev), 256, 256, 128, B,
                             torch.float32),  # row order of the wrong length
        lambda: ops.bsr_sddmm(B, B[:, :8].contiguous(), torch.zeros(3, **i64), ci, 256, 256, 128),  # N differs
        lambda: ops.bsr_spmm_t(blocks, torch.zeros(2, **i64), ci, ci, torch.empty(0, dtype=torch.int32, device=dev),
                               256, 256, 128, B),  # col_ptrs vs n
    ]
    # CSR: 10 x 20, 30 entries
    g = torch.Generator().manual_seed(0)
    dense = torch.randn(10, 20, generator=g) * (torch.rand(10, 20, generator=g) < 0.15)
    A = ts.from_dense(dense)
    vals, cols, ptrs, win = D._csr_device(A, dev)
    x = torch.randn(20, device=dev)
    ops.csr_spmv(vals, cols, ptrs, win, 10, 20, x, 1.0, None, 0.0)
    X = torch.randn(20, 4, device=dev)
    bad_csr = [
        lambda: ops.csr_spmv(vals.double(), cols, ptrs, win, 10, 20, x, 1.0, None, 0.0),  # fp64 values, fp32 x
        lambda: ops.csr_spmv(vals, cols, ptrs, win, 10, 20, x[:15], 1.0, None, 0.0),  # x shorter than n
        lambda: ops.csr_spmv(vals, cols, ptrs, win, 10, 20, x, 1.0, torch.ones(7, device=dev), 1.0),  # y vs m
        lambda: ops.csr_spmv(vals, cols.int(), ptrs, win, 10, 20, x, 1.0, None, 0.0),  # index widths differ
        lambda: ops.csr_spmv(vals, cols, ptrs, win, 12, 20, x, 1.0, None, 0.0),  # row_ptrs vs m
        lambda: ops.csr_spmm(vals, cols, ptrs, 10, 20, X[:12], 1.0, None, 0.0),  # X rows vs n
        lambda: ops.csr_spmm(vals, cols, ptrs, 10, 20, X, 1.0, torch.ones(10, 3, device=dev), 1.0),  # Y shape
    ]
    # screened: A must be square, diag and B must match it
    As = torch.randn(64, 64, device=dev)
    diag = torch.rand(64, device=dev)
    Bs = torch.randn(64, 8, device=dev)
    ops.screened_spmm(As, diag, Bs, 1e-3)
    bad_scr = [
        lambda: ops.screened_spmm(As[:, :32].contiguous(), diag, Bs, 1e-3),
        lambda: ops.screened_spmm(As, diag[:32], Bs, 1e-3),
        lambda: ops.screened_spmm(As, diag, Bs[:32], 1e-3),
        lambda: ops.screened_spmm_backward(As[:32].contiguous(), diag, Bs, 1e-3, Bs, True, True),
        lambda: ops.screened_spmm_backward(As, diag, Bs, 1e-3, Bs[:, :4].contiguous(), True, True),
    ]
    # attention: one shape and dtype for Q, K, V
    Q = torch.randn(2, 256, 64, device=dev)
    bad_attn = [
        lambda: ops.bsa_fwd(Q, Q.double(), Q, rp, ci, 128, 0.125, False),
        lambda: ops.bsa_fwd(Q, Q, Q, rp[:2], ci, 128, 0.125, False),
        lambda: ops.bsa_bwd(Q, Q, Q, Q, Q[:1], rp, ci, rp, ci, 2, 128, 0.125, torch.zeros(2, 256, device=dev),
                            torch.ones(2, 256, device=dev), torch.zeros(4, dtype=torch.int32, device=dev), 0, 0, 0),
        lambda: ops.bsa_bwd(Q, Q, Q, Q, Q, rp, ci, rp, ci, 2, 128, 0.125, torch.zeros(2, 100, device=dev),
                            torch.ones(2, 256, device=dev), torch.zeros(4, dtype=torch.int32, device=dev), 0, 0, 0),
        lambda: ops.bsa_bwd(Q, Q, Q, Q, Q, rp, ci, rp, ci, 2, 128, 0.125, torch.zeros(2, 256, device=dev),
                            torch.ones(2, 256, device=dev), torch.zeros(4, dtype=torch.int32, device=dev), 5, 0, 0),
    ]
    for i, call in enumerate(bad_bsr + bad_csr + bad_scr + bad_attn):
        with pytest.raises(RuntimeError):
            call()
    torch.cuda.synchronize()
