"""HIP graph capture of the public API on the hip backend.

A solver or training loop on MI355X captures its steady-state iteration in
a HIP graph instead of tracing it. After one eager warm-up call (which
builds and caches the per-matrix plans: row orders, CSR windows, the SpMV
column plan, the attention backward's column plan), each public op below is
captured once and replayed with new input contents; eager work and
synchronizations run between replays, and every replay must equal an eager
call on the same inputs bit for bit. Nothing inside a captured call may
synchronize with the host or record a memset (the kernels clear their own
scratch), which is what these tests would catch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import trnsparse_amd as ts
from trnsparse_amd import workloads as W
from trnsparse_amd.hip import dispatch as D

pytestmark = pytest.mark.gpu


def _capture(fn):
    """Warm fn up on a side stream, then capture it; return (graph, outputs)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out if isinstance(out, tuple) else (out,)


def _replays_match(fn, statics, fresh_sets, eager):
    graph, outs = _capture(fn)
    for fresh in fresh_sets:
        for t, v in zip(statics, fresh):
            t.copy_(v)
        graph.replay()
        torch.cuda.synchronize()
        want = eager(*fresh)
        want = want if isinstance(want, tuple) else (want,)
        torch.cuda.synchronize()
        for got, w in zip(outs, want):
            assert torch.equal(got, w)


def _csr(m, n, mean, seed):
    rng = np.random.default_rng(seed)
    v, c, p = W.random_csr(np.minimum(rng.poisson(mean, m), n), n, rng)
    return W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")


@pytest.mark.parametrize("mode", ["never", "always"])
def test_graph_spmv(hip_backend, mode):
    prev = D.get_spmv_plan()
    D.set_spmv_plan(mode)
    try:
        m, n = 30000, 25000
        A = _csr(m, n, 11, 1)
        g = torch.Generator(device="cuda").manual_seed(2)
        x = torch.randn(n, device="cuda", generator=g)
        y = torch.randn(m, device="cuda", generator=g)
        ts.spmv(A, x)  # builds the windows / the plan
        fresh = [(torch.randn(n, device="cuda", generator=g), torch.randn(m, device="cuda", generator=g))
                 for _ in range(3)]
        _replays_match(lambda: ts.spmv(A, x, alpha=0.5, y=y, beta=2.0), (x, y), fresh,
                       lambda xx, yy: ts.spmv(A, xx, alpha=0.5, y=yy, beta=2.0))
    finally:
        D.set_spmv_plan(prev)


def test_graph_spmm(hip_backend):
    m, n = 20000, 15000
    A = _csr(m, n, 9, 3)
    g = torch.Generator(device="cuda").manual_seed(4)
    B = torch.randn(n, 8, device="cuda", generator=g)
    ts.spmm(A, B)
    fresh = [(torch.randn(n, 8, device="cuda", generator=g),) for _ in range(3)]
    _replays_match(lambda: ts.spmm(A, B, alpha=1.5), (B,), fresh, lambda BB: ts.spmm(A, BB, alpha=1.5))


@pytest.mark.parametrize("dtype,out_dtype", [(torch.float32, None), (torch.bfloat16, torch.float32)])
def test_graph_bsr_spmm(hip_backend, dtype, out_dtype):
    gen = torch.Generator().manual_seed(5)
    mask = torch.rand(8, 8, generator=gen) < 0.3
    dense = torch.randn(1024, 1024, generator=gen) * mask.repeat_interleave(128, 0).repeat_interleave(128, 1)
    A = ts.BSRMatrix.from_dense(dense.to(dtype).cuda(), block_size=128)
    g = torch.Generator(device="cuda").manual_seed(6)
    B = torch.randn(1024, 96, device="cuda", generator=g).to(dtype)
    ts.bsr_spmm(A, B, out_dtype=out_dtype)
    fresh = [(torch.randn(1024, 96, device="cuda", generator=g).to(dtype),) for _ in range(3)]
    _replays_match(lambda: ts.bsr_spmm(A, B, out_dtype=out_dtype), (B,), fresh,
                   lambda BB: ts.bsr_spmm(A, BB, out_dtype=out_dtype))


def test_graph_screened_spmm(hip_backend):
    g = torch.Generator(device="cuda").manual_seed(7)
    n = 512
    A = torch.randn(n, n, device="cuda", generator=g)
    diag = 10.0 ** (-8 * torch.rand(n, device="cuda", generator=g))
    B = torch.randn(n, 64, device="cuda", generator=g)
    ts.screened_spmm(A, diag, B, 1e-6)
    fresh = [(torch.randn(n, n, device="cuda", generator=g), torch.randn(n, 64, device="cuda", generator=g))
             for _ in range(3)]
    _replays_match(lambda: ts.screened_spmm(A, diag, B, 1e-6), (A, B), fresh,
                   lambda AA, BB: ts.screened_spmm(AA, diag, BB, 1e-6))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_graph_attention_forward(hip_backend, dtype):
    S, d, heads = 1024, 128, 4
    mask = W.cfg5_block_mask(S // 128)
    bsr = W.bsr_from_block_mask(mask, 128)
    g = torch.Generator(device="cuda").manual_seed(8)
    Q, K, V = (torch.randn(heads, S, d, device="cuda", generator=g).to(dtype) for _ in range(3))
    ts.block_sparse_attention_tiled(Q, K, V, bsr)
    fresh = [tuple(torch.randn(heads, S, d, device="cuda", generator=g).to(dtype) for _ in range(3))
             for _ in range(3)]
    _replays_match(lambda: ts.block_sparse_attention_tiled(Q, K, V, bsr), (Q, K, V), fresh,
                   lambda q, k, v: ts.block_sparse_attention_tiled(q, k, v, bsr))


def _grads_replay_match(forward, leaves, gout_shape, dtype, seed):
    """Capture forward + backward (gradients of the leaves); every replay with
    new leaf and output-gradient contents equals torch.autograd.grad on
    fresh leaves."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    gout = torch.randn(gout_shape, device="cuda", generator=g).to(dtype)

    def step():
        for t in leaves:
            t.grad = None
        forward(*leaves).backward(gout)
        return tuple(t.grad for t in leaves)

    graph, grads = _capture(step)
    for _ in range(3):
        new = [torch.randn(t.shape, device="cuda", generator=g).to(dtype) for t in leaves]
        newg = torch.randn(gout_shape, device="cuda", generator=g).to(dtype)
        with torch.no_grad():
            for t, v in zip(leaves, new):
                t.copy_(v)
            gout.copy_(newg)
        graph.replay()
        torch.cuda.synchronize()
        fresh = [v.clone().requires_grad_(True) for v in new]
        want = torch.autograd.grad(forward(*fresh), fresh, newg)
        torch.cuda.synchronize()
        for got, w in zip(grads, want):
            assert torch.equal(got, w)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_graph_bsr_spmm_backward(hip_backend, dtype):
    gen = torch.Generator().manual_seed(9)
    mask = torch.rand(6, 6, generator=gen) < 0.35
    dense = torch.randn(768, 768, generator=gen) * mask.repeat_interleave(128, 0).repeat_interleave(128, 1)
    A0 = ts.BSRMatrix.from_dense(dense.to(dtype).cuda(), block_size=128)
    blocks = A0.blocks.clone().requires_grad_(True)
    B = torch.randn(768, 64, device="cuda", dtype=torch.float32).to(dtype).requires_grad_(True)

    mats = {}  # one BSRMatrix per blocks tensor: the captured one keeps its cached plans

    def forward(bl, BB):
        if id(bl) not in mats:
            mats[id(bl)] = ts.BSRMatrix(blocks=bl, block_col_indices=A0.block_col_indices,
                                        block_row_ptrs=A0.block_row_ptrs, shape=A0.shape, block_size=128)
        return ts.bsr_spmm(mats[id(bl)], BB)

    _grads_replay_match(forward, [blocks, B], (768, 64), dtype, 10)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_graph_attention_backward(hip_backend, dtype):
    S, d, heads = 1024, 128, 2
    bsr = W.bsr_from_block_mask(W.cfg5_block_mask(S // 128), 128)
    g = torch.Generator(device="cuda").manual_seed(11)
    leaves = [torch.randn(heads, S, d, device="cuda", generator=g).to(dtype).requires_grad_(True) for _ in range(3)]
    _grads_replay_match(lambda q, k, v: ts.block_sparse_attention_tiled(q, k, v, bsr), leaves, (heads, S, d), dtype,
                        12)


def test_compiled_public_ops(hip_backend):
    """torch.compile over code that calls the public ops (graph breaks at
    the planning calls are allowed; results must equal eager calls)."""
    A = _csr(20000, 15000, 9, 21)
    gen = torch.Generator().manual_seed(22)
    mask = torch.rand(4, 4, generator=gen) < 0.5
    dense = torch.randn(512, 512, generator=gen) * mask.repeat_interleave(128, 0).repeat_interleave(128, 1)
    Ab = ts.BSRMatrix.from_dense(dense.cuda(), block_size=128)
    bsr = W.bsr_from_block_mask(W.cfg5_block_mask(4), 128)
    g = torch.Generator(device="cuda").manual_seed(23)
    x = torch.randn(15000, device="cuda", generator=g)
    B = torch.randn(512, 32, device="cuda", generator=g)
    Q = torch.randn(2, 512, 128, device="cuda", generator=g).to(torch.bfloat16)

    def step(x, B, Q):
        y = ts.spmv(A, x * 2.0)
        C = ts.bsr_spmm(Ab, B) + 1.0
        O = ts.block_sparse_attention_tiled(Q, Q, Q, bsr)
        return y, C, O

    want = step(x, B, Q)
    got = torch.compile(step, backend="aot_eager")(x, B, Q)
    for a, b in zip(got, want):
        assert torch.equal(a, b)


def test_graph_spmm_backward(hip_backend):
    """Values and dense-operand gradients of the CSR product (the device
    transpose of the pattern and the SDDMM) captured with the forward."""
    m, n = 6000, 5000
    rng = np.random.default_rng(31)
    v, c, p = W.random_csr(np.minimum(rng.poisson(7, m), n), n, rng)
    cols, ptrs = torch.from_numpy(c).cuda(), torch.from_numpy(p).cuda()
    vals = torch.from_numpy(v).cuda().requires_grad_(True)
    X = torch.randn(n, 8, device="cuda").requires_grad_(True)
    mats = {}

    def forward(vv, XX):
        if id(vv) not in mats:
            mats[id(vv)] = ts.CSRMatrix(values=vv, col_indices=cols, row_ptrs=ptrs, shape=(m, n))
        return ts.spmm(mats[id(vv)], XX, alpha=0.75)

    _grads_replay_match(forward, [vals, X], (m, 8), torch.float32, 32)


def test_graph_screened_spmm_backward(hip_backend):
    g = torch.Generator(device="cuda").manual_seed(33)
    n = 384
    diag = 10.0 ** (-8 * torch.rand(n, device="cuda", generator=g))
    A = torch.randn(n, n, device="cuda", generator=g).requires_grad_(True)
    B = torch.randn(n, 48, device="cuda", generator=g).requires_grad_(True)
    _grads_replay_match(lambda AA, BB: ts.screened_spmm(AA, diag, BB, 1e-6), [A, B], (n, 48), torch.float32, 34)
