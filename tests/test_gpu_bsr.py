"""GPU parity of bsr_spmm (HIP kernels via the C ABI) against the CPU oracle.

Tolerances: fp32 max error <= 1e-4 and bf16 inputs
<= 2e-2, both measured relative to the dot-product scale (|A|.|B|)_ij; the
reference's own hardware tolerance (tests/test_nki_bsr.py:19, atol 1e-3,
rtol 1e-4 vs dense A@B) is checked as well for fp32.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import trnsparse_amd as ts
from oracle import ref
from trnsparse_amd import workloads as W

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4
TOL_BF16 = 2e-2


def _oracle(A: ts.BSRMatrix, B: torch.Tensor, rows=None):
    blocks = A.blocks.float().cpu().numpy() if A.dtype == torch.bfloat16 else A.blocks.cpu().numpy()
    Bn = B.float().cpu().numpy() if B.dtype == torch.bfloat16 else B.cpu().numpy()
    col = A.block_col_indices.cpu().numpy()
    ptr = A.block_row_ptrs.cpu().numpy()
    if rows is not None:  # restrict to a subset of block rows (full-size checks)
        keep_blocks = np.concatenate([np.arange(ptr[i], ptr[i + 1]) for i in rows])
        sub_ptr = np.zeros(len(rows) + 1, np.int64)
        sub_ptr[1:] = np.cumsum([ptr[i + 1] - ptr[i] for i in rows])
        blocks, col, ptr = blocks[keep_blocks], col[keep_blocks], sub_ptr
        shape = (len(rows) * A.block_size, A.shape[1])
    else:
        shape = A.shape
    exact = ref.bsr_spmm(blocks, col, ptr, shape, A.block_size, Bn)
    scale = ref.bsr_spmm(blocks, col, ptr, shape, A.block_size, Bn, absolute=True)
    return exact, scale


def _block_random(m_blocks, n_blocks, b, density, seed):
    torch.manual_seed(seed)
    A = torch.zeros(m_blocks * b, n_blocks * b)
    mask = torch.rand(m_blocks, n_blocks) < density
    for i in range(m_blocks):
        for j in range(n_blocks):
            if mask[i, j]:
                A[i * b : (i + 1) * b, j * b : (j + 1) * b] = torch.randn(b, b)
    return A


# reference grid: tests/test_nki_bsr.py:44-51 (seed 42)
@pytest.mark.parametrize("m_blocks,n_blocks,N,density", [(2, 2, 128, 0.5), (4, 4, 128, 0.25), (3, 3, 256, 0.5), (4, 2, 128, 0.5)])
def test_reference_grid(hip_backend, m_blocks, n_blocks, N, density):
    A = _block_random(m_blocks, n_blocks, 128, density, seed=42)
    bsr = ts.BSRMatrix.from_dense(A, block_size=128)
    B = torch.randn(n_blocks * 128, N)
    got = ts.bsr_spmm(bsr, B.cuda())
    assert got.is_cuda and got.dtype == torch.float32 and got.shape == (m_blocks * 128, N)
    exact, scale = _oracle(bsr, B)
    assert ref.scaled_error(got.cpu().numpy(), exact, scale) <= TOL_F32
    torch.testing.assert_close(got.cpu(), A @ B, atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize(
    "shape,b,N,density",
    [
        ((24, 24), 8, 16, 0.5),  # reference tests/test_bsr.py:68-74 (b = 8: 4x4x1 MFMA kernel)
        ((20, 14), 8, 10, 1.0),  # unaligned, :76-83
        ((40, 40), 8, 12, 0.1),  # sparse, :85-93
        ((200, 137), 128, 64, 1.0),  # unaligned 128-blocks (MFMA kernel bounds)
        ((300, 260), 128, 10, 1.0),  # N not a multiple of 4 (padded B panels)
        ((300, 260), 128, 11, 1.0),  # odd N: the fp32 kernel's unpaired last-column stores
        ((256, 384), 128, 129, 0.7),  # odd N past one column tile
        ((384, 256), 128, 200, 0.6),  # partial column tile
        ((256, 256), 64, 96, 0.7),  # block size 64 (small-block MFMA kernel)
    ],
)
def test_shapes(hip_backend, shape, b, N, density):
    g = torch.Generator().manual_seed(11)
    A = torch.randn(*shape, generator=g) * (torch.rand(*shape, generator=g) < density)
    bsr = ts.BSRMatrix.from_dense(A, block_size=b)
    B = torch.randn(shape[1], N, generator=g)
    got = ts.bsr_spmm(bsr, B.cuda()).cpu()
    exact, scale = _oracle(bsr, B)
    assert got.shape == (shape[0], N)
    assert ref.scaled_error(got.numpy(), exact, scale) <= TOL_F32


@pytest.mark.parametrize(
    "shape,b,N,density",
    [
        ((64, 64), 8, 64, 0.6),       # b = 8: whole tiles
        ((200, 150), 8, 37, 0.5),     # b = 8: ragged m, n, partial column tile
        ((96, 96), 8, 130, 0.4),      # b = 8: three column tiles, the last partial
        ((330, 260), 8, 1000, 0.4),   # b = 8: 16 column tiles
        ((64, 1024), 8, 96, 0.9),     # b = 8: long block rows (over 100 blocks)
        ((200, 150), 8, 256, 0.5),    # b = 8: 16-byte B rows, the last block column past n element-wise
        ((136, 136), 8, 384, 0.7),    # b = 8: three full 128-column tiles
        ((64, 64), 16, 64, 0.6),      # whole tiles
        ((200, 150), 16, 37, 0.5),    # ragged m, n (B rows past n read as zero), partial column tile
        ((96, 96), 32, 130, 0.4),     # three column tiles, the last partial
        ((150, 301), 32, 5, 0.8),     # narrow N
        ((320, 200), 64, 200, 0.3),   # ragged n inside a block column
        ((128, 2048), 64, 64, 0.9),   # long block rows (32 blocks)
        ((200, 150), 16, 512, 0.5),   # 8 column tiles, 13 block rows
        ((330, 260), 32, 1000, 0.4),  # 16 column tiles, the last partial
        ((256, 512), 64, 512, 0.3),
    ],
)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_small_block_mfma(hip_backend, shape, b, N, density, dtype):
    """b in {8, 16, 32, 64} runs bsr_spmm_small (fp32 MFMA; bf16 widened at the
    load), with empty block rows mixed in; fp32 out for fp32, bf16 in -> fp32
    and bf16 out."""
    g = torch.Generator().manual_seed(b + N)
    A = torch.randn(*shape, generator=g) * (torch.rand(*shape, generator=g) < density)
    A[b : 2 * b] = 0.0                                  # an empty block row
    A = A.to(dtype).float()
    bsr = ts.BSRMatrix.from_dense(A.to(dtype), block_size=b)
    B = torch.randn(shape[1], N, generator=g).to(dtype)
    exact, scale = _oracle(ts.BSRMatrix.from_dense(A, block_size=b), B.float())
    got = ts.bsr_spmm(bsr, B.cuda(), out_dtype=torch.float32).cpu()
    assert got.dtype == torch.float32 and got.shape == (shape[0], N)
    assert ref.scaled_error(got.numpy(), exact, scale) <= TOL_F32
    assert torch.count_nonzero(got[b : 2 * b]).item() == 0
    if dtype == torch.bfloat16:
        got16 = ts.bsr_spmm(bsr, B.cuda()).cpu()
        assert got16.dtype == torch.bfloat16
        assert ref.scaled_error(got16.float().numpy(), exact, scale) <= 1e-2


def test_empty_pattern_is_zero(hip_backend):
    A = torch.zeros(256, 256)
    bsr = ts.BSRMatrix.from_dense(A, block_size=128)
    assert bsr.n_blocks == 0
    got = ts.bsr_spmm(bsr, torch.randn(256, 64).cuda())
    assert torch.count_nonzero(got).item() == 0


def test_empty_rows_and_cpu_inputs(hip_backend):
    """Block rows without blocks give zeros; host inputs come back on the host."""
    A = _block_random(4, 4, 128, 0.5, seed=3)
    A[128:256] = 0.0
    bsr = ts.BSRMatrix.from_dense(A, block_size=128)
    B = torch.randn(512, 128)
    got = ts.bsr_spmm(bsr, B)
    assert got.device.type == "cpu"
    assert torch.count_nonzero(got[128:256]).item() == 0
    exact, scale = _oracle(bsr, B)
    assert ref.scaled_error(got.numpy(), exact, scale) <= TOL_F32


def test_f64_generic(hip_backend):
    A = _block_random(2, 3, 16, 0.6, seed=5).double()
    bsr = ts.BSRMatrix.from_dense(A, block_size=16)
    B = torch.randn(48, 7, dtype=torch.float64)
    got = ts.bsr_spmm(bsr, B.cuda()).cpu()
    torch.testing.assert_close(got, A @ B, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize(
    "shape,N,density",
    [((512, 384), 256, 0.5),     # fp64 MFMA kernel, aligned
     ((300, 260), 130, 0.6),     # ragged m, n, N (B rows past n read as zero, N padded to even)
     ((384, 512), 7, 1.0),       # narrow N
     ((256, 256), 128, 0.0)],    # empty pattern
)
def test_f64_mfma(hip_backend, shape, N, density):
    """fp64 with block size 128 runs v_mfma_f64_16x16x4_f64; against the
    float64 oracle within 1e-12 of the dot-product scale."""
    g = torch.Generator().manual_seed(shape[0] + N)
    A = torch.randn(*shape, generator=g, dtype=torch.float64) * (torch.rand(*shape, generator=g) < density)
    bsr = ts.BSRMatrix.from_dense(A, block_size=128)
    B = torch.randn(shape[1], N, generator=g, dtype=torch.float64)
    got = ts.bsr_spmm(bsr, B.cuda()).cpu()
    assert got.dtype == torch.float64 and got.shape == (shape[0], N)
    if bsr.n_blocks == 0:
        assert torch.count_nonzero(got).item() == 0
        return
    exact, scale = _oracle(bsr, B)
    assert ref.scaled_error(got.numpy(), exact[: shape[0]], scale[: shape[0]]) <= 1e-12


def test_f64_mfma_empty_rows_and_cfg3_rows(hip_backend):
    """cfg3's pattern in fp64 (32 block rows): every row against the oracle;
    block rows without blocks give exact zeros."""
    A, B = W.cfg3_bsr(nb=32, ncols=256, dtype=torch.float64)
    got = ts.bsr_spmm(A, B.cuda()).cpu()
    exact, scale = _oracle(A, B)
    assert ref.scaled_error(got.numpy(), exact, scale) <= 1e-12
    mask = torch.tensor([[True, False, True], [False, False, False], [False, True, False]])
    E = W.bsr_from_block_mask(mask, 128, blocks=torch.randn(3, 128, 128, dtype=torch.float64))
    Bz = torch.randn(384, 64, dtype=torch.float64)
    out = ts.bsr_spmm(E, Bz.cuda()).cpu()
    assert torch.count_nonzero(out[128:256]).item() == 0
    ex, sc = _oracle(E, Bz)
    assert ref.scaled_error(out.numpy(), ex, sc) <= 1e-12


def test_dtype_mismatch_raises(hip_backend):
    bsr = ts.BSRMatrix.from_dense(torch.randn(128, 128), block_size=128)
    with pytest.raises(RuntimeError):
        ts.bsr_spmm(bsr, torch.randn(128, 8, dtype=torch.float64).cuda())
    with pytest.raises(AssertionError):
        ts.bsr_spmm(bsr, torch.randn(64, 8).cuda())


def _f64_pass(A: ts.BSRMatrix, B: torch.Tensor):
    """(exact, scale) = (A @ B, |A| @ |B|) over every block row in float64
    on the CPU: per block row, its stored blocks side by side times the
    matching B row panels stacked (torch float64 matmuls, independent of
    the numpy oracle's loop)."""
    b = A.block_size
    blocks = A.blocks.double()
    B64 = B.double()
    ptr, col = A.block_row_ptrs.tolist(), A.block_col_indices.tolist()
    m = A.shape[0]
    exact = torch.zeros(m, B.shape[1], dtype=torch.float64)
    scale = torch.zeros(m, B.shape[1], dtype=torch.float64)
    for i in range(len(ptr) - 1):
        k0, k1 = ptr[i], ptr[i + 1]
        if k0 == k1:
            continue
        arow = blocks[k0:k1].permute(1, 0, 2).reshape(b, (k1 - k0) * b)          # [A_i,c0 | A_i,c1 | ...]
        panels = torch.cat([B64[c * b:(c + 1) * b] for c in col[k0:k1]], dim=0)  # [B_c0; B_c1; ...]
        r1 = min(m, (i + 1) * b)
        exact[i * b:r1] = (arow @ panels)[: r1 - i * b]
        scale[i * b:r1] = (arow.abs() @ panels.abs())[: r1 - i * b]
    return exact, scale


def _whole_output_error(got: torch.Tensor, exact: torch.Tensor, scale: torch.Tensor) -> float:
    return ((got.double().cpu() - exact).abs() / scale.clamp_min(1e-30)).max().item()


def test_cfg1_plumbing(hip_backend):
    A, B, Ad = W.cfg1_bsr_plumbing()
    assert A.n_blocks == 24
    got = ts.bsr_spmm(A, B.cuda()).cpu()
    exact, scale = _oracle(A, B)
    assert ref.scaled_error(got.numpy(), exact, scale) <= TOL_F32


def test_cfg3_fp32_full_size(hip_backend):
    """16384^2, 10% block density, N=512: every element of C against a
    float64 pass over all 128 block rows, plus 16 block rows against the
    numpy oracle and the full-size checksum property
    sum(C) = colsum(A) . rowsum(B)."""
    A, B = W.cfg3_bsr()
    C = ts.bsr_spmm(A, B.cuda())
    exact64, scale64 = _f64_pass(A, B)
    assert _whole_output_error(C, exact64, scale64) <= TOL_F32
    rows = list(range(0, 128, 16)) + [1, 126, 127]
    exact, scale = _oracle(A, B, rows=rows)
    got = torch.cat([C[r * 128 : (r + 1) * 128] for r in rows]).cpu().numpy()
    assert ref.scaled_error(got, exact, scale) <= TOL_F32
    # linearity: C @ 1 = A @ (B @ 1) for every row, at full size
    ones = torch.ones(B.shape[1], 1, dtype=torch.float64)
    lhs = C.double().cpu() @ ones
    rhs = ts.bsr_spmm(A, (B.double() @ ones).float().cuda()).double().cpu()
    sc = torch.from_numpy(ref.bsr_spmm(A.blocks.numpy(), A.block_col_indices.numpy(), A.block_row_ptrs.numpy(), A.shape, 128, np.abs(B.numpy()).sum(1, keepdims=True), absolute=True))
    assert ((lhs - rhs).abs() / sc.clamp_min(1e-30)).max().item() <= TOL_F32


def test_repeat_calls_are_deterministic(hip_backend):
    A, B = W.cfg3_bsr(nb=32, ncols=256)
    Bd = B.cuda()
    c1 = ts.bsr_spmm(A, Bd)
    c2 = ts.bsr_spmm(A, Bd)
    assert torch.equal(c1, c2)


# ------------------------------------------------------------------ bf16


@pytest.mark.parametrize("out_dtype", [None, torch.float32])
@pytest.mark.parametrize(
    "shape,N,density",
    [((256, 256), 128, 0.5), ((512, 512), 256, 0.25), ((384, 384), 512, 0.5), ((512, 256), 128, 0.5),
     ((200, 137), 64, 1.0), ((300, 260), 10, 1.0), ((384, 256), 200, 0.6)],
)
def test_bf16_mfma(hip_backend, shape, N, density, out_dtype):
    g = torch.Generator().manual_seed(21)
    A = (torch.randn(*shape, generator=g) * (torch.rand(*shape, generator=g) < density)).bfloat16()
    bsr = ts.BSRMatrix.from_dense(A, block_size=128)
    B = torch.randn(shape[1], N, generator=g).bfloat16()
    got = ts.bsr_spmm(bsr, B.cuda(), out_dtype=out_dtype).cpu()
    assert got.dtype == (out_dtype or torch.bfloat16) and got.shape == (shape[0], N)
    exact, scale = _oracle(bsr, B)
    assert ref.scaled_error(got.float().numpy(), exact, scale) <= TOL_BF16
    if out_dtype == torch.float32:  # fp32 accumulation of exact bf16 products: near fp32 accuracy
        assert ref.scaled_error(got.numpy(), exact, scale) <= TOL_F32


def test_cfg3b_bf16_full_size(hip_backend):
    A, B = W.cfg3_bsr(dtype=torch.bfloat16)
    C = ts.bsr_spmm(A, B.cuda(), out_dtype=torch.float32)
    assert C.dtype == torch.float32 and C.shape == (16384, 512)
    # every element against a float64 pass over the exact bf16 values: fp32
    # accumulation of exact bf16 products holds the fp32 bar
    exact64, scale64 = _f64_pass(A, B)
    assert _whole_output_error(C, exact64, scale64) <= TOL_F32
    rows = list(range(3, 128, 16)) + [0, 127]
    exact, scale = _oracle(A, B, rows=rows)
    got = torch.cat([C[r * 128 : (r + 1) * 128] for r in rows]).cpu().numpy()
    assert ref.scaled_error(got, exact, scale) <= TOL_F32
    # linearity over every row at full size: C @ 1 = A @ (B @ 1), the right
    # side through the fp32 kernel on the exactly widened blocks
    ones = torch.ones(B.shape[1], 1, dtype=torch.float64)
    lhs = C.double().cpu() @ ones
    A32 = ts.BSRMatrix(A.blocks.float(), A.block_col_indices, A.block_row_ptrs, A.shape, 128)
    rhs = ts.bsr_spmm(A32, (B.double() @ ones).float().cuda()).double().cpu()
    sc = torch.from_numpy(ref.bsr_spmm(A32.blocks.numpy(), A.block_col_indices.numpy(), A.block_row_ptrs.numpy(),
                                       A.shape, 128, np.abs(B.float().numpy()).sum(1, keepdims=True), absolute=True))
    assert ((lhs - rhs).abs() / sc.clamp_min(1e-30)).max().item() <= TOL_F32


def test_fp16_widened(hip_backend):
    """fp16 blocks and B run the fp32 kernel on widened operands; the result
    and the autograd gradients come back in fp16."""
    g = torch.Generator().manual_seed(21)
    A = torch.randn(256, 384, generator=g) * (torch.rand(256, 384, generator=g) < 0.5)
    bsr = ts.BSRMatrix.from_dense(A.half(), block_size=128)
    B = torch.randn(384, 96, generator=g).half()
    C = ts.bsr_spmm(bsr, B.cuda())
    assert C.dtype == torch.float16
    exact = A.half().double() @ B.double()
    scale = A.half().double().abs() @ B.double().abs()
    assert ((C.double().cpu() - exact).abs() / scale.clamp_min(1e-30)).max().item() <= 2e-2
    blocks = bsr.blocks.cuda().requires_grad_(True)
    Bd = B.cuda().requires_grad_(True)
    ts.bsr_spmm(ts.BSRMatrix(blocks, bsr.block_col_indices, bsr.block_row_ptrs, bsr.shape, 128), Bd).float().sum().backward()
    assert blocks.grad.dtype == torch.float16 and Bd.grad.dtype == torch.float16
