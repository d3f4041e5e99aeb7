"""GPU parity of block_sparse_attention_tiled (HIP kernels) against the oracle.

Masks follow the reference's builders (local window, dilated, global tokens;
examples/block_sparse_attention.py:49-109) and the BASELINE config-5 mask.
Error measure: |O - O_exact| / (P |V|)_ij with the float64 oracle's softmax
weights P — fp32 inputs <= 1e-4 (fp32 MFMA kernel for b = 128 and D in
{64, 128, 256}, other D below 256 zero-padded to those, generic kernel
otherwise), bf16 inputs <= 2e-2 (MFMA kernel, oracle run on the exact bf16
values). The reference's hardware test
tolerance (tests/test_nki_attn.py:63-67, atol 1e-3 / rtol 1e-4 against the
torch path) is checked for fp32 as well.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import trnsparse_amd as ts
from oracle import ref
from trnsparse_amd import workloads as W
from trnsparse_amd.hip.dispatch import hip_block_sparse_attention

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4
TOL_BF16 = 2e-2


def local_mask(nb, window):
    i = torch.arange(nb)
    return (i[:, None] - i[None, :]).abs() <= window


def dilated_mask(nb, stride):
    i = torch.arange(nb)
    return ((i[:, None] - i[None, :]) % stride) == 0


def global_mask(nb, window, n_global):
    m = local_mask(nb, window)
    m[:n_global, :] = True
    m[:, :n_global] = True
    return m


def _oracle(Q, K, V, mask_bsr, scale, rows=None):
    """(out, rmax, rden, scale_PV) per head, float64."""
    q, k, v = (t.float().cpu().numpy() for t in (Q, K, V))
    ptr, col = mask_bsr.block_row_ptrs.numpy(), mask_bsr.block_col_indices.numpy()
    out, rmax, rden = ref.block_sparse_attention(q, k, v, ptr, col, mask_bsr.block_size, scale, rows=rows)
    # error scale: same softmax weights applied to |V|
    sc, _, _ = ref.block_sparse_attention(q, k, np.abs(v), ptr, col, mask_bsr.block_size, scale, rows=rows)
    return out, rmax, rden, sc


def _err(got, exact, sc):
    return ref.scaled_error(got, exact, np.maximum(sc, 1e-30))


@pytest.mark.parametrize("S,D,mask", [
    (256, 32, local_mask(2, 1)), (256, 32, dilated_mask(2, 2)), (384, 32, global_mask(3, 1, 1)),
    (256, 32, torch.ones(2, 2, dtype=torch.bool)), (256, 256, local_mask(2, 1)), (256, 256, dilated_mask(2, 2)),
    (512, 64, local_mask(4, 2)), (512, 64, global_mask(4, 2, 2)), (384, 100, global_mask(3, 1, 1)),
    (300, 48, local_mask(3, 1)),
])
def test_fp32_reference_cases(hip_backend, S, D, mask):
    torch.manual_seed(10)
    Q, K, V = (torch.randn(S, D) for _ in range(3))
    mask_bsr = W.bsr_from_block_mask(mask, 128)
    got = ts.block_sparse_attention_tiled(Q.cuda(), K.cuda(), V.cuda(), mask_bsr).cpu()
    out, _, _, sc = _oracle(Q, K, V, mask_bsr, D**-0.5)
    assert _err(got.numpy(), out, sc) <= TOL_F32
    ts.set_backend("pytorch")
    expect = ts.block_sparse_attention_tiled(Q, K, V, mask_bsr)
    ts.set_backend("hip")
    torch.testing.assert_close(got, expect, atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("S,D,mask", [
    (512, 128, local_mask(4, 2)), (512, 64, dilated_mask(4, 2)), (1024, 128, global_mask(8, 1, 2)),
    (1024, 128, torch.ones(8, 8, dtype=torch.bool)), (640, 64, W.cfg5_block_mask(5)),
    (512, 256, local_mask(4, 2)), (1024, 256, global_mask(8, 1, 2)), (700, 256, torch.ones(6, 6, dtype=torch.bool)),
    (640, 200, W.cfg5_block_mask(5)),  # head_dim zero-padded to 256
])
def test_bf16_mfma(hip_backend, S, D, mask):
    g = torch.Generator().manual_seed(11)
    Q, K, V = (torch.randn(S, D, generator=g).bfloat16() for _ in range(3))
    mask_bsr = W.bsr_from_block_mask(mask, 128)
    got, rmax, rden = hip_block_sparse_attention(Q.cuda(), K.cuda(), V.cuda(), mask_bsr, D**-0.5, return_stats=True)
    assert got.dtype == torch.bfloat16
    out, em, ed, sc = _oracle(Q, K, V, mask_bsr, D**-0.5)
    assert _err(got.float().cpu().numpy(), out, sc) <= TOL_BF16
    np.testing.assert_allclose(rmax.cpu().numpy(), em, rtol=1e-3, atol=1e-3)
    np.testing.assert_allclose(rden.cpu().numpy(), ed, rtol=2e-2)


@pytest.mark.parametrize("S,D,mask,H", [
    (512, 128, local_mask(4, 2), 1), (1024, 128, global_mask(8, 1, 2), 9),
    (700, 128, torch.ones(6, 6, dtype=torch.bool), 2), (640, 64, W.cfg5_block_mask(5), 3),
    (300, 64, local_mask(3, 1), 1), (512, 64, torch.ones(4, 4, dtype=torch.bool), 8),
    (512, 256, local_mask(4, 2), 1), (700, 256, global_mask(6, 1, 2), 9), (640, 256, W.cfg5_block_mask(5), 2),
    (384, 136, global_mask(3, 1, 1), 1),  # head_dim zero-padded to 256
])
def test_fp32_mfma(hip_backend, S, D, mask, H):
    """fp32, b = 128, D in {64, 128, 256} runs bsa_fwd_f32_mfma: ragged S (keys
    past S inside a stored block), more heads than a multiple of 8, and
    queries with wide score ranges (the running max moves by more than the
    lazy-rescale threshold)."""
    g = torch.Generator().manual_seed(15)
    Q, K, V = (torch.randn(H, S, D, generator=g) for _ in range(3))
    Q[:, ::7] *= 8
    mask_bsr = W.bsr_from_block_mask(mask, 128)
    got, rmax, rden = hip_block_sparse_attention(Q.cuda(), K.cuda(), V.cuda(), mask_bsr, D**-0.5, return_stats=True)
    assert got.dtype == torch.float32
    for hh in range(H):
        out, em, ed, sc = _oracle(Q[hh], K[hh], V[hh], mask_bsr, D**-0.5)
        assert _err(got[hh].cpu().numpy(), out, sc) <= TOL_F32
        np.testing.assert_allclose(rmax[hh].cpu().numpy(), em, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(rden[hh].cpu().numpy(), ed, rtol=1e-4)


@pytest.mark.parametrize("D", [64, 256])
def test_fp32_mfma_long_row(hip_backend, D):
    """A block row with more than 64 stored blocks (the kernel reads the
    row's block columns 64 at a time)."""
    nb = 67
    S = nb * 128
    mask = local_mask(nb, 0)
    mask[1, :] = True
    mask_bsr = W.bsr_from_block_mask(mask, 128)
    g = torch.Generator().manual_seed(16)
    Q, K, V = (torch.randn(S, D, generator=g) for _ in range(3))
    got = ts.block_sparse_attention_tiled(Q.cuda(), K.cuda(), V.cuda(), mask_bsr).cpu()
    rows = [0, 1, 2, 66]
    out, _, _, sc = _oracle(Q, K, V, mask_bsr, D**-0.5, rows=rows)
    sel = np.concatenate([np.arange(r * 128, (r + 1) * 128) for r in rows])
    assert _err(got.numpy()[sel], out[sel], sc[sel]) <= TOL_F32


def test_empty_rows_ragged_seq_and_scale(hip_backend):
    """Empty block rows give zeros and stats (0, 1e-12); rows past
    (S // b) * b are zero; keys past S are absent; `scale` is honoured."""
    S, D = 300, 64
    g = torch.Generator().manual_seed(12)
    mask = torch.tensor([[False, False, False], [True, False, True], [True, True, True]])
    mask_bsr = W.bsr_from_block_mask(mask, 128)
    for dt, tol in ((torch.float32, TOL_F32), (torch.bfloat16, TOL_BF16)):
        Q, K, V = (torch.randn(S, D, generator=g).to(dt) for _ in range(3))
        got, rmax, rden = hip_block_sparse_attention(Q.cuda(), K.cuda(), V.cuda(), mask_bsr, 0.37, return_stats=True)
        got = got.float().cpu()
        assert torch.count_nonzero(got[:128]).item() == 0 and torch.count_nonzero(got[256:]).item() == 0
        assert torch.all(rmax[0] == 0) and torch.all(rden[0] == 1e-12)
        out, _, _, sc = _oracle(Q, K, V, mask_bsr, 0.37)
        assert _err(got.numpy(), out, sc) <= tol


def test_batched_heads(hip_backend):
    g = torch.Generator().manual_seed(13)
    H, S, D = 5, 512, 128
    Q, K, V = (torch.randn(H, S, D, generator=g).bfloat16() for _ in range(3))
    mask_bsr = W.bsr_from_block_mask(local_mask(4, 1), 128)
    got = ts.block_sparse_attention_tiled(Q.cuda(), K.cuda(), V.cuda(), mask_bsr).float().cpu()
    for hh in range(H):
        out, _, _, sc = _oracle(Q[hh], K[hh], V[hh], mask_bsr, D**-0.5)
        assert _err(got[hh].numpy(), out, sc) <= TOL_BF16


def test_backward_vs_pytorch_backend_f64(hip_backend):
    torch.manual_seed(40)
    S, D = 256, 32
    mask_bsr = W.bsr_from_block_mask(local_mask(2, 1), 128)
    Q, K, V, dO = (torch.randn(S, D, dtype=torch.float64) for _ in range(4))
    grads = {}
    for be in ("hip", "pytorch"):
        ts.set_backend(be)
        q, k, v = (t.clone().requires_grad_(True) for t in (Q, K, V))
        out = ts.block_sparse_attention_tiled(q, k, v, mask_bsr)
        out.backward(dO)
        grads[be] = (out.detach(), q.grad, k.grad, v.grad)
    ts.set_backend("hip")
    for a, b in zip(grads["hip"], grads["pytorch"]):
        torch.testing.assert_close(a, b, rtol=1e-9, atol=1e-9)


def test_gradcheck_f64(hip_backend):
    torch.manual_seed(41)
    S, D = 256, 16
    mask_bsr = W.bsr_from_block_mask(dilated_mask(2, 2), 128)
    Q, K, V = (torch.randn(S, D, dtype=torch.float64, device="cuda", requires_grad=True) for _ in range(3))
    assert torch.autograd.gradcheck(lambda q, k, v: ts.block_sparse_attention_tiled(q, k, v, mask_bsr), (Q, K, V),
                                    eps=1e-4, atol=1e-3, rtol=1e-3)


def test_cfg5_full_size_sampled(hip_backend):
    Q, K, V, mask_bsr = W.cfg5_attention()
    assert mask_bsr.n_blocks == 370
    got = ts.block_sparse_attention_tiled(Q.cuda(), K.cuda(), V.cuda(), mask_bsr)
    assert got.shape == (32, 8192, 128) and got.dtype == torch.bfloat16
    rows = [0, 1, 4, 5, 33, 63]
    for hh in (0, 17, 31):
        out, _, _, sc = _oracle(Q[hh], K[hh], V[hh], mask_bsr, 128**-0.5, rows=rows)
        sel = np.concatenate([np.arange(r * 128, (r + 1) * 128) for r in rows])
        assert _err(got[hh].float().cpu().numpy()[sel], out[sel], sc[sel]) <= TOL_BF16


def test_cfg5_full_size_every_row(hip_backend):
    """Whole-output check at full size, every (head, row, column): O of all
    32 heads against a float64 P.V over each block row's stored blocks on
    the CPU (bf16 bar, relative to P.|V|), the saved row_max / row_denom of
    all heads against the same pass, and V = 1 giving O = 1 on every row
    (all of cfg5's block rows hold blocks)."""
    from trnsparse_amd.hip.dispatch import hip_block_sparse_attention

    Q, K, V, mask_bsr = W.cfg5_attention()
    H, S, D = Q.shape
    scale = D**-0.5
    ones = torch.ones_like(V).cuda()
    O1 = ts.block_sparse_attention_tiled(Q.cuda(), K.cuda(), ones, mask_bsr)
    assert (O1.float() - 1.0).abs().max().item() <= TOL_BF16
    del O1, ones
    O, rm, rd = hip_block_sparse_attention(Q.cuda(), K.cuda(), V.cuda(), mask_bsr, scale, return_stats=True)
    O = O.double().cpu()
    rm = rm.double().cpu().reshape(H, S)
    rd = rd.double().cpu().reshape(H, S)
    ptr, col = mask_bsr.block_row_ptrs.tolist(), mask_bsr.block_col_indices.tolist()
    q64, k64, v64 = Q.double(), K.double(), V.double()
    worst = 0.0
    for i in range(S // 128):
        cols = col[ptr[i]:ptr[i + 1]]
        keys = torch.cat([k64[:, c * 128:(c + 1) * 128] for c in cols], dim=1)   # (H, nb*128, D)
        vals = torch.cat([v64[:, c * 128:(c + 1) * 128] for c in cols], dim=1)   # (H, nb*128, D)
        s = scale * torch.bmm(q64[:, i * 128:(i + 1) * 128], keys.transpose(1, 2).contiguous())
        mx = s.max(dim=2).values
        e = torch.exp(s - mx[..., None])
        den = e.sum(dim=2)
        sl = slice(i * 128, (i + 1) * 128)
        assert (rm[:, sl] - mx).abs().max().item() <= 1e-4 * (1.0 + mx.abs().max().item()), i
        assert ((rd[:, sl] - den).abs() / den).max().item() <= 1e-4, i
        P = e / den[..., None]
        exact = torch.bmm(P, vals)                     # (H, 128, D)
        bound = torch.bmm(P, vals.abs()).clamp_min(1e-30)
        err = ((O[:, sl] - exact).abs() / bound).max().item()
        worst = max(worst, err)
        assert err <= TOL_BF16, (i, err)
    assert worst > 0.0  # the check compared real values


def test_fp16_widened(hip_backend):
    """fp16 Q/K/V run the fp32 kernels on widened operands: O comes back in
    fp16 within the 16-bit tolerance, and the backward gives fp16 gradients."""
    S, D = 512, 64
    g = torch.Generator().manual_seed(17)
    mask_bsr = W.bsr_from_block_mask(global_mask(4, 1, 1), 128)
    Q, K, V = (torch.randn(S, D, generator=g).half() for _ in range(3))
    got = ts.block_sparse_attention_tiled(Q.cuda(), K.cuda(), V.cuda(), mask_bsr)
    assert got.dtype == torch.float16
    out, _, _, sc = _oracle(Q, K, V, mask_bsr, D**-0.5)
    assert _err(got.float().cpu().numpy(), out, sc) <= TOL_BF16
    q, k, v = (t.cuda().requires_grad_(True) for t in (Q, K, V))
    ts.block_sparse_attention_tiled(q, k, v, mask_bsr).float().sum().backward()
    assert q.grad.dtype == torch.float16 and torch.isfinite(q.grad.float()).all()


@pytest.mark.parametrize("mask,seed", [(local_mask(4, 2), 50), (dilated_mask(4, 2), 51)])
def test_reference_head_dim_256_case(hip_backend, mask, seed):
    """The reference's head_dim-256 hardware case (tests/test_nki_attn.py:
    153-201): fp32, seq 512, 128-blocks, local window 2 and dilated stride 2,
    forward and backward against the torch path at atol 1e-3 / rtol 1e-4,
    and against the float64 oracle."""
    from oracle import ref as R

    torch.manual_seed(seed)
    S, D = 512, 256
    Q, K, V = (torch.randn(S, D) for _ in range(3))
    mask_bsr = W.bsr_from_block_mask(mask, 128)
    ts.set_backend("pytorch")
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (Q, K, V))
    expect = ts.block_sparse_attention_tiled(qr, kr, vr, mask_bsr)
    dO = torch.randn_like(expect)
    expect.backward(dO)
    ts.set_backend("hip")
    qg, kg, vg = (t.cuda().requires_grad_(True) for t in (Q, K, V))
    got = ts.block_sparse_attention_tiled(qg, kg, vg, mask_bsr)
    got.backward(dO.cuda())
    torch.testing.assert_close(got.detach().cpu(), expect.detach(), atol=1e-3, rtol=1e-4)
    for a, b in ((qg, qr), (kg, kr), (vg, vr)):
        torch.testing.assert_close(a.grad.cpu(), b.grad, atol=1e-3, rtol=1e-4)
    out, _, _, sc = _oracle(Q, K, V, mask_bsr, D**-0.5)
    assert _err(got.detach().cpu().numpy(), out, sc) <= TOL_F32
    args = (Q.double().numpy(), K.double().numpy(), V.double().numpy(), got.detach().cpu().double().numpy(),
            dO.double().numpy(), mask_bsr.block_row_ptrs.numpy(), mask_bsr.block_col_indices.numpy(), 128, D**-0.5)
    exact = R.block_sparse_attention_backward(*args)
    bound = R.block_sparse_attention_backward(*args, absolute=True)
    for gr, e, a in zip((qg.grad, kg.grad, vg.grad), exact, bound):
        assert R.scaled_error(gr.cpu().double().numpy(), e, np.maximum(a, 1e-30)) <= TOL_F32


# ------------------------------------------------ bf16 head_dim 512, one pass


@pytest.mark.parametrize("S,D,mask,H", [
    (640, 512, W.cfg5_block_mask(5), 3),
    (512, 512, local_mask(4, 2), 9),                     # heads past a multiple of 8
    (700, 512, global_mask(6, 1, 2), 2),                 # ragged S: the last key block crosses it
    (512, 384, global_mask(4, 1, 1), 2),                 # zero-padded to 512
    (384, 264, torch.tensor([[True, False, True], [False, False, False], [True, True, True]]), 1),  # empty row
])
def test_bf16_d512_forward(hip_backend, S, D, mask, H):
    """bf16 with 256 < head_dim <= 512 runs the one-pass kernel in which the
    two wavefronts of a pair split the head dimension and add their partial
    scores through LDS: O and the stats of every head against the oracle,
    with wide score ranges (rows of Q scaled by 6) so the running max
    moves."""
    g = torch.Generator().manual_seed(62 + D)
    Q, K, V = (torch.randn(H, S, D, generator=g).to(torch.bfloat16) for _ in range(3))
    Q[:, ::5] *= 6
    mask_bsr = W.bsr_from_block_mask(mask, 128)
    got, rmax, rden = hip_block_sparse_attention(Q.cuda(), K.cuda(), V.cuda(), mask_bsr, D**-0.5, return_stats=True)
    assert got.dtype == torch.bfloat16 and got.shape == (H, S, D)
    Mt = S // 128
    for hh in range(H):
        out, em, ed, sc = _oracle(Q[hh], K[hh], V[hh], mask_bsr, D**-0.5)
        assert _err(got[hh].float().cpu().numpy(), out, sc) <= TOL_BF16
        np.testing.assert_allclose(rmax[hh].cpu().numpy(), em[:Mt], rtol=1e-4, atol=2e-2)
        np.testing.assert_allclose(rden[hh].cpu().numpy(), ed[:Mt], rtol=3e-2)


# ------------------------------------------- head_dim over 256: block products


@pytest.mark.parametrize("S,D,mask,H,dt", [
    (512, 512, local_mask(4, 2), 1, torch.float32),
    (512, 512, dilated_mask(4, 2), 2, torch.float32),
    (640, 640, W.cfg5_block_mask(5), 3, torch.bfloat16),
    (512, 768, global_mask(4, 1, 1), 2, torch.bfloat16),
    (256, 300, local_mask(2, 1), 1, torch.float32),   # head_dim zero-padded to 304
    (384, 1024, torch.ones(3, 3, dtype=torch.bool), 1, torch.float32),
])
def test_block_products_forward(hip_backend, S, D, mask, H, dt):
    """head_dim over 256 (fp32, and bf16 over 512; 128-blocks, whole blocks)
    runs as SDDMM scores, the block softmax and a BSR SpMM with V over the
    mask stacked over heads: O and the stats of every head against the
    oracle."""
    g = torch.Generator().manual_seed(60)
    Q, K, V = (torch.randn(H, S, D, generator=g).to(dt) for _ in range(3))
    Q[:, ::5] *= 6  # wide score ranges
    mask_bsr = W.bsr_from_block_mask(mask, 128)
    got, rmax, rden = hip_block_sparse_attention(Q.cuda(), K.cuda(), V.cuda(), mask_bsr, D**-0.5, return_stats=True)
    assert got.dtype == dt and got.shape == (H, S, D)
    tol = TOL_F32 if dt == torch.float32 else TOL_BF16
    for hh in range(H):
        out, em, ed, sc = _oracle(Q[hh], K[hh], V[hh], mask_bsr, D**-0.5)
        assert _err(got[hh].float().cpu().numpy(), out, sc) <= tol
        np.testing.assert_allclose(rmax[hh].cpu().numpy(), em, rtol=1e-4, atol=1e-4 if dt == torch.float32 else 2e-2)
        np.testing.assert_allclose(rden[hh].cpu().numpy(), ed, rtol=1e-4 if dt == torch.float32 else 3e-2)


def test_block_products_empty_rows_and_columns_past_seq(hip_backend):
    """Block products with an empty block row (zeros, stats 0 and 1e-12)
    and a mask wider than the sequence (its block columns past S hold no
    keys)."""
    S, D = 384, 320
    mask = torch.tensor([[True, False, False, True], [False, False, False, False], [True, True, True, True],
                         [True, True, True, True]])
    mask_bsr = W.bsr_from_block_mask(mask, 128)
    g = torch.Generator().manual_seed(61)
    Q, K, V = (torch.randn(S, D, generator=g) for _ in range(3))
    got, rmax, rden = hip_block_sparse_attention(Q.cuda(), K.cuda(), V.cuda(), mask_bsr, 0.05, return_stats=True)
    got = got.cpu()
    assert torch.count_nonzero(got[128:256]).item() == 0
    assert torch.all(rmax[1] == 0) and torch.all(rden[1] == 1e-12)
    # the oracle on the mask cut to the sequence's 3 block columns
    cut = W.bsr_from_block_mask(mask[:3, :3], 128)
    out, em, ed, sc = _oracle(Q, K, V, cut, 0.05)
    assert _err(got.numpy(), out, sc) <= TOL_F32
    np.testing.assert_allclose(rmax.cpu().numpy(), em, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("mask,seed", [(local_mask(4, 2), 52), (dilated_mask(4, 2), 53)])
def test_reference_large_head_dim_case_512(hip_backend, mask, seed):
    """The reference's large-head_dim hardware case (tests/test_nki_attn.py:
    153-201, K-tiled head_dim; the reference supports 256 and 512,
    trnsparse/nki/dispatch.py:515-518) at head_dim 512: fp32, seq 512,
    forward and backward against the torch path at atol 1e-3 / rtol 1e-4."""
    torch.manual_seed(seed)
    S, D = 512, 512
    Q, K, V = (torch.randn(S, D) for _ in range(3))
    mask_bsr = W.bsr_from_block_mask(mask, 128)
    ts.set_backend("pytorch")
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (Q, K, V))
    ref_out = ts.block_sparse_attention_tiled(qr, kr, vr, mask_bsr)
    dO = torch.randn_like(ref_out)
    ref_out.backward(dO)
    ts.set_backend("hip")
    q, k, v = (t.cuda().requires_grad_(True) for t in (Q, K, V))
    out = ts.block_sparse_attention_tiled(q, k, v, mask_bsr)
    out.backward(dO.cuda())
    torch.testing.assert_close(out.detach().cpu(), ref_out.detach(), atol=1e-3, rtol=1e-4)
    for got, want in ((q.grad, qr.grad), (k.grad, kr.grad), (v.grad, vr.grad)):
        torch.testing.assert_close(got.cpu(), want, atol=1e-3, rtol=1e-4)
