"""CPU oracle for the trnsparse compute path — TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import this package, and only as the checker. The product
(`trnsparse_amd`) never imports, calls or links anything here.

Each function restates the reference semantics in numpy, accumulating in
float64, so the GPU result can be judged against the exact value with a
tolerance scaled by |A|.|B| (the dot-product error scale). Citations point
into the reference tree (trnsci/trnsparse).

How each function is pinned (tests/test_oracle.py):
- bsr_from_dense / bsr_to_dense: brute-force per-block loops on tiny grids,
  round trips, the empty-matrix case, padding of unaligned shapes.
- bsr_spmm: closed form to_dense(A) @ B (numpy matmul), empty pattern -> 0.
- csr_from_dense: scipy.sparse (independent) for positive thresholds, a
  brute-force double loop for negative ones (zeros kept) and NaN entries.
- coo_to_csr: scipy.sparse for distinct coordinates, a brute-force sort of
  (row, col, position) tuples with duplicates.
- coo_sum_to_csr / sparse_add / csr_transpose / spmv_symmetric: scipy.sparse
  sums and transposes (canonical: duplicates summed, sorted), a dense
  (A + strict(A)^T) @ x for the symmetric SpMV.
- bsr_spmm_backward: torch float64 autograd through the dense product
  to_dense(A) @ B (dA read back on the stored blocks), empty pattern -> 0.
- csr_spmv / csr_spmm: scipy.sparse (independent implementation), the
  reference's known answers [9, 16] and 7.0 (tests/test_ops.py:25-32, 61-67),
  identity.
- screened_mask / screened_spmm: threshold 0 -> A@B, 1e30 -> exact zeros,
  hand-built values straddling fl32(1e-10) (torch's fp32 compare).
- block_sparse_attention: dense masked softmax (numpy), a full mask equals
  dense attention, empty block rows give zeros.
- chebyshev_coeffs / chebyshev / richardson: closed forms — the
  reference's recurrence gives alpha_k = (2/c) U_k(s)/U_{k+1}(s), beta_k =
  U_{k-1}(s)/U_{k+1}(s) (s = d/c, U: Chebyshev polynomials of the second
  kind) and the residual polynomial U_K((d - lam)/c) / U_K(s); both solvers
  on diagonal matrices against their closed-form iterates.
- block_sparse_attention_backward: torch float64 autograd through a dense
  masked softmax attention (empty block rows and rows past S // b give zero
  output there, keys past S absent), on full, local, ragged and
  empty-row masks; the absolute form bounds the signed one.
"""

from __future__ import annotations

import math

import numpy as np

# ------------------------------------------------------------------ BSR


def bsr_from_dense(A: np.ndarray, b: int, threshold: float = 0.0):
    """(blocks, col_idx, row_ptrs, shape) as formats.py:183-221 builds them.

    Pad to a block multiple; block (i, j) is kept iff max|v| > threshold;
    blocks are listed row-major (block columns ascending within a row).
    """
    m, n = A.shape
    mp, np_ = -(-m // b) * b, -(-n // b) * b
    P = np.zeros((mp, np_), dtype=A.dtype)
    P[:m, :n] = A
    mb, nbc = mp // b, np_ // b
    grid = P.reshape(mb, b, nbc, b).transpose(0, 2, 1, 3)
    keep = np.abs(grid).max(axis=(2, 3)) > threshold if mb and nbc else np.zeros((mb, nbc), bool)
    row_ptrs = np.zeros(mb + 1, dtype=np.int64)
    row_ptrs[1:] = np.cumsum(keep.sum(axis=1))
    rows, cols = np.nonzero(keep)
    blocks = np.ascontiguousarray(grid[rows, cols]) if len(rows) else np.zeros((0, b, b), A.dtype)
    return blocks, cols.astype(np.int64), row_ptrs, (m, n)


def csr_from_dense(A: np.ndarray, threshold: float = 0.0):
    """(values, col_idx, row_ptrs) as formats.py:269-278 builds them: entries
    with |v| > threshold (numpy compares in A's dtype), rows in order, columns
    ascending (torch.where's row-major order, kept by the COO sort)."""
    m, _ = A.shape
    mask = np.abs(A) > threshold
    rows, cols = np.nonzero(mask)
    row_ptrs = np.zeros(m + 1, dtype=np.int64)
    row_ptrs[1:] = np.cumsum(np.bincount(rows, minlength=m))
    return A[mask], cols.astype(np.int64), row_ptrs


def coo_to_csr(values, rows, cols, shape):
    """(values, col_idx, row_ptrs) as formats.py:104-124 builds them: entries
    ordered by the key row*n + col, equal keys in input order (a stable sort;
    the reference's argsort leaves their order unspecified), row_ptrs the
    cumulative row counts."""
    m, n = shape
    order = np.argsort(np.asarray(rows, np.int64) * n + np.asarray(cols, np.int64), kind="stable")
    row_ptrs = np.zeros(m + 1, dtype=np.int64)
    row_ptrs[1:] = np.cumsum(np.bincount(np.asarray(rows)[order], minlength=m)) if len(order) else 0
    return np.asarray(values)[order], np.asarray(cols, np.int64)[order], row_ptrs


def coo_sum_to_csr(values, rows, cols, shape):
    """Coalesced CSR: one entry per distinct (row, col), ordered by row*n + col,
    holding the sum of its duplicates in input order (explicit zeros kept) —
    torch's coalesce as sparse_add uses it (ops.py:107-132)."""
    v, c, p = coo_to_csr(values, rows, cols, shape)
    m, n = shape
    rows_s = np.repeat(np.arange(m), np.diff(p))
    keys = rows_s * n + c
    if len(keys) == 0:
        return v, c, p
    head = np.ones(len(keys), bool)
    head[1:] = keys[1:] != keys[:-1]
    seg = np.cumsum(head) - 1
    out_v = np.zeros(int(head.sum()), dtype=np.float64)
    np.add.at(out_v, seg, np.asarray(v, np.float64))
    out_c = c[head]
    out_p = np.zeros(m + 1, dtype=np.int64)
    out_p[1:] = np.cumsum(np.bincount(rows_s[head], minlength=m))
    return out_v, out_c, out_p


def sparse_add(A, B, alpha=1.0, beta=1.0):
    """(values, col_idx, row_ptrs) of alpha A + beta B on the union pattern
    (ops.py:107-132); A, B given as (values, col_idx, row_ptrs, shape)."""
    (va, ca, pa, shape), (vb, cb, pb, _) = A, B
    ra = np.repeat(np.arange(shape[0]), np.diff(pa))
    rb = np.repeat(np.arange(shape[0]), np.diff(pb))
    return coo_sum_to_csr(np.concatenate([alpha * np.asarray(va, np.float64), beta * np.asarray(vb, np.float64)]),
                          np.concatenate([ra, rb]), np.concatenate([ca, cb]), shape)


def csr_transpose(values, col_idx, row_ptrs, shape):
    """CSR of A^T (ops.py:145-154): rows expanded, (col, row) keys sorted stably."""
    m, n = shape
    rows = np.repeat(np.arange(m), np.diff(row_ptrs))
    return coo_to_csr(values, col_idx, rows, (n, m))


def spmv_symmetric(values, col_idx, row_ptrs, shape, x, alpha=1.0, absolute=False):
    """alpha (A x + S^T x), S = A's entries with row != col (ops.py:81-104), float64."""
    m, _ = shape
    rows = np.repeat(np.arange(m), np.diff(row_ptrs))
    v = np.abs(np.asarray(values, np.float64)) if absolute else np.asarray(values, np.float64)
    xv = np.abs(np.asarray(x, np.float64)) if absolute else np.asarray(x, np.float64)
    y = np.zeros(m)
    np.add.at(y, rows, v * xv[col_idx])
    off = rows != col_idx
    np.add.at(y, col_idx[off], v[off] * xv[rows[off]])
    return abs(alpha) * y if absolute else alpha * y


def bsr_to_dense(blocks, col_idx, row_ptrs, shape, b):
    m, n = shape
    mp, np_ = -(-m // b) * b, -(-n // b) * b
    D = np.zeros((mp, np_), dtype=np.float64)
    for i in range(len(row_ptrs) - 1):
        for idx in range(row_ptrs[i], row_ptrs[i + 1]):
            j = col_idx[idx]
            D[i * b : (i + 1) * b, j * b : (j + 1) * b] = blocks[idx]
    return D[:m, :n]


def bsr_spmm(blocks, col_idx, row_ptrs, shape, b, B, absolute: bool = False):
    """C = A @ B in float64 over stored blocks (reference ops.py:162-192).

    With absolute=True returns |A| @ |B|, the per-element error scale.
    """
    m, n = shape
    N = B.shape[1]
    mb = len(row_ptrs) - 1
    Bp = np.zeros((-(-n // b) * b, N))
    Bp[:n] = np.abs(B) if absolute else B
    C = np.zeros((mb * b, N))
    for i in range(mb):
        acc = C[i * b : (i + 1) * b]
        for idx in range(row_ptrs[i], row_ptrs[i + 1]):
            j = col_idx[idx]
            blk = blocks[idx].astype(np.float64)
            acc += (np.abs(blk) if absolute else blk) @ Bp[j * b : (j + 1) * b]
    return C[:m]


def bsr_spmm_backward(blocks, col_idx, row_ptrs, shape, b, B, G, absolute: bool = False):
    """Gradients of C = A @ B for the upstream gradient G = dC, in float64
    (reference autograd, trnsparse/nki/dispatch.py:331-369):
      dA_k = G[rows of block row i] @ B[rows of block column j]^T per stored
             block k = (i, j) (rows past m / n of the padded operands are 0)
      dB   = A^T @ G
    Returns (d_blocks (n_blocks, b, b), dB (n, N)). With absolute=True both
    use |.| operands: the per-element error scales.
    """
    m, n = shape
    N = B.shape[1]
    mb = len(row_ptrs) - 1
    nbc = -(-n // b)
    f = np.abs if absolute else (lambda x: x)
    Bp = np.zeros((nbc * b, N))
    Bp[:n] = f(B)
    Gp = np.zeros((mb * b, N))
    Gp[:m] = f(G)
    dblocks = np.zeros((len(col_idx), b, b))
    dB = np.zeros((nbc * b, N))
    for i in range(mb):
        gi = Gp[i * b : (i + 1) * b]
        for idx in range(row_ptrs[i], row_ptrs[i + 1]):
            j = col_idx[idx]
            dblocks[idx] = gi @ Bp[j * b : (j + 1) * b].T
            dB[j * b : (j + 1) * b] += f(blocks[idx].astype(np.float64)).T @ gi
    return dblocks, dB[:n]


# ------------------------------------------------------------------ CSR


def csr_rows(row_ptrs: np.ndarray) -> np.ndarray:
    m = len(row_ptrs) - 1
    return np.repeat(np.arange(m, dtype=np.int64), np.diff(row_ptrs))


def csr_spmv(values, col_idx, row_ptrs, shape, x, alpha=1.0, y=None, beta=0.0, absolute=False):
    """y = alpha*(A@x) [+ beta*y] in float64 (reference ops.py:30-48)."""
    m, _ = shape
    v = values.astype(np.float64)
    xv = x.astype(np.float64)
    if absolute:
        v, xv = np.abs(v), np.abs(xv)
    prod = v * xv[col_idx]
    out = np.bincount(csr_rows(row_ptrs), weights=prod, minlength=m)
    out = (abs(alpha) if absolute else alpha) * out
    if y is not None and beta != 0.0:
        yy = y.astype(np.float64)
        out = out + ((abs(beta) * np.abs(yy)) if absolute else beta * yy)
    return out


def csr_spmm(values, col_idx, row_ptrs, shape, B, alpha=1.0, C=None, beta=0.0, absolute=False):
    """C = alpha*(A@B) [+ beta*C] in float64 (reference ops.py:51-78)."""
    m, _ = shape
    v = values.astype(np.float64)
    Bv = B.astype(np.float64)
    if absolute:
        v, Bv = np.abs(v), np.abs(Bv)
    out = np.zeros((m, B.shape[1]))
    np.add.at(out, csr_rows(row_ptrs), v[:, None] * Bv[col_idx])
    out = (abs(alpha) if absolute else alpha) * out
    if C is not None and beta != 0.0:
        Cv = C.astype(np.float64)
        out = out + ((abs(beta) * np.abs(Cv)) if absolute else beta * Cv)
    return out


# ------------------------------------------------------------- screened


def screened_mask(diag: np.ndarray, threshold: float) -> np.ndarray:
    """mask[i,j] = fl(Q_i*Q_j) > fl(sqrt(threshold)), Q = fl(sqrt(|d|)).

    All three operations run in diag's precision (reference ops.py:273-276:
    torch evaluates the product in the tensor dtype and converts the Python
    float sqrt(threshold) to that dtype before comparing).
    """
    dt = diag.dtype
    Q = np.sqrt(np.abs(diag)).astype(dt)
    pair = np.multiply.outer(Q, Q).astype(dt)
    return pair > dt.type(math.sqrt(threshold))


def screened_spmm(A, diag, B, threshold, absolute=False):
    """C = (A * mask) @ B in float64 (reference ops.py:262-277)."""
    mask = screened_mask(diag, threshold)
    Am = np.where(mask, A.astype(np.float64), 0.0)
    Bv = B.astype(np.float64)
    if absolute:
        Am, Bv = np.abs(Am), np.abs(Bv)
    return Am @ Bv


def screened_spmm_backward(A, diag, B, threshold, dC, absolute=False):
    """(dA, dB) of C = (A * mask) @ B in float64 (reference
    nki/dispatch.py:478-484: grad_A = (grad_out @ B.T) * mask, grad_B =
    (A * mask).T @ grad_out; no gradient to diag or threshold). `absolute`
    gives the same products over |A|, |B|, |dC| (the error scale)."""
    mask = screened_mask(diag, threshold)
    Av, Bv, Gv = (x.astype(np.float64) for x in (A, B, dC))
    if absolute:
        Av, Bv, Gv = np.abs(Av), np.abs(Bv), np.abs(Gv)
    dA = np.where(mask, Gv @ Bv.T, 0.0)
    dB = np.where(mask, Av, 0.0).T @ Gv
    return dA, dB


# ------------------------------------------------------------ attention


def block_sparse_attention(Q, K, V, row_ptrs, col_idx, b, scale, rows=None):
    """Block-sparse attention in float64 (reference ops.py:280-357).

    The reference's pass 1 + reduction (tile max / stable exp-sum combined
    into row_max, row_denom) computes the exact row max and softmax
    denominator over the keys of the stored blocks; in float64 they are
    formed directly here. A block listed twice counts twice, as there.
    Keys at or past seq_len do not exist (the reference slices K/V, which
    come back short). `rows` restricts the work to some block rows (the
    other rows are left zero). Returns (out, row_max, row_denom) with stats
    shaped (M_tiles, b). Empty block rows: row_max 0, row_denom 1e-12,
    output 0.
    """
    S, D = Q.shape
    Mt = S // b
    q, k, v = (t.astype(np.float64) for t in (Q, K, V))
    out = np.zeros((S, D))
    rmax = np.zeros((Mt, b))
    rden = np.full((Mt, b), 1e-12)
    for m in range(Mt) if rows is None else rows:
        s, e = row_ptrs[m], row_ptrs[m + 1]
        if s == e:
            continue
        cols = col_idx[s:e]
        keys = np.concatenate([np.arange(c * b, min((c + 1) * b, S)) for c in cols])
        sc = (q[m * b : (m + 1) * b] @ k[keys].T) * scale
        mx = sc.max(axis=1)
        p = np.exp(sc - mx[:, None])
        den = np.maximum(p.sum(axis=1), 1e-12)
        out[m * b : (m + 1) * b] = (p / den[:, None]) @ v[keys]
        rmax[m] = mx
        rden[m] = den
    return out, rmax, rden


def block_sparse_attention_backward(Q, K, V, O, dO, row_ptrs, col_idx, b, scale, row_max=None, row_denom=None,
                                    absolute=False, rows=None, cols=None):
    """Tiled attention backward in float64 (reference ops.py:360-473).

    D = rowsum(dO * O); per stored block (m, c) of block rows m < S // b,
    P = exp(scale * Q_m K_c^T - row_max) / row_denom, dS = P * (dO_m V_c^T -
    D), dQ_m += scale * dS K_c, dK_c += scale * dS^T Q_m, dV_c += P^T dO_m.
    Keys at or past S do not exist (short K_c, V_c as in the reference's
    slices). Stats default to the oracle forward's. `rows` / `cols` restrict
    the dQ / (dK, dV) contributions to some block rows / block columns.
    absolute=True returns the error scale of each gradient element instead:
    dS replaced by P * (|dO V^T| + |D|) and Q, K, dO by their magnitudes.
    Returns (dQ, dK, dV) of shape (S, D).
    """
    S, Dh = Q.shape
    Mt = S // b
    q, k, v, o, do = (np.asarray(t, dtype=np.float64) for t in (Q, K, V, O, dO))
    if row_max is None or row_denom is None:
        _, row_max, row_denom = block_sparse_attention(q, k, v, row_ptrs, col_idx, b, scale)
    rmax = np.asarray(row_max, dtype=np.float64).reshape(-1)
    rden = np.asarray(row_denom, dtype=np.float64).reshape(-1)
    Dv = (do * o).sum(axis=1)
    qx, kx, dox = (np.abs(t) for t in (q, k, do)) if absolute else (q, k, do)
    dQ, dK, dV = np.zeros((S, Dh)), np.zeros((S, Dh)), np.zeros((S, Dh))
    rows = None if rows is None else set(int(r) for r in rows)
    cols = None if cols is None else set(int(c) for c in cols)
    for m in range(Mt):
        for idx in range(row_ptrs[m], row_ptrs[m + 1]):
            c = int(col_idx[idx])
            want_q = rows is None or m in rows
            want_kv = cols is None or c in cols
            if not (want_q or want_kv) or c * b >= S:
                continue
            qs, ks = slice(m * b, (m + 1) * b), slice(c * b, min((c + 1) * b, S))
            P = np.exp((q[qs] @ k[ks].T) * scale - rmax[qs, None]) / rden[qs, None]
            dp = do[qs] @ v[ks].T
            dS = P * (np.abs(dp) + np.abs(Dv[qs])[:, None]) if absolute else P * (dp - Dv[qs, None])
            if want_q:
                dQ[qs] += (dS @ kx[ks]) * scale
            if want_kv:
                dK[ks] += (dS.T @ qx[qs]) * scale
                dV[ks] += P.T @ dox[qs]
    return dQ, dK, dV


def dense_masked_attention(Q, K, V, mask, scale):
    """softmax(scale*Q@K^T masked to -inf off `mask`) @ V in float64
    (the dense oracle of the reference, examples/block_sparse_attention.py:161-172)."""
    sc = (Q.astype(np.float64) @ K.astype(np.float64).T) * scale
    sc = np.where(mask, sc, -np.inf)
    mx = sc.max(axis=1, keepdims=True)
    p = np.exp(sc - mx)
    p /= p.sum(axis=1, keepdims=True)
    return p @ V.astype(np.float64)


# ------------------------------------------------------------- solvers


def chebyshev_coeffs(lam_min, lam_max, K, dtype=np.float32):
    """(alpha, beta) of the fixed-step Chebyshev iteration in momentum form
    as the reference computes them (iterative.py:148-197, after Barrett et
    al., Templates, 1994, Algorithm 2.1): alpha_0 = 1/d and the generic step
    from k = 1 on, which makes the residual polynomial the second-kind
    U_K((d - lam)/c) / U_K(d/c); float64 recurrence, returned in `dtype`."""
    c, d = (lam_max - lam_min) / 2.0, (lam_max + lam_min) / 2.0
    alpha, beta = np.zeros(K), np.zeros(K)
    if K:
        alpha[0] = prev = 1.0 / d
        for k in range(1, K):
            t = (c * prev / 2.0) ** 2
            alpha[k] = 1.0 / (d - t / prev)
            beta[k] = alpha[k] * t / prev
            prev = alpha[k]
    return alpha.astype(dtype), beta.astype(dtype)


def richardson(matvec, b, omega, K, x0=None):
    """K steps of x <- x + omega (b - A x) in float64 (reference iterative.py:256-295)."""
    x = np.zeros_like(b, dtype=np.float64) if x0 is None else np.array(x0, dtype=np.float64)
    for _ in range(K):
        x = x + omega * (b - matvec(x))
    return x


def chebyshev(matvec, b, alpha, beta, K, x0=None):
    """K Chebyshev steps in float64 with the given coefficients (reference
    iterative.py:200-253): x_{k+1} = x_k + alpha_k r_k + beta_k (x_k - x_{k-1})."""
    x = np.zeros_like(b, dtype=np.float64) if x0 is None else np.array(x0, dtype=np.float64)
    x_prev = x.copy()
    for k in range(K):
        x_new = x + float(alpha[k]) * (b - matvec(x))
        if k > 0:
            x_new = x_new + float(beta[k]) * (x - x_prev)
        x_prev, x = x, x_new
    return x


def bsr_matvec(blocks, col_idx, row_ptrs, shape, b):
    """x -> A x in float64 for a BSR matrix (the N = 1 case of bsr_spmm)."""
    def mv(x):
        return bsr_spmm(blocks, col_idx, row_ptrs, shape, b, np.asarray(x, dtype=np.float64)[:, None])[:, 0]
    return mv


# ------------------------------------------------------------- metrics


def scaled_error(got, ref, scale, floor: float = 1e-30) -> float:
    """max_ij |got-ref| / (|A|.|B|)_ij — the dot-product error measure."""
    got = np.asarray(got, dtype=np.float64)
    return float(np.max(np.abs(got - ref) / np.maximum(scale, floor), initial=0.0))


def rel_max_error(got, ref) -> float:
    """max|got-ref| / max|ref|."""
    got = np.asarray(got, dtype=np.float64)
    den = float(np.max(np.abs(ref), initial=0.0))
    num = float(np.max(np.abs(got - ref), initial=0.0))
    return num / den if den > 0 else num
