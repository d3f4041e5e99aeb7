"""GPU parity of the column-sorted SpMV plan (tsp_csr_colplan_*) against the oracle.

The plan path computes the reference's spmv (trnsparse/ops.py:30-48) from a
reordered copy of the matrix; these tests drive it through the public
`spmv` with the plan forced on, and through the C ABI for the tiling hints.
Cases: tile edges (m, n not multiples of the tile), empty rows and empty
tiles, one row / one column, int32 and int64 indices, alpha / beta / y,
new values on a cached pattern (refresh), NaN in x at unreferenced
columns (lanes past a tile's end must not leak into a row), and the
full-size BASELINE config 2 (Poisson and Zipf rows) against the C oracle
with a float64 accumulator plus the checksum property sum(y) = colsum(A).x.
fp32 tolerance: max error <= 1e-4 relative to the (|A|.|x|)_i scale.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import trnsparse_amd as ts
from oracle import build as oracle_c
from oracle import ref
from trnsparse_amd import workloads as W
from trnsparse_amd.hip import _lib
from trnsparse_amd.hip import dispatch as D

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture
def plan_always(hip_backend):
    prev = D.get_spmv_plan()
    D.set_spmv_plan("always")
    yield
    D.set_spmv_plan(prev)


def _random(m, n, lens, seed, index_dtype=np.int64):
    rng = np.random.default_rng(seed)
    v, c, p = W.random_csr(lens, n, rng)
    return v, c.astype(index_dtype), p.astype(index_dtype), rng


def _check(v, c, p, shape, x, got, alpha=1.0, y=None, beta=0.0):
    exact = ref.csr_spmv(v, c.astype(np.int64), p.astype(np.int64), shape, x, alpha, y, beta)
    scale = ref.csr_spmv(v, c.astype(np.int64), p.astype(np.int64), shape, x, alpha, y, beta, absolute=True)
    err = ref.scaled_error(got, exact, scale)
    assert err <= TOL, err


@pytest.mark.parametrize(
    "m,n,mean,seed",
    [
        (5000, 7000, 9, 0),        # one row block, several column groups
        (40000, 33333, 12, 1),     # m, n not multiples of the tile
        (17000, 1, 1, 2),          # a single column
        (1, 50000, 3000, 3),       # a single long row
        (70000, 200000, 2, 4),     # sparse: tiles with few or no entries
    ],
)
@pytest.mark.parametrize("index_dtype", [np.int64, np.int32])
def test_colplan_spmv_shapes(plan_always, m, n, mean, seed, index_dtype):
    rng0 = np.random.default_rng(100 + seed)
    lens = np.minimum(rng0.poisson(mean, m), n)
    lens[rng0.random(m) < 0.1] = 0                    # empty rows
    v, c, p, rng = _random(m, n, lens, seed, index_dtype)
    A = W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")
    x = rng.standard_normal(n).astype(np.float32)
    got = ts.spmv(A, torch.from_numpy(x).cuda())
    assert getattr(A, "_hip_colplan", None) is not None or len(v) == 0
    _check(v, c, p, (m, n), x, got.cpu().numpy())
    y = rng.standard_normal(m).astype(np.float32)
    got = ts.spmv(A, torch.from_numpy(x).cuda(), alpha=-1.5, y=torch.from_numpy(y).cuda(), beta=0.25)
    _check(v, c, p, (m, n), x, got.cpu().numpy(), -1.5, y, 0.25)


@pytest.mark.parametrize("rbits,tiles", [(12, 0), (13, 7), (14, 1), (14, 600), (12, 4096)])
def test_colplan_tiling_hints_via_c_abi(hip_backend, rbits, tiles):
    """Every tiling the geometry allows gives the oracle's result; G == 1
    (no partial vectors) and G > 1 (partials summed by the second kernel)."""
    m, n = 30000, 90000
    rng0 = np.random.default_rng(rbits * 1000 + tiles)
    v, c, p, rng = _random(m, n, rng0.poisson(11, m), rbits + tiles)
    A = W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")
    vals, cols, ptrs, _ = D._csr_device(A, torch.device("cuda"))
    prev = D.get_spmv_plan()
    D.set_spmv_plan("always")
    try:
        geom, plan = D._csr_colplan(A, vals, cols, ptrs, torch.device("cuda"), rbits, tiles)
    finally:
        D.set_spmv_plan(prev)
    assert geom[0] == rbits and geom[4] == geom[1] * geom[3]
    assert geom[3] == -(-n // (1 << int(geom[2])))
    x = rng.standard_normal(n).astype(np.float32)
    y = rng.standard_normal(m).astype(np.float32)
    xd, yd = torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda()
    out = torch.empty(m, device="cuda")
    work = torch.empty(max(1, int(geom[8])), dtype=torch.uint8, device="cuda")
    csr = (vals.data_ptr(), cols.data_ptr(), ptrs.data_ptr(), _lib.index_code(cols.dtype))
    _lib.call("tsp_csr_colplan_spmv", plan.data_ptr(), _lib.TSP_F32, m, n, len(v), geom.ctypes.data, *csr,
              xd.data_ptr(), 0.5, yd.data_ptr(), -2.0, out.data_ptr(), work.data_ptr(),
              _lib.stream_handle(torch.device("cuda")))
    _check(v, c, p, (m, n), x, out.cpu().numpy(), 0.5, y, -2.0)
    # a geometry that does not belong to the shape is refused on the host
    bad = geom.copy()
    bad[3] += 1
    with pytest.raises(RuntimeError, match="geometry"):
        _lib.call("tsp_csr_colplan_spmv", plan.data_ptr(), _lib.TSP_F32, m, n, len(v), bad.ctypes.data, *csr,
                  xd.data_ptr(), 1.0, None, 0.0, out.data_ptr(), work.data_ptr(), 0)


@pytest.mark.parametrize("rbits,tiles", [(13, 1), (12, 0)])
def test_colplan_runs_across_lanes_and_wavefronts(hip_backend, rbits, tiles):
    """Rows whose entries fill most of an epoch (many lanes of one
    instruction adding to the same LDS row sum) next to rows of one or two
    entries. With tiles=1 a tile holds all columns, so a row of 30000
    entries takes most positions of its epochs. Two calls must agree bit
    for bit."""
    m, n = 8192, 60000
    rng0 = np.random.default_rng(21)
    lens = rng0.poisson(2, m)
    heavy = rng0.choice(m, 12, replace=False)
    lens[heavy] = [8, 9, 16, 63, 512, 513, 1500, 4096, 9000, 20000, 30000, 59000]
    v, c, p, rng = _random(m, n, lens, 22)
    A = W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")
    vals, cols, ptrs, _ = D._csr_device(A, torch.device("cuda"))
    prev = D.get_spmv_plan()
    D.set_spmv_plan("always")
    try:
        geom, plan = D._csr_colplan(A, vals, cols, ptrs, torch.device("cuda"), rbits, tiles)
    finally:
        D.set_spmv_plan(prev)
    x = rng.standard_normal(n).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    outs = []
    for _ in range(2):
        out = torch.empty(m, device="cuda")
        work = torch.empty(max(1, int(geom[8])), dtype=torch.uint8, device="cuda")
        _lib.call("tsp_csr_colplan_spmv", plan.data_ptr(), _lib.TSP_F32, m, n, len(v), geom.ctypes.data,
                  vals.data_ptr(), cols.data_ptr(), ptrs.data_ptr(), _lib.index_code(cols.dtype), xd.data_ptr(), 1.0,
                  None, 0.0, out.data_ptr(), work.data_ptr(), _lib.stream_handle(torch.device("cuda")))
        outs.append(out.cpu().numpy())
    _check(v, c, p, (m, n), x, outs[0])
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


@pytest.mark.parametrize("index_dtype", [np.int64, np.int32])
def test_colplan_view_with_nonzero_first_row_pointer(hip_backend, index_dtype):
    """A CSR view whose row_ptrs[0] is not zero (the pattern's entries start
    `base` entries into the arrays): the plan keeps each entry's position
    relative to row_ptrs[0], so the build, the SpMV and a refresh with new
    values all read values[row_ptrs[0] + k], whatever base is."""
    m, n, base = 12000, 15000, 777
    v, c, p, rng = _random(m, n, np.random.default_rng(5).poisson(9, m), 31, index_dtype)
    junk_v = rng.standard_normal(base).astype(np.float32) * 1e6
    junk_c = rng.integers(0, n, base).astype(index_dtype)
    dev = torch.device("cuda")
    vals = torch.from_numpy(np.concatenate([junk_v, v])).to(dev)
    cols = torch.from_numpy(np.concatenate([junk_c, c])).to(dev)
    ptrs = torch.from_numpy((p + base).astype(index_dtype)).to(dev)
    nnz = len(v)
    geom = np.zeros(10, dtype=np.int64)
    _lib.call("tsp_csr_colplan_geometry", m, n, nnz, 0, 0, geom.ctypes.data)
    plan = torch.empty(int(geom[6]), dtype=torch.uint8, device=dev)
    work = torch.empty(int(geom[7]), dtype=torch.uint8, device=dev)
    st = _lib.stream_handle(dev)
    _lib.call("tsp_csr_colplan_build", vals.data_ptr(), _lib.TSP_F32, cols.data_ptr(), ptrs.data_ptr(),
              _lib.index_code(cols.dtype), m, n, nnz, geom.ctypes.data, plan.data_ptr(), work.data_ptr(), st)
    x = rng.standard_normal(n).astype(np.float32)
    xd = torch.from_numpy(x).to(dev)
    out = torch.empty(m, device=dev)
    ws = torch.empty(max(1, int(geom[8])), dtype=torch.uint8, device=dev)

    def run():
        _lib.call("tsp_csr_colplan_spmv", plan.data_ptr(), _lib.TSP_F32, m, n, nnz, geom.ctypes.data, vals.data_ptr(),
                  cols.data_ptr(), ptrs.data_ptr(), _lib.index_code(cols.dtype), xd.data_ptr(), 1.0, None, 0.0,
                  out.data_ptr(), ws.data_ptr(), st)
        return out.cpu().numpy()

    _check(v, c, p, (m, n), x, run())
    v2 = rng.standard_normal(nnz).astype(np.float32)
    vals[base:] = torch.from_numpy(v2).to(dev)
    _lib.call("tsp_csr_colplan_refresh", vals.data_ptr(), _lib.TSP_F32, ptrs.data_ptr(), _lib.index_code(ptrs.dtype),
              m, n, nnz, geom.ctypes.data, plan.data_ptr(), st)
    _check(v2, c, p, (m, n), x, run())


def test_colplan_refresh_follows_new_values(plan_always):
    m, n = 20000, 20000
    v, c, p, rng = _random(m, n, np.full(m, 16), 7)
    A = W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")
    x = rng.standard_normal(n).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    _check(v, c, p, (m, n), x, ts.spmv(A, xd).cpu().numpy())
    plan_before = A._hip_colplan[3]
    v2 = rng.standard_normal(len(v)).astype(np.float32)
    A.values.copy_(torch.from_numpy(v2))           # in place: same pattern, new values
    _check(v2, c, p, (m, n), x, ts.spmv(A, xd).cpu().numpy())
    assert A._hip_colplan[3] is plan_before        # regathered, not rebuilt


def test_colplan_nan_at_unreferenced_columns(plan_always):
    """x holds NaN / inf at every column no entry references; lanes past a
    tile's end (which read padding or the next tile) must not reach a row."""
    m, n = 9000, 40000
    v, c, p, rng = _random(m, n, np.full(m, 5), 8)
    x = np.full(n, np.nan, np.float32)
    x[1::3] = np.inf
    used = np.unique(c)
    x[used] = rng.standard_normal(len(used)).astype(np.float32)
    A = W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")
    got = ts.spmv(A, torch.from_numpy(x).cuda()).cpu().numpy()
    assert np.isfinite(got).all()
    _check(v, c, p, (m, n), x, got)


def _check_nonfinite(v, c, p, shape, x, got):
    """inf / NaN exactly where the float64 oracle has them (same sign of
    inf), the finite rows within the tolerance."""
    exact = ref.csr_spmv(v, c.astype(np.int64), p.astype(np.int64), shape, x)
    scale = ref.csr_spmv(v, c.astype(np.int64), p.astype(np.int64), shape, x, absolute=True)
    assert np.array_equal(np.isnan(got), np.isnan(exact))
    inf = np.isinf(exact)
    assert np.array_equal(np.isinf(got), inf) and np.array_equal(got[inf], exact[inf])
    fin = np.isfinite(exact)
    assert ref.scaled_error(got[fin], exact[fin], scale[fin]) <= TOL


@pytest.mark.parametrize("index_dtype", [np.int64, np.int32])
def test_colplan_nonfinite_x_at_referenced_columns(plan_always, index_dtype):
    """inf and NaN in x where entries reference them: the rows that read them
    come out inf / NaN as the reference's fp32 products make them (0 * inf
    = NaN, inf - inf = NaN); every other row is unaffected."""
    m, n = 6000, 9000
    v, c, p, rng = _random(m, n, np.full(m, 6), 40, index_dtype)
    x = rng.standard_normal(n).astype(np.float32)
    x[c[:50]] = np.inf
    x[c[200:230]] = -np.inf
    x[c[400:420]] = np.nan
    v[5] = 0.0  # a stored zero times inf
    A = W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")
    got = ts.spmv(A, torch.from_numpy(x).cuda()).cpu().numpy()
    _check_nonfinite(v, c, p, (m, n), x, got)


@pytest.mark.parametrize("case", ["outlier", "nan"])
def test_colplan_long_rows_summed_again(plan_always, case):
    """Rows longer than the finish kernel's serial limit on the slow path:
    one huge |x| makes every row's products small against the scale (so
    every row is summed again from the CSR arrays, the long ones by a whole
    wavefront), or a NaN in x sends every row there; results match the
    oracle row for row."""
    m, n = 3000, 50000
    rng0 = np.random.default_rng(45)
    lens = rng0.poisson(8, m)
    lens[rng0.choice(m, 300, replace=False)] = rng0.integers(33, 5000, 300)
    v, c, p, rng = _random(m, n, lens, 46)
    x = rng.standard_normal(n).astype(np.float32)
    if case == "outlier":
        x[n - 1] = 3e30                    # far above every other |x|
    else:
        x[c[p[17]]] = np.nan               # read by row 17 only (among others by chance)
    A = W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")
    got = ts.spmv(A, torch.from_numpy(x).cuda()).cpu().numpy()
    _check_nonfinite(v, c, p, (m, n), x, got)
    again = ts.spmv(A, torch.from_numpy(x).cuda()).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))


def test_colplan_nonfinite_values(plan_always):
    """inf / NaN values (rows summed from the CSR arrays) next to finite rows."""
    m, n = 6000, 9000
    v, c, p, rng = _random(m, n, np.full(m, 6), 41)
    v[[10, 500, 3000]] = [np.inf, -np.inf, np.nan]
    A = W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")
    x = rng.standard_normal(n).astype(np.float32)
    got = ts.spmv(A, torch.from_numpy(x).cuda()).cpu().numpy()
    _check_nonfinite(v, c, p, (m, n), x, got)


@pytest.mark.parametrize("xscale", [1e-15, 1.0, 1e15])
def test_colplan_relative_accuracy_across_scales(plan_always, xscale):
    """The fixed-point row sums follow the scale of x and of each row: with
    positive values and x (no cancellation) every row keeps fp32 relative
    accuracy whatever the magnitudes, including rows whose values are 1e-20
    of another row's and x scaled by 1e-15 or 1e15 (no fp32 product
    underflows)."""
    m, n = 8000, 12000
    v, c, p, rng = _random(m, n, np.random.default_rng(42).poisson(10, m), 43)
    v = np.abs(v) + 0.01
    rows = np.repeat(np.arange(m), np.diff(p))
    v = (v * np.where(rows % 3 == 0, 1e-20, 1.0)[rows]).astype(np.float32)  # every third row tiny
    x = ((np.abs(rng.standard_normal(n)) + 0.01) * xscale).astype(np.float32)
    A = W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")
    got = ts.spmv(A, torch.from_numpy(x).cuda()).cpu().numpy().astype(np.float64)
    exact = ref.csr_spmv(v, c, p, (m, n), x)
    nz = exact != 0
    assert np.max(np.abs(got[nz] - exact[nz]) / exact[nz]) <= 1e-5
    assert np.all(got[~nz] == 0)


def test_colplan_small_products_beside_large_values(plan_always):
    """A row whose large values meet x = 0 and whose result comes from
    products far below the row's scale (rounded in fixed point, so the row
    is summed again from the CSR arrays), a row with a subnormal value that
    the plan's scaling would flush (always summed from the CSR arrays), and
    a row whose products cancel exactly."""
    n = 8
    c = np.array([0, 1, 2, 3, 4, 5, 6, 7, 0, 1], dtype=np.int64)
    p = np.array([0, 4, 6, 8, 10], dtype=np.int64)
    v = np.array([1e30, -3e29, 2e-20, 5e-21, 1e30, 1e-40, 3.0, -3.0, 0.5, -0.5], dtype=np.float32)
    x = np.array([0.0, 0.0, 1.0, 3.0, 0.0, 1e30, 7.0, 7.0, 2.0, 2.0], dtype=np.float32)[:n]
    x[0], x[1] = 2.0, 2.0  # row 3: 0.5*2 - 0.5*2 = 0 exactly; row 0 reads cols 0, 1 too
    v[0], v[1] = 1e30, -1e30  # row 0: 1e30*2 - 1e30*2 cancel, 2e-20*1 + 5e-21*3 remain
    m = 4
    A = W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")
    got = ts.spmv(A, torch.from_numpy(x).cuda()).cpu().numpy().astype(np.float64)
    exact = ref.csr_spmv(v, c, p, (m, n), x)
    assert abs(got[0] - exact[0]) <= 1e-6 * abs(exact[0])
    assert abs(got[1] - exact[1]) <= 1e-6 * abs(exact[1])
    assert got[2] == exact[2] == 0.0 and got[3] == exact[3] == 0.0


def test_colplan_zero_x_and_beta(plan_always):
    m, n = 3000, 4000
    v, c, p, rng = _random(m, n, np.full(m, 7), 44)
    A = W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")
    y = rng.standard_normal(m).astype(np.float32)
    got = ts.spmv(A, torch.zeros(n, device="cuda"), alpha=2.0, y=torch.from_numpy(y).cuda(), beta=0.5)
    assert torch.equal(got.cpu(), torch.from_numpy(y) * 0.5)


def test_colplan_operator_compile_and_graph(plan_always):
    """The plan SpMV operator (x-max pre-pass, tile kernel, finish, one
    workspace per call) under torch.compile and in a captured HIP graph:
    every replay with new x contents, with eager work and synchronizations
    between replays, equals the eager call bit for bit (a solver loop
    captures exactly this)."""
    m, n = 40000, 33333
    lens = np.minimum(np.random.default_rng(61).poisson(12, m), n)
    v, c, p, rng = _random(m, n, lens, 62)
    A = W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")
    vals, cols, ptrs = A.values, A.col_indices, A.row_ptrs
    x0 = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda()
    ts.spmv(A, x0)                                   # builds and caches the plan
    _, _, geom, plan, _ = A._hip_colplan
    ops = _lib.ops()
    gt = D._geometry_list(geom)

    def call(x, y=None, beta=0.0):
        return ops.csr_colplan_spmv(plan, gt, vals, cols, ptrs, m, n, x, 1.25, y, beta)

    want = call(x0)
    assert torch.equal(want, ts.spmv(A, x0, alpha=1.25))
    _check(v, c, p, (m, n), x0.cpu().numpy(), want.cpu().numpy(), 1.25)

    @torch.compile(fullgraph=True, backend="aot_eager")
    def f(x):
        return call(x * 2.0) + 1.0

    torch.testing.assert_close(f(x0), 2.0 * want + 1.0, rtol=1e-6, atol=1e-5)

    static_x = x0.clone()
    static_y = torch.from_numpy(rng.standard_normal(m).astype(np.float32)).cuda()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call(static_x, static_y, -0.5)               # warm up on the side stream
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = call(static_x, static_y, -0.5)
    for rep in range(3):
        newx = torch.from_numpy(np.random.default_rng(70 + rep).standard_normal(n).astype(np.float32)).cuda()
        if rep == 2:
            newx[17] = float("nan")                  # the slow path inside the graph as well
        static_x.copy_(newx)
        graph.replay()
        torch.cuda.synchronize()
        eager = call(newx, static_y, -0.5)
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager) if rep < 2 else torch.equal(static_out.isnan(), eager.isnan())
        if rep == 2:
            keep = ~eager.isnan()
            assert keep.any() and torch.equal(static_out[keep], eager[keep])


def test_colplan_auto_mode_builds_on_reuse(hip_backend):
    prev = D.get_spmv_plan()
    D.set_spmv_plan("auto")
    try:
        m = n = 1 << 15
        v, c, p, rng = _random(m, n, np.full(m, 12), 9)
        A = W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")
        xd = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda()
        first = ts.spmv(A, xd)
        assert getattr(A, "_hip_colplan", None) is None      # one-off use: windowed kernel
        second = ts.spmv(A, xd)
        assert getattr(A, "_hip_colplan", None) is not None  # reused unchanged: plan built
        _check(v, c, p, (m, n), xd.cpu().numpy(), second.cpu().numpy())
        # the two kernels add a row's products in different orders: the first
        # two auto-mode calls agree to tolerance, not bit for bit; from the
        # second call on the plan runs and repeats exactly
        torch.testing.assert_close(first, second, rtol=1e-5, atol=1e-4)
        assert torch.equal(ts.spmv(A, xd), second)
        D.set_spmv_plan("never")
        assert torch.equal(ts.spmv(A, xd), first)  # "never": always the windowed kernel, bit-stable
    finally:
        D.set_spmv_plan(prev)


def test_colplan_auto_mode_regathers_reused_values_only(hip_backend):
    """Under "auto", new values on a planned pattern run the windowed kernel
    once; the plan takes them (one regather) when they come back, and
    values that change on every call never pay the regather."""
    prev = D.get_spmv_plan()
    D.set_spmv_plan("auto")
    try:
        m = n = 1 << 15
        v, c, p, rng = _random(m, n, np.full(m, 12), 10)
        A = W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")
        x = rng.standard_normal(n).astype(np.float32)
        xd = torch.from_numpy(x).cuda()
        ts.spmv(A, xd)
        ts.spmv(A, xd)                                   # plan built on reuse
        key0 = A._hip_colplan[1]
        for _ in range(2):                               # new values every call
            v = rng.standard_normal(len(v)).astype(np.float32)
            A.values.copy_(torch.from_numpy(v))
            _check(v, c, p, (m, n), x, ts.spmv(A, xd).cpu().numpy())
            assert A._hip_colplan[1] == key0             # not regathered
        _check(v, c, p, (m, n), x, ts.spmv(A, xd).cpu().numpy())  # the same values again
        assert A._hip_colplan[1] != key0                 # regathered once
        _check(v, c, p, (m, n), x, ts.spmv(A, xd).cpu().numpy())
    finally:
        D.set_spmv_plan(prev)


@pytest.mark.parametrize("dist", ["poisson", "zipf"])
@pytest.mark.parametrize("index_dtype", [np.int64, np.int32])
def test_colplan_cfg2_full_size(plan_always, dist, index_dtype):
    v, c, p, x, shape = W.cfg2_csr(dist=dist, index_dtype=index_dtype)
    A = W.csr_matrix_from_arrays(v, c, p, shape, device="cuda")
    xd = torch.from_numpy(x).cuda()
    got = ts.spmv(A, xd).cpu().numpy()
    assert A._hip_colplan is not None
    exact = oracle_c.csr_spmv_f64(v, c, p, shape[0], x)
    scale = oracle_c.csr_spmv_f64(v, c, p, shape[0], x, absolute=True)
    assert ref.scaled_error(got, exact, scale) <= TOL
    colsum = np.bincount(c.astype(np.int64), weights=v.astype(np.float64), minlength=shape[1])
    assert abs(got.astype(np.float64).sum() - colsum @ x) <= TOL * float(np.abs(v).astype(np.float64) @ np.abs(x[c]))
    again = ts.spmv(A, xd).cpu().numpy()
    assert ref.scaled_error(again, exact, scale) <= TOL


# ----------------------------------------------------- length-bucketed rows


@pytest.fixture
def plan_bucketed(hip_backend):
    prev = D.get_spmv_plan()
    D.set_spmv_plan("bucketed")
    yield
    D.set_spmv_plan(prev)


@pytest.mark.parametrize("index_dtype", [np.int64, np.int32])
def test_bucketed_spmv_every_bucket(plan_bucketed, index_dtype):
    """Rows of every class (empty, <= 32, the 32 / 33 and 2048 / 2049 edges,
    a 100000-entry row) against the oracle, with alpha / beta / y; the plan
    holds exactly the rows above 32 and above 2048 entries."""
    m, n = 6000, 150000
    rng0 = np.random.default_rng(11)
    lens = np.minimum(rng0.poisson(9, m), n)
    lens[rng0.random(m) < 0.1] = 0
    lens[[5, 6, 7, 8, 9]] = [32, 33, 2048, 2049, 100000]
    lens[rng0.choice(m, 200, replace=False)] = rng0.integers(34, 3000, 200)
    v, c, p, rng = _random(m, n, lens, 12, index_dtype)
    A = W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")
    x = rng.standard_normal(n).astype(np.float32)
    got = ts.spmv(A, torch.from_numpy(x).cuda())
    _check(v, c, p, (m, n), x, got.cpu().numpy())
    plan, n_med, n_long = A._hip_bucket_plan[1]
    assert n_med == int(((lens > 32) & (lens <= 2048)).sum()) and n_long == int((lens > 2048).sum())
    assert sorted(plan[4:4 + n_med].cpu().tolist()) == np.flatnonzero((lens > 32) & (lens <= 2048)).tolist()
    assert sorted(plan[4 + m:4 + m + n_long].cpu().tolist()) == np.flatnonzero(lens > 2048).tolist()
    y = rng.standard_normal(m).astype(np.float32)
    got = ts.spmv(A, torch.from_numpy(x).cuda(), alpha=0.5, y=torch.from_numpy(y).cuda(), beta=-2.0)
    _check(v, c, p, (m, n), x, got.cpu().numpy(), 0.5, y, -2.0)


def test_bucketed_spmv_f64_and_empty(plan_bucketed):
    m, n = 3000, 5000
    rng0 = np.random.default_rng(13)
    lens = np.minimum(rng0.poisson(40, m), n)
    v, c, p, rng = _random(m, n, lens, 14)
    v = v.astype(np.float64)
    A = W.csr_matrix_from_arrays(v, c, p, (m, n), device="cuda")
    x = rng.standard_normal(n)
    got = ts.spmv(A, torch.from_numpy(x).cuda()).cpu().numpy()
    exact = ref.csr_spmv(v, c, p, (m, n), x)
    scale = ref.csr_spmv(v, c, p, (m, n), x, absolute=True)
    assert ref.scaled_error(got, exact, scale) <= 1e-12
    E = W.csr_matrix_from_arrays(np.zeros(0, np.float32), np.zeros(0, np.int64), np.zeros(m + 1, np.int64), (m, n),
                                 device="cuda")
    assert torch.count_nonzero(ts.spmv(E, torch.ones(n, device="cuda"))).item() == 0


@pytest.mark.parametrize("dist", ["poisson", "zipf"])
def test_bucketed_cfg2_full_size(plan_bucketed, dist):
    v, c, p, x, shape = W.cfg2_csr(dist=dist, index_dtype=np.int64)
    A = W.csr_matrix_from_arrays(v, c, p, shape, device="cuda")
    got = ts.spmv(A, torch.from_numpy(x).cuda()).cpu().numpy()
    exact = oracle_c.csr_spmv_f64(v, c, p, shape[0], x)
    scale = oracle_c.csr_spmv_f64(v, c, p, shape[0], x, absolute=True)
    assert ref.scaled_error(got, exact, scale) <= TOL
