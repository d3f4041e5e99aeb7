#!/usr/bin/env python3
"""Benchmark of the trnsparse compute path on one MI355X.

`python bench.py [--gpus 1] [--steps K] [--warmup W]` prints ONE JSON line.

Headline (BASELINE metric "bsr_spmm effective GFLOP/s (nnz blocks) + % MFMA
peak"): bsr_spmm at config 3a — 16384x16384 in 128x128 blocks, 10% block
density (1638 stored blocks), B 16384x512, fp32. One step = one bsr_spmm
call over the resident operands; FLOPs = 2 * n_blocks * 128^2 * 512
(stored blocks only). The `secondary` list carries the other configs
(CSR SpMV HBM GB/s, bf16 bsr_spmm, bsr_spmm backward, screened_spmm,
block-sparse attention),
each timed with HIP events on the stream the kernel runs on.

`roofline` is for the dominant kernel of the headline (bsr_spmm_f32_dma):
achieved = algorithmic FLOPs per launch / average launch time from HIP
events over the timed region, peak = 157.3 TFLOP/s (MI355X dense fp32
matrix). `traffic` (HBM bytes per launch) comes from the committed
rocprofv3 PMC summary in profiles/ when present.

`cpu_baseline` is the reference's torch CPU path for the same workload
(oracle/cpu_baseline.py) timed on this host's cores.

All inputs are synthetic and seeded (trnsparse_amd/workloads.py).
"""

from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2500.0
FP64_MFMA_PEAK_TFLOPS = 78.6
HBM_PEAK_GBS = 8000.0


def _events():
    import torch

    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def prewarm(fn, seconds: float = 0.25):
    """Run `fn` back to back for about `seconds` (untimed) so the GPU clocks
    reach their sustained level before measuring; a cold MI355X measures
    10-15% slow over the first tens of milliseconds."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def time_gpu(fn, steps: int, warmup: int, flush=None, prewarm_s: float = 0.25):
    """(wall ms/step, event ms/step). With `flush`, each step is timed alone
    after `flush()` evicts L2/MALL, and the event time is the median.
    Untimed: a clock pre-warm of `prewarm_s` seconds, then `warmup` steps."""
    import torch

    if prewarm_s > 0:
        prewarm(fn, prewarm_s)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    if flush is None:
        s, e = _events()
        t0 = time.perf_counter()
        s.record()
        for _ in range(steps):
            fn()
        e.record()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3 / steps
        return wall, s.elapsed_time(e) / steps
    times = []
    t0 = time.perf_counter()
    for _ in range(steps):
        flush()
        s, e = _events()
        s.record()
        fn()
        e.record()
        torch.cuda.synchronize()
        times.append(s.elapsed_time(e))
    wall = (time.perf_counter() - t0) * 1e3 / steps
    times.sort()
    return wall, times[len(times) // 2]


def time_gpu_spread(fn, steps: int, warmup: int, segments: int = 5, prewarm_s: float = 0.25):
    """Per-launch event times of `segments` back-to-back timed segments of
    `steps` launches each (same pre-warm and warmup as time_gpu), as
    (median, min, max) in ms: the spread of a line across segments of one
    run, next to its median."""
    import torch

    if prewarm_s > 0:
        prewarm(fn, prewarm_s)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    seg = []
    for _ in range(segments):
        s, e = _events()
        s.record()
        for _ in range(steps):
            fn()
        e.record()
        torch.cuda.synchronize()
        seg.append(s.elapsed_time(e) / steps)
    seg.sort()
    return seg[len(seg) // 2], seg[0], seg[-1]


_CLOCK_LIB = None


def shader_clock_ghz(fn, per_call_ms: float, window_ms: float = 1.0):
    """Shader clock (GHz) while `fn` runs back to back, or None when the probe
    library (trnsparse_amd/libtrnsparse_clock.so) is not built.

    A one-wave probe on a side stream counts shader-clock cycles over
    `window_ms` of the 100 MHz real-time counter; it starts once a few
    launches of `fn` have finished (an event wait) and the train continues
    for twice the window behind it. The MFMA kernels here run at a clock the
    power manager sets by load and by board: the same bf16 kernel costs a
    fixed number of shader cycles, so its time moves with this figure."""
    import ctypes
    import math

    import torch

    global _CLOCK_LIB
    if _CLOCK_LIB is None:
        path = ROOT / "trnsparse_amd" / "libtrnsparse_clock.so"
        if not path.exists():
            return None
        lib = ctypes.CDLL(str(path))
        lib.tsp_probe_shader_clock.argtypes = [ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p]
        lib.tsp_probe_shader_clock.restype = ctypes.c_int
        _CLOCK_LIB = lib
    dev = torch.device("cuda", torch.cuda.current_device())
    out = torch.zeros(2, dtype=torch.int64, device=dev)
    side = torch.cuda.Stream(device=dev)
    lead = max(2, int(math.ceil(0.2 * window_ms / per_call_ms)))
    tail = max(4, int(math.ceil(2.0 * window_ms / per_call_ms)))
    torch.cuda.synchronize()
    for _ in range(lead):
        fn()
    started = torch.cuda.Event()
    started.record()
    side.wait_event(started)
    if _CLOCK_LIB.tsp_probe_shader_clock(int(window_ms * 1e5), out.data_ptr(), side.cuda_stream) != 0:
        raise RuntimeError("tsp_probe_shader_clock failed")
    for _ in range(tail):
        fn()
    torch.cuda.synchronize()
    cycles, ticks = out.cpu().tolist()
    return round(cycles / ticks * 0.1, 3) if ticks else None


def host_cpu() -> dict:
    """The GPU box's host CPU as the CPU baselines see it: model name,
    sockets (distinct physical ids), logical CPUs in the machine and in this
    process's affinity mask, and the thread count the baselines use."""
    from oracle import cpu_baseline as cb

    model, phys = None, set()
    try:
        for ln in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
            k, _, v = ln.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name" and model is None:
                model = v
            elif k == "physical id":
                phys.add(v)
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    return {"model": model, "sockets": len(phys) or None, "logical_cpus": os.cpu_count(),
            "affinity_cpus": affinity, "baseline_threads": cb.threads(),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def make_flush():
    """Read 1 GiB to evict L2 and the 256 MiB MALL between timed reps.

    A read (a sum over a buffer written once up front) leaves the caches
    holding clean lines; a write flush would leave the MALL full of dirty
    lines whose write-back the next kernel's misses pay for (measured: the
    cold BSR-SpMV kernel 43.8 us after a 1 GiB fill, 22.6 us after a 1 GiB
    read; the CSR SpMV, gather-bound, 136 vs 135 us)."""
    import torch

    buf = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()

    def flush():
        torch.sum(buf)

    return flush


def _traffic(kernel: str, workload: str):
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        data = json.loads(p.read_text())
        return data.get(f"{kernel}:{workload}")
    except Exception:
        return None


# ------------------------------------------------------------- headline


def bench_bsr_fp32(steps: int, warmup: int, cpu: bool):
    import torch

    import trnsparse_amd as ts
    from trnsparse_amd import workloads as W

    A, B = W.cfg3_bsr(dtype=torch.float32)
    flops = 2.0 * A.n_blocks * 128 * 128 * B.shape[1]
    Ad = ts.BSRMatrix(A.blocks.cuda(), A.block_col_indices, A.block_row_ptrs, A.shape, A.block_size)
    Bd = B.cuda()
    wall_ms, ev_ms = time_gpu(lambda: ts.bsr_spmm(Ad, Bd), steps, warmup)
    achieved = flops / (ev_ms * 1e-3) / 1e12
    res = {
        "value": flops / (wall_ms * 1e-3) / 1e9,
        "ms_per_step": wall_ms,
        "event_ms": ev_ms,
        "flops": flops,
        "shader_ghz": shader_clock_ghz(lambda: ts.bsr_spmm(Ad, Bd), ev_ms),
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": FP32_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
            "traffic": _traffic("bsr_spmm_f32_dma", "cfg3a"),
        },
    }
    if cpu:
        from oracle import cpu_baseline as cb

        nthr = cb.threads()
        torch.set_num_threads(nthr)
        secs, reps = cb.time_call(lambda: cb.bsr_spmm(A.blocks, A.block_col_indices, A.block_row_ptrs, A.shape, 128, B), reps=5)
        res["cpu_baseline"] = {
            "value": round(flops / secs / 1e9, 2),
            "unit": "GFLOP/s",
            "cores": nthr,
            "kind": "port",
            "sample": "full cfg3a (1638 blocks, N=512, fp32) through the reference's torch loop "
            f"(one MKL sgemm per stored block), median of {reps} reps after a warmup, torch threads = {nthr}",
        }
    return res


# ------------------------------------------------------------ secondary


def bench_bsr_small(steps: int, warmup: int):
    """bsr_spmm with block sizes 8, 16, 32 and 64 (bsr_spmm_small) on cfg3's
    dense size (16384 x 16384, N = 512) and block density (10 %, banded plus
    uniform), fp32: GFLOP/s over the stored blocks."""
    import torch

    import trnsparse_amd as ts
    from trnsparse_amd import workloads as W

    out = []
    n, N = 16384, 512
    g = torch.Generator().manual_seed(21)
    B = torch.randn(n, N, generator=g).cuda()
    for b in (8, 16, 32, 64):
        nb = n // b
        mask = W.cfg3_block_mask(nb, half_band=3 * 128 // b, density=0.10, seed=22)
        blocks = torch.randn(int(mask.sum()), b, b, generator=g)
        A = W.bsr_from_block_mask(mask, b, blocks=blocks)
        A = ts.BSRMatrix(A.blocks.cuda(), A.block_col_indices.cuda(), A.block_row_ptrs.cuda(), A.shape, b)
        flops = 2.0 * A.n_blocks * b * b * N
        _, ms = time_gpu(lambda: ts.bsr_spmm(A, B), steps, warmup)
        tf = flops / (ms * 1e-3) / 1e12
        out.append({"name": f"bsr_spmm b={b} 16384^2 10% blocks N=512 fp32", "value": round(tf * 1e3, 1),
                    "unit": "GFLOP/s", "us": round(ms * 1e3, 1), "frac_fp32_mfma": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)})
    return out


def bench_bsr_bf16(steps: int, warmup: int, cpu: bool = False):
    """bsr_spmm at config 3b: bf16 A and B, fp32 accumulation and output.
    `us` is the median of 5 timed segments, `us_spread` their min and max."""
    import torch

    import trnsparse_amd as ts
    from trnsparse_amd import workloads as W

    A, B = W.cfg3_bsr(dtype=torch.bfloat16)
    flops = 2.0 * A.n_blocks * 128 * 128 * B.shape[1]
    Ad = ts.BSRMatrix(A.blocks.cuda(), A.block_col_indices, A.block_row_ptrs, A.shape, A.block_size)
    Bd = B.cuda()
    fwd = lambda: ts.bsr_spmm(Ad, Bd, out_dtype=torch.float32)
    ev_ms, lo, hi = time_gpu_spread(fwd, steps, warmup)
    tf = flops / (ev_ms * 1e-3) / 1e12
    byts = A.n_blocks * 128 * 128 * 2 + B.numel() * 2 + B.numel() * 4
    res = {
        "name": "bsr_spmm cfg3b bf16->fp32",
        "value": round(tf * 1e3, 1),
        "unit": "GFLOP/s",
        "us": round(ev_ms * 1e3, 1),
        "us_spread": [round(lo * 1e3, 1), round(hi * 1e3, 1)],
        "shader_ghz": shader_clock_ghz(fwd, ev_ms),
        "frac_bf16_mfma": round(tf / BF16_MFMA_PEAK_TFLOPS, 4),
        "frac_hbm_min_bytes": round(byts / (ev_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
    }
    if cpu:
        from oracle import cpu_baseline as cb

        nthr = cb.threads()
        torch.set_num_threads(nthr)
        secs, reps = cb.time_call(lambda: cb.bsr_spmm(A.blocks, A.block_col_indices, A.block_row_ptrs, A.shape, 128, B),
                                  reps=5, budget_s=20.0)
        res["cpu_baseline"] = {
            "value": round(flops / secs / 1e9, 2),
            "unit": "GFLOP/s",
            "cores": nthr,
            "kind": "port",
            "sample": "full cfg3b (1638 blocks, N=512) through the reference's torch loop in the input dtype "
            f"(bf16 blocks and B, one torch bf16 matmul per stored block, `+=` into a bf16 output, ops.py:162-192), "
            f"median of {reps} reps after a warmup, torch threads = {nthr}",
        }
    return res


def bench_bsr_small_backward(steps: int, warmup: int):
    """Backward of bsr_spmm at block sizes 8, 16, 32, 64 on the workload of
    bench_bsr_small (16384^2, 10 % blocks, N = 512, fp32): dA (SDDMM on the
    stored pattern, bsr_sddmm_small) and dB = A^T dC (bsr_spmm_small over the
    block-column view), each 2 * nnzb * b^2 * N flops."""
    import torch

    from trnsparse_amd import workloads as W
    from trnsparse_amd.hip import _lib
    from trnsparse_amd.hip import dispatch as D

    out = []
    n, N = 16384, 512
    dev = torch.device("cuda", torch.cuda.current_device())
    g = torch.Generator().manual_seed(21)
    B = torch.randn(n, N, generator=g).to(dev)
    G = torch.randn(n, N, generator=g).to(dev)
    st = _lib.stream_handle(dev)
    code = _lib.dtype_code(torch.float32)
    for b in (8, 16, 32, 64):
        mask = W.cfg3_block_mask(n // b, half_band=3 * 128 // b, density=0.10, seed=22)
        A = W.bsr_from_block_mask(mask, b, blocks=torch.randn(int(mask.sum()), b, b, generator=g))
        rp, ci, blk = A.block_row_ptrs.to(dev), A.block_col_indices.to(dev), A.blocks.to(dev)
        nb = A.n_blocks
        brow, cp, cbid, crow, corder = D._bsr_bwd_plan(rp, ci, n // b, n // b, dev)
        gb = torch.empty_like(blk)
        dB = torch.empty(n, N, device=dev)
        sddmm = lambda: _lib.call("tsp_bsr_sddmm", G.data_ptr(), N, n, B.data_ptr(), N, n, N, brow.data_ptr(),
                                  ci.data_ptr(), nb, b, code, gb.data_ptr(), st)
        spmm_t = lambda: _lib.call("tsp_bsr_spmm_t", blk.data_ptr(), code, cp.data_ptr(), cbid.data_ptr(),
                                   crow.data_ptr(), n // b, b, n, n, G.data_ptr(), N, N, dB.data_ptr(), N,
                                   corder.data_ptr(), st)
        flops = 2.0 * nb * b * b * N
        for name, fn in ((f"bsr_spmm backward dA b={b} 16384^2 10% blocks N=512 fp32", sddmm),
                         (f"bsr_spmm backward dB b={b} 16384^2 10% blocks N=512 fp32", spmm_t)):
            _, ms = time_gpu(fn, steps, warmup)
            tf = flops / (ms * 1e-3) / 1e12
            out.append({"name": name, "value": round(tf * 1e3, 1), "unit": "GFLOP/s", "us": round(ms * 1e3, 1),
                        "frac_fp32_mfma": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)})
    return out


def bench_bsr_backward(steps: int, warmup: int):
    """Backward of bsr_spmm at config 3a (fp32) and 3b (bf16): the two
    kernels the autograd backward launches, each 27.48 GFLOP — tsp_bsr_sddmm
    (dA on the stored pattern) and tsp_bsr_spmm_t (dB = A^T dC over the
    block-column view)."""
    import torch

    from trnsparse_amd import workloads as W
    from trnsparse_amd.hip import _lib
    from trnsparse_amd.hip import dispatch as D

    out = []
    for dt, cfg, peak, key in ((torch.float32, "cfg3a fp32", FP32_MFMA_PEAK_TFLOPS, "frac_fp32_mfma"),
                               (torch.bfloat16, "cfg3b bf16", BF16_MFMA_PEAK_TFLOPS, "frac_bf16_mfma")):
        A, B = W.cfg3_bsr(dtype=dt)
        m, n = A.shape
        N = B.shape[1]
        flops = 2.0 * A.n_blocks * 128 * 128 * N
        dev = torch.device("cuda", torch.cuda.current_device())
        blocks, Bd = A.blocks.to(dev), B.to(dev)
        G = torch.randn(m, N, generator=torch.Generator().manual_seed(9)).to(dt).to(dev)
        rp = A.block_row_ptrs.to(dev)
        ci = A.block_col_indices.to(dev)
        brow, cp, cbid, crow, corder = D._bsr_bwd_plan(rp, ci, 128, 128, dev)
        gb = torch.empty_like(blocks)
        dB = torch.empty(n, N, device=dev, dtype=dt)
        st = _lib.stream_handle(dev)
        code = _lib.dtype_code(dt)
        sddmm = lambda: _lib.call("tsp_bsr_sddmm", G.data_ptr(), N, m, Bd.data_ptr(), N, n, N, brow.data_ptr(),
                                  ci.data_ptr(), A.n_blocks, 128, code, gb.data_ptr(), st)
        spmm_t = lambda: _lib.call("tsp_bsr_spmm_t", blocks.data_ptr(), code, cp.data_ptr(), cbid.data_ptr(),
                                   crow.data_ptr(), 128, 128, m, n, G.data_ptr(), N, N, dB.data_ptr(), N,
                                   corder.data_ptr(), st)
        for name, fn in ((f"bsr_spmm backward dA (sddmm) {cfg}", sddmm), (f"bsr_spmm backward dB (A^T dC) {cfg}", spmm_t)):
            ms, lo, hi = time_gpu_spread(fn, steps, warmup)
            tf = flops / (ms * 1e-3) / 1e12
            out.append({"name": name, "value": round(tf * 1e3, 1), "unit": "GFLOP/s", "us": round(ms * 1e3, 1),
                        "us_spread": [round(lo * 1e3, 1), round(hi * 1e3, 1)], key: round(tf / peak, 4),
                        "shader_ghz": shader_clock_ghz(fn, ms)})
    return out


def bench_bsr_f64(steps: int, warmup: int):
    """bsr_spmm on config 3a's pattern and sizes in fp64 (bsr_spmm_f64_dma)."""
    import torch

    import trnsparse_amd as ts
    from trnsparse_amd import workloads as W

    A, B = W.cfg3_bsr(dtype=torch.float64)
    flops = 2.0 * A.n_blocks * 128 * 128 * B.shape[1]
    Ad = ts.BSRMatrix(A.blocks.cuda(), A.block_col_indices, A.block_row_ptrs, A.shape, A.block_size)
    Bd = B.cuda()
    _, ms = time_gpu(lambda: ts.bsr_spmm(Ad, Bd), steps, warmup)
    tf = flops / (ms * 1e-3) / 1e12
    return {"name": "bsr_spmm cfg3a pattern fp64", "value": round(tf * 1e3, 1), "unit": "GFLOP/s",
            "us": round(ms * 1e3, 1), "frac_fp64_mfma": round(tf / FP64_MFMA_PEAK_TFLOPS, 4)}


def bench_bsr_spmv(steps: int, warmup: int, cpu: bool = False):
    """BSR times one vector (bsr_spmm with N = 1 -> tsp_bsr_spmv) on config
    3's A (fp32, 1638 blocks = 107.4 MB), HBM-bound: algorithmic bytes =
    blocks + x + y + structure, every launch cold (L2 and MALL flushed).
    Then richardson_bsr on an SPD matrix of the same size (128 x 128 blocks
    of 128, band 2 plus 502 symmetric pairs = 1638 blocks), K = 50: one fused
    pass over A per step, A warm in the MALL across steps; bytes per step =
    blocks + 3 vectors read + 1 written."""
    import torch

    import trnsparse_amd as ts
    from trnsparse_amd import workloads as W

    out = []
    A, _ = W.cfg3_bsr(dtype=torch.float32)
    m, n = A.shape
    dev = torch.device("cuda", torch.cuda.current_device())
    Ad = ts.BSRMatrix(A.blocks.to(dev), A.block_col_indices.to(dev), A.block_row_ptrs.to(dev), A.shape, 128)
    x = torch.randn(n, 1, generator=torch.Generator().manual_seed(2)).to(dev)
    flush = make_flush()
    _, ms = time_gpu(lambda: ts.bsr_spmm(Ad, x), steps, warmup, flush=flush)
    byts = A.blocks.numel() * 4 + (n + m) * 4 + (A.n_blocks + A.block_row_ptrs.numel()) * 8
    res = {"name": "bsr_spmm N=1 (BSR-SpMV) cfg3 fp32, cold", "value": round(byts / (ms * 1e-3) / 1e9, 1),
           "unit": "GB/s", "us": round(ms * 1e3, 1), "frac_hbm": round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    if cpu:
        from oracle import cpu_baseline as cb

        xc = x.cpu()
        ptr, col = A.block_row_ptrs, A.block_col_indices
        secs, reps = cb.time_call(lambda: cb.bsr_spmm(A.blocks, col, ptr, A.shape, 128, xc), reps=5, budget_s=10.0)
        res["cpu_baseline"] = {"value": round(byts / secs / 1e9, 2), "unit": "GB/s", "cores": cb.threads(),
                               "kind": "port", "sample": f"the full cfg3 matvec through the reference's torch loop, "
                                                         f"median of {reps} reps after a warmup"}
    out.append(res)
    S, lo, hi = W.spd_bsr(nb=128, b=128, band=2, n_pairs=502)
    Sd = ts.BSRMatrix(S.blocks.to(dev), S.block_col_indices.to(dev), S.block_row_ptrs.to(dev), S.shape, 128)
    rhs = torch.randn(S.shape[0], generator=torch.Generator().manual_seed(3)).to(dev)
    K = 50
    _, ms = time_gpu(lambda: ts.richardson_bsr(Sd, rhs, 2.0 / (lo + hi), K=K), max(2, steps // 5), 1)
    per = ms / (K + 1)  # K steps and the final residual pass
    byts = S.blocks.numel() * 4 + 4 * S.shape[0] * 4
    res = {"name": f"richardson_bsr K={K} SPD 16384^2 ({S.n_blocks} blocks) fp32, fused step",
           "value": round(byts / (per * 1e-3) / 1e9, 1), "unit": "GB/s", "us_per_step": round(per * 1e3, 1),
           "us_total": round(ms * 1e3, 1)}
    if cpu:
        from oracle import cpu_baseline as cb

        ptr, col = S.block_row_ptrs, S.block_col_indices
        rc = rhs.cpu()

        def ref_steps(k=3):
            xx = torch.zeros_like(rc)
            for _ in range(k):
                xx = xx + (2.0 / (lo + hi)) * (rc - cb.bsr_spmm(S.blocks, col, ptr, S.shape, 128, xx[:, None])[:, 0])
            return xx

        secs, reps = cb.time_call(ref_steps, reps=5, budget_s=10.0)
        secs /= 3
        res["cpu_baseline"] = {"value": round(byts / secs / 1e9, 2), "unit": "GB/s", "cores": cb.threads(),
                               "kind": "port", "sample": f"3 Richardson steps through the reference's torch loop, "
                                                         f"median of {reps} reps after a warmup"}
    out.append(res)
    return out


def bench_spmv(dist: str, index_bits: int, steps: int, warmup: int, cpu: bool = False, plan: str = "always"):
    """CSR SpMV at config 2: algorithmic HBM bytes / kernel time, L2+MALL
    flushed before every timed launch (the working set fits in the MALL).

    plan "always": the column-sorted plan (tsp_csr_colplan_spmv; built once
    per matrix outside the timed region, its build time reported beside);
    plan "never": the windowed kernel over the caller's CSR arrays
    (tsp_csr_spmv, deterministic); plan "bucketed": the row-per-wavefront
    kernels with long rows split out by length (tsp_csr_bucketed_spmv, plan
    built outside the timed region). `algorithmic_bytes` is the reference
    layout's traffic (nnz*(4+idx) + (m+1)*idx + 4n + 4m) and defines `value`
    and `frac_hbm`; `kernel_bytes` is what the kernels themselves have to move
    (the plan's 8-byte entries, x twice, y, the column groups' partial sums
    and the row exponents)."""
    import numpy as np
    import torch

    import trnsparse_amd as ts
    from trnsparse_amd import workloads as W
    from trnsparse_amd.hip import dispatch as D

    idt = np.int64 if index_bits == 64 else np.int32
    v, c, p, x, shape = W.cfg2_csr(dist=dist, index_dtype=idt)
    m, n = shape
    nnz = len(v)
    A = W.csr_matrix_from_arrays(v, c, p, shape, device="cuda")
    xd = torch.from_numpy(x).cuda()
    ib = index_bits // 8
    byts = nnz * (4 + ib) + (m + 1) * ib + n * 4 + m * 4
    prev = D.get_spmv_plan()
    D.set_spmv_plan(plan)
    try:
        build_ms = None
        kbytes = byts
        if plan == "always":
            ts.spmv(A, xd)  # builds the plan (the first use also loads the kernels)
            # build time on a second matrix object of the same pattern, after
            # the one-time kernel loading
            A2 = W.csr_matrix_from_arrays(v, c, p, shape, device="cuda")
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            ts.spmv(A2, xd)
            torch.cuda.synchronize()
            build_ms = (time.perf_counter() - t0) * 1e3
            del A2
            geom = A._hip_colplan[2]
            G = int(geom[3])
            # 8-byte entry per nonzero, x (the max pre-pass and the gathers' slices), y, the
            # column groups' partial sums written and read, the row exponents
            kbytes = nnz * 8 + 2 * n * 4 + m * 4 + 2 * G * m * 4 + 2 * m
        if plan == "bucketed":
            ts.spmv(A, xd)  # builds the bucket plan
        flush = make_flush()
        _, ev_ms = time_gpu(lambda: ts.spmv(A, xd), steps, warmup, flush=flush)
        buckets = A._hip_bucket_plan[1][1:] if plan == "bucketed" else None
    finally:
        D.set_spmv_plan(prev)
    gbs = byts / (ev_ms * 1e-3) / 1e9
    kind = {"always": "column-sorted plan", "bucketed": "length-bucketed rows"}.get(plan, "windowed")
    res = {
        "name": f"csr_spmv cfg2 {dist} int{index_bits} ({kind})",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "us": round(ev_ms * 1e3, 2),
        "nnz": nnz,
        "algorithmic_bytes": byts,
        "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
        "timing": f"median of {steps} launches, each after a 1 GiB read flush of L2 and MALL",
    }
    if buckets is not None:
        res["rows_medium_long"] = list(buckets)
    if plan == "always":
        res["kernel_bytes"] = kbytes
        res["frac_hbm_kernel_bytes"] = round(kbytes / (ev_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        res["plan_build_ms"] = round(build_ms, 2)
        res["plan_geometry"] = {"rows_per_tile": 1 << int(geom[0]), "cols_per_group": 1 << int(geom[2]),
                                "groups": G, "tiles": int(geom[4])}
    if cpu:
        from oracle import build as oracle_c
        from oracle import cpu_baseline as cb

        nthr = cb.threads()
        torch.set_num_threads(nthr)
        vt, ct, pt, xt = (torch.from_numpy(a) for a in (v, c, p, x))
        secs, reps = cb.time_call(lambda: cb.spmv(vt, ct, pt, shape, xt), reps=5, budget_s=15.0)
        res["cpu_baseline"] = {"value": round(byts / secs / 1e9, 2), "unit": "GB/s", "cores": nthr,
                               "kind": "port",
                               "sample": f"full cfg2 matrix through the reference's CPU path "
                                         f"(torch.sparse_csr_tensor @ x, ops.py:25-45), median of {reps} reps "
                                         f"after a warmup, torch threads = {nthr}"}
        csecs, creps = cb.time_call(lambda: oracle_c.csr_spmv_f32(v, c, p, m, x), reps=5, budget_s=10.0)
        res["cpu_c_loop"] = {"value": round(byts / csecs / 1e9, 2), "unit": "GB/s", "cores": nthr,
                             "sample": f"oracle/csr_spmv.c fp32 OpenMP over rows, median of {creps} reps"}
    return res


def bench_spmm(steps: int, warmup: int):
    """CSR SpMM (spmm) with config 2's matrix (poisson rows, int64 indices)
    and dense B of N = 8 and 64 columns. Reported as GFLOP/s (2 nnz N) and as
    the bytes the kernel requests: the stream (values, indices, row offsets),
    one B row slice per nonzero and the output — B rows are re-read from
    cache, so this is a request rate, not HBM traffic."""
    import torch

    import trnsparse_amd as ts
    from trnsparse_amd import workloads as W

    v, c, p, _, shape = W.cfg2_csr()
    m, n = shape
    nnz = len(v)
    A = W.csr_matrix_from_arrays(v, c, p, shape, device="cuda")
    out = []
    for N in (8, 64):
        B = torch.randn(n, N, generator=torch.Generator().manual_seed(N)).cuda()
        _, ms = time_gpu(lambda: ts.spmm(A, B), steps, warmup)
        req = nnz * 12 + (m + 1) * 8 + nnz * N * 4 + m * N * 4
        out.append({"name": f"csr_spmm cfg2 poisson int64, B {n}x{N} fp32", "value": round(2.0 * nnz * N / (ms * 1e-3) / 1e9, 1),
                    "unit": "GFLOP/s", "us": round(ms * 1e3, 1), "requested_GBps": round(req / (ms * 1e-3) / 1e9, 1)})
    return out


def bench_screened(steps: int, warmup: int, cpu: bool = False):
    """screened_spmm at config 4 (n=4096, threshold 1e-20): GFLOP/s counting
    the 128x128 A tiles that are not fully screened, and dense-equivalent."""
    import numpy as np
    import torch

    import trnsparse_amd as ts
    from trnsparse_amd import workloads as W

    A, diag, B, thr = W.cfg4_screened()
    n = A.shape[0]
    Q = torch.sqrt(torch.abs(diag))
    qmax = Q.view(-1, 128).amax(dim=1)
    active = int(((qmax[:, None] * qmax[None, :]) > np.float32(np.sqrt(thr))).sum())
    flops = 2.0 * 128 * 128 * B.shape[1] * active
    dense_flops = 2.0 * n * n * B.shape[1]
    Ad, dd, Bd = A.cuda(), diag.cuda(), B.cuda()
    _, ev_ms = time_gpu(lambda: ts.screened_spmm(Ad, dd, Bd, thr), steps, warmup)
    tf = flops / (ev_ms * 1e-3) / 1e12
    res = {
        "name": "screened_spmm cfg4 n=4096 fp32",
        "value": round(tf * 1e3, 1),
        "unit": "GFLOP/s",
        "us": round(ev_ms * 1e3, 1),
        "active_tiles": active,
        "dense_equiv_gflops": round(dense_flops / (ev_ms * 1e-3) / 1e9, 1),
        "frac_fp32_mfma": round(tf / FP32_MFMA_PEAK_TFLOPS, 4),
    }
    if cpu:
        from oracle import cpu_baseline as cb

        secs, reps = cb.time_call(lambda: cb.screened_spmm(A, diag, B, thr), reps=5, budget_s=20.0)
        res["cpu_baseline"] = {"value": round(flops / secs / 1e9, 2), "unit": "GFLOP/s", "cores": cb.threads(),
                               "kind": "port", "sample": f"full cfg4 through the reference's torch path (mask, A*mask, "
                                                         f"MKL sgemm), median of {reps} reps after a warmup"}
    # the same workload with fp64 A, diag and B (screened_f64_dma)
    A64, d64, B64 = Ad.double(), dd.double(), Bd.double()
    _, ms64 = time_gpu(lambda: ts.screened_spmm(A64, d64, B64, thr), max(2, steps // 2), warmup)
    tf64 = flops / (ms64 * 1e-3) / 1e12
    res64 = {"name": "screened_spmm cfg4 n=4096 fp64", "value": round(tf64 * 1e3, 1),
             "unit": "GFLOP/s", "us": round(ms64 * 1e3, 1), "frac_fp64_mfma": round(tf64 / FP64_MFMA_PEAK_TFLOPS, 4)}
    del A64, d64, B64
    # backward in fp32 (tsp_screened_spmm_backward: dA and dB, each a product
    # over the active tile pairs with the same flop count as the forward)
    from trnsparse_amd.hip import dispatch as Dp

    G = torch.randn(B.shape, generator=torch.Generator().manual_seed(9)).cuda()
    dev = Ad.device
    _, msb = time_gpu(lambda: Dp._screened_backward(Ad, dd, thr, Bd, G, True, True, dev), max(2, steps // 2), warmup)
    tfb = 2 * flops / (msb * 1e-3) / 1e12
    resb = {"name": "screened_spmm backward cfg4 n=4096 fp32 (dA and dB)", "value": round(tfb * 1e3, 1),
            "unit": "GFLOP/s", "us": round(msb * 1e3, 1), "frac_fp32_mfma": round(tfb / FP32_MFMA_PEAK_TFLOPS, 4),
            "dense_equiv_gflops": round(2 * dense_flops / (msb * 1e-3) / 1e9, 1)}
    return [res, res64, resb]


def bench_attention(steps: int, warmup: int, cpu: bool = False):
    """block_sparse_attention_tiled at config 5: 32 heads x 8192 x 128 bf16,
    370 stored 128x128 blocks. FLOPs = 4 * nnzb * 128^2 * d * heads."""
    import torch

    import trnsparse_amd as ts
    from trnsparse_amd import workloads as W

    Q, K, V, mask = W.cfg5_attention()
    H, S, D = Q.shape
    flops = 4.0 * mask.n_blocks * 128 * 128 * D * H
    byts = 4 * H * S * D * 2
    Qd, Kd, Vd = Q.cuda(), K.cuda(), V.cuda()
    fwd = lambda: ts.block_sparse_attention_tiled(Qd, Kd, Vd, mask)
    ev_ms, lo, hi = time_gpu_spread(fwd, steps, warmup)
    tf = flops / (ev_ms * 1e-3) / 1e12
    res = {
        "name": "block_sparse_attention cfg5 32x8192x128 bf16",
        "value": round(tf * 1e3, 1),
        "unit": "GFLOP/s",
        "us": round(ev_ms * 1e3, 1),
        "us_spread": [round(lo * 1e3, 1), round(hi * 1e3, 1)],
        "shader_ghz": shader_clock_ghz(fwd, ev_ms),
        "frac_bf16_mfma": round(tf / BF16_MFMA_PEAK_TFLOPS, 4),
        "frac_hbm_min_bytes": round(byts / (ev_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
    }
    if cpu:
        from oracle import cpu_baseline as cb

        b = 128
        ptr, col = mask.block_row_ptrs, mask.block_col_indices
        secs, reps = cb.time_call(lambda: cb.attention_head(Q[0], K[0], V[0], ptr, col, b, D**-0.5), reps=5,
                                  budget_s=20.0)
        res["cpu_baseline"] = {"value": round(flops / H / secs / 1e9, 2), "unit": "GFLOP/s", "cores": cb.threads(),
                               "kind": "port", "sample": f"one head of cfg5 (bf16) through the reference's torch "
                                                         f"two-pass loops, median of {reps} reps after a warmup"}
    # the same workload with fp32 Q / K / V (bsa_fwd_f32_mfma)
    Qf, Kf, Vf = (t.float() for t in (Qd, Kd, Vd))
    _, ms32 = time_gpu(lambda: ts.block_sparse_attention_tiled(Qf, Kf, Vf, mask), steps, warmup)
    tf32 = flops / (ms32 * 1e-3) / 1e12
    res32 = {"name": "block_sparse_attention cfg5 32x8192x128 fp32", "value": round(tf32 * 1e3, 1), "unit": "GFLOP/s",
             "us": round(ms32 * 1e3, 1), "frac_fp32_mfma": round(tf32 / FP32_MFMA_PEAK_TFLOPS, 4)}
    return [res, res32]


def bench_attention_d256(steps: int, warmup: int):
    """Config 5's mask and shape at head_dim 256 (32 heads x 8192 x 256):
    forward in bf16 (bsa_fwd_bf16_stream<256>) and fp32
    (bsa_fwd_f32_mfma<256>), backward in fp32 (the 16-row-tile row and
    column passes). FLOPs as the head_dim-128 lines: 4 (forward) and 10
    (backward) x nnzb x 128^2 x d x heads."""
    import torch

    import trnsparse_amd as ts
    from trnsparse_amd import workloads as W
    from trnsparse_amd.hip import _lib
    from trnsparse_amd.hip import dispatch as Dp

    Q, K, V, mask = W.cfg5_attention(d=256)
    H, S, D = Q.shape
    out = []
    dev = torch.device("cuda", torch.cuda.current_device())
    for dt in (torch.bfloat16, torch.float32):
        Qd, Kd, Vd = (t.to(dt).to(dev) for t in (Q, K, V))
        _, ms = time_gpu(lambda: ts.block_sparse_attention_tiled(Qd, Kd, Vd, mask), steps, warmup)
        tf = 4.0 * mask.n_blocks * 128 * 128 * D * H / (ms * 1e-3) / 1e12
        peak, key, tag = ((BF16_MFMA_PEAK_TFLOPS, "frac_bf16_mfma", "bf16") if dt == torch.bfloat16 else
                          (FP32_MFMA_PEAK_TFLOPS, "frac_fp32_mfma", "fp32"))
        out.append({"name": f"block_sparse_attention cfg5 mask 32x8192x256 {tag}", "value": round(tf * 1e3, 1),
                    "unit": "GFLOP/s", "us": round(ms * 1e3, 1), key: round(tf / peak, 4)})
        del Qd, Kd, Vd
    rp, ci, _ = Dp._bsr_plan(mask.block_col_indices, mask.block_row_ptrs, S // 128, dev, holder=mask)
    cp, crow, nbc, plan, (ni, ns, npart) = Dp._attn_bwd_plan(mask, H, S, dev)
    ws = torch.empty(_lib.load().tsp_bsa_bwd_workspace_size(H, S, D, npart), dtype=torch.uint8, device=dev)
    Qd, Kd, Vd = (t.float().to(dev) for t in (Q, K, V))
    dO = torch.randn(Q.shape, generator=torch.Generator().manual_seed(14)).to(dev)
    O, rm, rd = Dp.hip_block_sparse_attention(Qd, Kd, Vd, mask, D**-0.5, return_stats=True)
    dQ, dK, dV = (torch.empty_like(Qd) for _ in range(3))
    st = _lib.stream_handle(dev)
    call = lambda: _lib.call("tsp_bsa_bwd", Qd.data_ptr(), Kd.data_ptr(), Vd.data_ptr(), O.data_ptr(), dO.data_ptr(),
                             _lib.TSP_F32, H, S, D, rp.data_ptr(), ci.data_ptr(), cp.data_ptr(), crow.data_ptr(), nbc,
                             128, D**-0.5, rm.data_ptr(), rd.data_ptr(), dQ.data_ptr(), dK.data_ptr(), dV.data_ptr(),
                             plan.data_ptr(), ni, ns, npart, ws.data_ptr(), st)
    _, ms = time_gpu(call, steps, warmup)
    tf = 10.0 * mask.n_blocks * 128 * 128 * D * H / (ms * 1e-3) / 1e12
    out.append({"name": "block_sparse_attention backward cfg5 mask 32x8192x256 fp32", "value": round(tf * 1e3, 1),
                "unit": "GFLOP/s", "us": round(ms * 1e3, 1), "frac_fp32_mfma": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)})
    return out


def bench_attention_blocks(steps: int, warmup: int):
    """Config 5's mask and shape (32 heads x 8192) on the block-product path:
    bf16 backward at head_dim 256, and forward and backward at head_dim 512 in
    bf16 and fp32 (SDDMM scores, block softmax / gradient, BSR SpMMs over the
    mask stacked over heads); the bf16 forward at 512 also on the one-pass
    kernel the API runs. FLOPs as the other attention lines: 4 (forward)
    and 10 (backward) x nnzb x 128^2 x d x heads. Each step is the whole
    sequence of launches; `us` is the median of 5 timed segments."""
    import torch

    from trnsparse_amd import workloads as W
    from trnsparse_amd.hip import dispatch as Dp

    out = []
    dev = torch.device("cuda", torch.cuda.current_device())
    for d, dt, fwd in ((256, torch.bfloat16, False), (512, torch.bfloat16, True), (512, torch.float32, True)):
        Q, K, V, mask = W.cfg5_attention(d=d)
        H, S, D = Q.shape
        Qd, Kd, Vd = (t.to(dt).to(dev) for t in (Q, K, V))
        del Q, K, V
        tag = "bf16" if dt == torch.bfloat16 else "fp32"
        peak, key = ((BF16_MFMA_PEAK_TFLOPS, "frac_bf16_mfma") if dt == torch.bfloat16 else
                     (FP32_MFMA_PEAK_TFLOPS, "frac_fp32_mfma"))
        O, rm, rd = Dp.hip_block_sparse_attention(Qd, Kd, Vd, mask, D**-0.5, return_stats=True)
        if fwd:
            # bf16 at 512: the one-pass kernel (tsp_bsa_fwd), and the block
            # products beside it; fp32: block products
            runs = [("block products", lambda: Dp._attention_blocks_fwd(Qd, Kd, Vd, mask, D**-0.5, dev))]
            if dt == torch.bfloat16:
                runs.insert(0, ("one pass", lambda: Dp.hip_block_sparse_attention(Qd, Kd, Vd, mask, D**-0.5,
                                                                                   return_stats=True)))
            for how, fn in runs:
                ms, lo, hi = time_gpu_spread(fn, steps, warmup)
                tf = 4.0 * mask.n_blocks * 128 * 128 * D * H / (ms * 1e-3) / 1e12
                out.append({"name": f"block_sparse_attention cfg5 mask 32x8192x{D} {tag} ({how})",
                            "value": round(tf * 1e3, 1), "unit": "GFLOP/s", "us": round(ms * 1e3, 1),
                            "us_spread": [round(lo * 1e3, 1), round(hi * 1e3, 1)], key: round(tf / peak, 4)})
        dO = torch.randn(Qd.shape, generator=torch.Generator().manual_seed(14)).to(dt).to(dev)
        rmf, rdf = rm.reshape(H, S), rd.reshape(H, S)
        ms, lo, hi = time_gpu_spread(lambda: Dp._attention_blocks_bwd(Qd, Kd, Vd, O, dO, mask, D**-0.5, rmf, rdf, dev),
                                     steps, warmup)
        tf = 10.0 * mask.n_blocks * 128 * 128 * D * H / (ms * 1e-3) / 1e12
        out.append({"name": f"block_sparse_attention backward cfg5 mask 32x8192x{D} {tag} (block products)",
                    "value": round(tf * 1e3, 1), "unit": "GFLOP/s", "us": round(ms * 1e3, 1),
                    "us_spread": [round(lo * 1e3, 1), round(hi * 1e3, 1)], key: round(tf / peak, 4)})
        del Qd, Kd, Vd, O, dO, rm, rd
        torch.cuda.empty_cache()
    return out


def bench_attention_backward(steps: int, warmup: int, cpu: bool = False):
    """Backward of block_sparse_attention_tiled at config 5 (tsp_bsa_bwd: the
    row pass for dQ, the column pass for dK / dV and the reduce of split
    columns), from the forward's O and stats. Algorithmic FLOPs: the five
    block products of the backward (S, dP = dO V^T, dV, dK, dQ), 10 * nnzb *
    128^2 * d * heads; the kernels recompute S and dP in both passes (7
    products)."""
    import torch

    from trnsparse_amd import workloads as W
    from trnsparse_amd.hip import _lib
    from trnsparse_amd.hip import dispatch as Dp

    Q, K, V, mask = W.cfg5_attention()
    H, S, D = Q.shape
    flops = 10.0 * mask.n_blocks * 128 * 128 * D * H
    dev = torch.device("cuda", torch.cuda.current_device())
    rp, ci, _ = Dp._bsr_plan(mask.block_col_indices, mask.block_row_ptrs, S // 128, dev, holder=mask)
    cp, crow, nbc, plan, (ni, ns, npart) = Dp._attn_bwd_plan(mask, H, S, dev)
    st = _lib.stream_handle(dev)
    ws = torch.empty(_lib.load().tsp_bsa_bwd_workspace_size(H, S, D, npart), dtype=torch.uint8, device=dev)
    out = []
    for dt in (torch.bfloat16, torch.float32):
        Qd, Kd, Vd = Q.to(dt).to(dev), K.to(dt).to(dev), V.to(dt).to(dev)
        dO = torch.randn(Q.shape, generator=torch.Generator().manual_seed(14)).to(torch.bfloat16).to(dt).to(dev)
        O, rm, rd = Dp.hip_block_sparse_attention(Qd, Kd, Vd, mask, D**-0.5, return_stats=True)
        dQ, dK, dV = (torch.empty_like(Qd) for _ in range(3))
        code = _lib.dtype_code(dt)
        call = lambda: _lib.call("tsp_bsa_bwd", Qd.data_ptr(), Kd.data_ptr(), Vd.data_ptr(), O.data_ptr(), dO.data_ptr(),
                                 code, H, S, D, rp.data_ptr(), ci.data_ptr(), cp.data_ptr(), crow.data_ptr(), nbc, 128,
                                 D**-0.5, rm.data_ptr(), rd.data_ptr(), dQ.data_ptr(), dK.data_ptr(), dV.data_ptr(),
                                 plan.data_ptr(), ni, ns, npart, ws.data_ptr(), st)
        ms, lo, hi = time_gpu_spread(call, steps, warmup)
        tf = flops / (ms * 1e-3) / 1e12
        peak, key, tag = ((BF16_MFMA_PEAK_TFLOPS, "frac_bf16_mfma", "bf16") if dt == torch.bfloat16 else
                          (FP32_MFMA_PEAK_TFLOPS, "frac_fp32_mfma", "fp32"))
        out.append({"name": f"block_sparse_attention backward cfg5 32x8192x128 {tag}", "value": round(tf * 1e3, 1),
                    "unit": "GFLOP/s", "us": round(ms * 1e3, 1), "us_spread": [round(lo * 1e3, 1), round(hi * 1e3, 1)],
                    key: round(tf / peak, 4), "split_columns": ns, "items": ni, "shader_ghz": shader_clock_ghz(call, ms)})
        if dt == torch.bfloat16:
            keep = (Qd, Kd, Vd, O, dO, rm, rd)
    res = out[0]
    Qd, Kd, Vd, O, dO, rm, rd = keep
    if cpu:
        from oracle import cpu_baseline as cb

        args = [t[0].cpu() for t in (Qd, Kd, Vd, O, dO)]
        r0, d0 = rm[0].reshape(-1).cpu().to(torch.bfloat16), rd[0].reshape(-1).cpu().to(torch.bfloat16)
        secs, reps = cb.time_call(lambda: cb.attention_backward_head(*args, mask.block_row_ptrs, mask.block_col_indices,
                                                                     128, D**-0.5, r0, d0), reps=5, budget_s=20.0)
        res["cpu_baseline"] = {"value": round(flops / H / secs / 1e9, 2), "unit": "GFLOP/s", "cores": cb.threads(),
                               "kind": "port",
                               "sample": f"one head of cfg5 (bf16) through the reference's torch backward loops, "
                                         f"median of {reps} reps after a warmup"}
    return out


def bench_formats(steps: int, warmup: int, cpu: bool = False):
    """Device format construction at config 3's dense size (16384^2 fp32,
    1638 nonzero 128x128 blocks): BSRMatrix.from_dense (algorithmic bytes:
    read A once, read + write the kept blocks), formats.from_dense to CSR
    (read A twice: count pass and fill pass; write values and int64
    columns) and COOMatrix.to_csr of that matrix's entries (read rows, cols,
    values; write columns, values and row pointers; the sort's own passes
    are not counted). Each call includes its host read of the entry count."""
    import torch

    import trnsparse_amd as ts
    from trnsparse_amd import workloads as W

    A, _ = W.cfg3_bsr(dtype=torch.float32)
    dev = torch.device("cuda", torch.cuda.current_device())
    D = ts.BSRMatrix(A.blocks.to(dev), A.block_col_indices.to(dev), A.block_row_ptrs.to(dev), A.shape, 128).to_dense()
    m, n = D.shape
    kept = A.blocks.numel() * 4
    out = []
    _, ms = time_gpu(lambda: ts.BSRMatrix.from_dense(D, block_size=128), steps, warmup)
    byts = m * n * 4 + 2 * kept
    res = {"name": "BSRMatrix.from_dense cfg3 16384^2 fp32 (device)", "value": round(byts / (ms * 1e-3) / 1e9, 1),
           "unit": "GB/s", "us": round(ms * 1e3, 1), "frac_hbm": round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    if cpu:
        from oracle import cpu_baseline as cb

        Dc = D.cpu()
        secs, reps = cb.time_call(lambda: cb.bsr_from_dense(Dc, 128), reps=5, budget_s=20.0)
        res["cpu_baseline"] = {"value": round(byts / secs / 1e9, 2), "unit": "GB/s", "cores": cb.threads(),
                               "kind": "port", "sample": f"the full cfg3 dense matrix through the reference's torch "
                                                         f"ops, median of {reps} reps after a warmup"}
    out.append(res)
    csr = ts.from_dense(D)
    nnz = csr.nnz
    _, ms = time_gpu(lambda: ts.from_dense(D), steps, warmup)
    byts = 2 * m * n * 4 + nnz * 12 + (m + 1) * 8
    out.append({"name": "formats.from_dense (CSR) cfg3 16384^2 fp32 (device)", "nnz": nnz,
                "value": round(byts / (ms * 1e-3) / 1e9, 1), "unit": "GB/s", "us": round(ms * 1e3, 1),
                "frac_hbm": round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
    coo = csr.to_coo()
    perm = torch.randperm(nnz, generator=torch.Generator().manual_seed(3)).to(dev)
    shuffled = ts.COOMatrix(coo.values[perm], coo.row_indices[perm], coo.col_indices[perm], coo.shape)
    _, ms = time_gpu(lambda: shuffled.to_csr(), steps, warmup)
    byts = nnz * (8 + 8 + 4) + nnz * (8 + 4) + (m + 1) * 8
    out.append({"name": "COOMatrix.to_csr cfg3 entries shuffled (device)", "nnz": nnz,
                "value": round(byts / (ms * 1e-3) / 1e9, 1), "unit": "GB/s", "us": round(ms * 1e3, 1)})
    return out


def bench_csr_ops(steps: int, warmup: int):
    """The remaining CSR ops on the device at config 2 (1 M x 1 M, Poisson(16)
    rows, 16.8 M entries, fp32 values, int64 indices): sparse_transpose
    (stable sort of 32-bit column keys carrying (row, value)),
    sparse_add(A, A^T) (sort of 33.6 M (row, col) keys carrying the values +
    segmented sum) and spmv_symmetric (two CSR
    SpMVs, the strict transpose cached). Reported in entries per second;
    the sorts dominate the first two."""
    import numpy as np
    import torch

    import trnsparse_amd as ts
    from trnsparse_amd import workloads as W

    v, c, p, x, shape = W.cfg2_csr(dist="poisson", index_dtype=np.int64)
    A = ts.CSRMatrix(torch.from_numpy(v).cuda(), torch.from_numpy(c).cuda(), torch.from_numpy(p).cuda(), shape)
    xd = torch.from_numpy(x).cuda()
    nnz = A.nnz
    T = ts.sparse_transpose(A)
    out = []
    for name, fn, ent in (("sparse_transpose", lambda: ts.sparse_transpose(A), nnz),
                          ("sparse_add(A, A^T)", lambda: ts.sparse_add(A, T), 2 * nnz),
                          ("spmv_symmetric (strict transpose cached)", lambda: ts.spmv_symmetric(A, xd), 2 * nnz)):
        _, ms = time_gpu(fn, steps, warmup)
        out.append({"name": f"{name} cfg2 1M^2 fp32 (device)", "value": round(ent / (ms * 1e-3) / 1e6, 1),
                    "unit": "M entries/s", "us": round(ms * 1e3, 1)})
    return out


def calibrate_peaks():
    """Achievable peaks on this box next to the spec ones: a 1 GiB device copy
    (read + write bytes / time), and dense 8192^3 GEMMs in fp32 and bf16
    through torch (hipBLASLt), each after the clock pre-warm."""
    import torch

    res = {}
    a = torch.ones(1 << 28, device="cuda")
    b = torch.empty_like(a)
    _, ms = time_gpu(lambda: b.copy_(a), 20, 3)
    res["copy_1GiB_GBps"] = round(2 * a.numel() * 4 / (ms * 1e-3) / 1e9, 1)
    res["hbm_spec_GBps"] = HBM_PEAK_GBS
    del a, b
    n = 8192
    for dt, name, peak in ((torch.float32, "fp32", FP32_MFMA_PEAK_TFLOPS), (torch.bfloat16, "bf16", BF16_MFMA_PEAK_TFLOPS)):
        x = torch.randn(n, n, device="cuda").to(dt)
        y = torch.randn(n, n, device="cuda").to(dt)
        _, ms = time_gpu(lambda: x @ y, 10, 3)
        tf = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
        res[f"gemm_{name}_8192_TFLOPs"] = round(tf, 1)
        res[f"gemm_{name}_spec_TFLOPs"] = peak
        res[f"gemm_{name}_frac_of_spec"] = round(tf / peak, 4)
    return res


def calibrate_gather():
    """What the x gathers cost at cfg2. torch.index_select(x, 0, cols) with
    cfg2's column indices (uniform over 1 M) and with sequential indices has
    the same streaming traffic (16.8 M int64 indices read, 16.8 M fp32
    written); only the gathers' locality differs. spmv is timed beside them.
    Every launch is cold (L2 and MALL flushed)."""
    import numpy as np
    import torch

    import trnsparse_amd as ts
    from trnsparse_amd import workloads as W

    v, c, p, x, shape = W.cfg2_csr(dist="poisson", index_dtype=np.int64)
    m, n = shape
    A = W.csr_matrix_from_arrays(v, c, p, shape, device="cuda")
    xd = torch.from_numpy(x).cuda()
    cols = torch.from_numpy(c).cuda()
    seq = torch.arange(len(c), device="cuda", dtype=torch.int64) % n
    flush = make_flush()
    res = {"nnz": len(c), "n": n}
    for name, fn in (("index_select_random_us", lambda: torch.index_select(xd, 0, cols)),
                     ("index_select_sequential_us", lambda: torch.index_select(xd, 0, seq)),
                     ("spmv_us", lambda: ts.spmv(A, xd))):
        _, ms = time_gpu(fn, 15, 3, flush=flush)
        res[name] = round(ms * 1e3, 2)
    res["random_gather_penalty_us"] = round(res["index_select_random_us"] - res["index_select_sequential_us"], 2)
    return res


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-secondary", action="store_true", help="headline only")
    ap.add_argument("--only", metavar="JOB", default=None,
                    help="run only the named secondary job (e.g. 'spmv poisson int64') and print its result; for "
                    "profiling one kernel")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a plain 256 MiB device copy (known bytes) to calibrate PMC byte counters")
    ap.add_argument("--calibrate-peaks", action="store_true",
                    help="run only the achievable-peak calibration: 1 GiB device copy, fp32 and bf16 dense "
                    "GEMMs (torch/hipBLASLt) beside the spec peaks")
    ap.add_argument("--calibrate-gather", action="store_true",
                    help="run only the SpMV gather-floor calibration on cfg2 (torch index_select, random vs "
                    "sequential indices, next to spmv)")
    args = ap.parse_args(argv)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}); "
            "this build has no multi-GPU path",
            file=sys.stderr,
        )
        return 2

    import torch

    import trnsparse_amd as ts
    from trnsparse_amd.hip import _lib

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    if args.calibrate_peaks:
        print(json.dumps(calibrate_peaks()), flush=True)
        return 0
    if args.calibrate_copy:
        a = torch.ones(1 << 26, device="cuda")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes_read": a.numel() * 4, "calibrate_copy_bytes_written": b.numel() * 4}))
        return 0
    _lib.load()
    ts.set_backend("hip")
    if args.calibrate_gather:
        print(json.dumps(calibrate_gather()), flush=True)
        return 0

    secondary = []
    if args.only is None:
        head = bench_bsr_fp32(args.steps, args.warmup, cpu=not args.no_cpu)
    if not args.no_secondary:
        jobs = [
            ("spmv poisson int64", lambda: bench_spmv("poisson", 64, 20, 3, cpu=not args.no_cpu)),
            ("spmv poisson int32", lambda: bench_spmv("poisson", 32, 20, 3)),
            ("spmv zipf int64", lambda: bench_spmv("zipf", 64, 10, 2)),
            ("spmv windowed poisson int64", lambda: bench_spmv("poisson", 64, 20, 3, plan="never")),
            ("spmv windowed poisson int32", lambda: bench_spmv("poisson", 32, 20, 3, plan="never")),
            ("spmv windowed zipf int64", lambda: bench_spmv("zipf", 64, 10, 2, plan="never")),
            ("spmv bucketed poisson int64", lambda: bench_spmv("poisson", 64, 20, 3, plan="bucketed")),
            ("spmv bucketed zipf int64", lambda: bench_spmv("zipf", 64, 10, 2, plan="bucketed")),
            ("spmm", lambda: bench_spmm(10, 2)),
            ("bsr bf16", lambda: bench_bsr_bf16(max(5, args.steps // 2), 3, cpu=not args.no_cpu)),
            ("bsr f64", lambda: bench_bsr_f64(10, 2)),
            ("bsr small", lambda: bench_bsr_small(10, 2)),
            ("bsr small backward", lambda: bench_bsr_small_backward(3, 1)),
            ("bsr backward", lambda: bench_bsr_backward(10, 2)),
            ("screened", lambda: bench_screened(10, 2, cpu=not args.no_cpu)),
            ("attention", lambda: bench_attention(10, 2, cpu=not args.no_cpu)),
            ("attention backward", lambda: bench_attention_backward(10, 2, cpu=not args.no_cpu)),
            ("attention d256", lambda: bench_attention_d256(5, 2)),
            ("attention blocks", lambda: bench_attention_blocks(3, 1)),
            ("formats", lambda: bench_formats(5, 1, cpu=not args.no_cpu)),
            ("bsr spmv", lambda: bench_bsr_spmv(20, 3, cpu=not args.no_cpu)),
            ("csr ops", lambda: bench_csr_ops(5, 1)),
        ]
        if args.only is not None:
            chosen = [j for j in jobs if j[0] == args.only]
            if not chosen:
                print(f"--only: no job named {args.only!r}; jobs: {[j[0] for j in jobs]}", file=sys.stderr)
                return 2
            print(json.dumps(chosen[0][1]()), flush=True)
            return 0
        for name, fn in jobs:
            try:
                r = fn()
                secondary.extend(r if isinstance(r, list) else [r])
            except Exception as exc:  # report, do not hide
                secondary.append({"name": name, "error": repr(exc)})
            print(f"# done: {name}", file=sys.stderr, flush=True)

    line = {
        "metric": "bsr_spmm effective GFLOP/s (nnz blocks) + % MFMA peak; CSR SpMV HBM GB/s",
        "value": round(head["value"], 1),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "bsr_spmm cfg3a: A 16384x16384 in 128x128 blocks, band |i-j|<=3 + uniform off-band, "
            "10% block density (1638 blocks), B 16384x512 N(0,1), fp32 in/out, seed 2",
            "n_blocks": 1638,
            "block_size": 128,
            "ncols": 512,
            "flops_per_step": head["flops"],
        },
        "roofline": head["roofline"],
        "shader_ghz": head.get("shader_ghz"),
        "cpu_baseline": head.get("cpu_baseline"),
        "host_cpu": host_cpu(),
        "secondary": secondary,
        "timing": "HIP events on the launch stream; untimed 0.25 s clock pre-warm of the same op, then the W warmup steps; "
        "shader_ghz: shader clock during a separate back-to-back train of the same op (s_memtime against the 100 MHz "
        "s_memrealtime, one probe wave on a side stream)",
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
