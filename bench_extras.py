"""GEMM and SpMV legs of bench.py (inputs generated on device, resident before timing), and the
bounded CPU baselines timed beside each leg.

The CPU baselines run the oracle's C restatements of the reference's CPU algorithms on the same
seeded inputs (the counter-based generator gives the host the same elements the device fill
wrote). They are reported beside the GPU figures, never measured as the product.
"""
from __future__ import annotations

import os
import statistics
import time

import numpy as np


def host_cores() -> int:
    """Threads the multi-threaded CPU baselines use: this process's CPU share, at most 16."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def cpu_median(fn, reps: int, budget_s: float, warm: bool = False):
    """Median host wall time (s) of fn() over up to `reps` timed runs (fewer once `budget_s` of timed
    work has accumulated; at least one), after one untimed run when `warm`."""
    if warm:
        fn()
    ts = []
    while len(ts) < reps and (not ts or sum(ts) < budget_s):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return statistics.median(ts), len(ts)


def runs(r: int) -> str:
    return f"median of {r} runs" if r > 1 else "one run"


def cpu_baseline(value: float, unit: str, cores: int, sample: str, **more) -> dict:
    d = {"value": float(f"{value:.4g}"), "unit": unit, "cores": cores, "kind": "port", "sample": sample}
    d.update(more)
    return d


def gemm_cpu_baseline(n: int, cores: int, log) -> dict:
    """OptimizedMatrixMultiplyKernel's parallel-for over rows with the naive i-j-k fp32 loop (oracle
    restatement) on the same A and B. Above 1024 a subset of rows is timed (every row costs the same
    n*n multiply-adds) and the full-matrix time is extrapolated from it."""
    import oracle

    rows = n if n <= 1024 else 2 * cores
    a = oracle.gen_uniform_f32(rows * n, 42, 0).reshape(rows, n)  # rows [0, rows) of the device's A
    b = oracle.gen_uniform_f32(n * n, 43, 0).reshape(n, n)
    t, reps = cpu_median(lambda: oracle.gemm_f32_naive(a, b, threads=cores), 3, 2.5)
    tflops = 2.0 * rows * n * n / t / 1e12
    full_ms = t * n / rows * 1e3
    sample = (f"all {n} rows" if rows == n else f"rows 0..{rows - 1} of {n}, full-matrix time extrapolated "
              f"x{n // rows}") + f"; {runs(reps)} of the oracle's naive i-j-k fp32 loop on {cores} threads"
    log(f"[bench] cpu gemm_f32 {n}: {tflops * 1e3:.2f} GFLOP/s ({full_ms:.0f} ms full matrix, {sample})")
    return cpu_baseline(tflops, "TFLOP/s", cores, sample, ms=round(full_ms, 1))


def bench_gemm(ctx, log, time_launches, roofline, fp32_peak, bf16_peak, sizes=(1024, 4096, 8192),
               cpu_cores: int | None = None) -> dict:
    out = {}
    for n in sizes:
        a = ctx.empty((n, n), np.float32)
        b = ctx.empty((n, n), np.float32)
        c = ctx.empty((n, n), np.float32)
        ctx.fill_uniform_f32(a, seed=42, stream=0)
        ctx.fill_uniform_f32(b, seed=43, stream=0)
        f = lambda: ctx.gemm_f32(a, b, c, n, n, n)
        f()
        ctx.synchronize()
        iters = 20 if n <= 4096 else 5
        ms = time_launches(ctx, f, iters)
        tflops = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
        out[f"gemm_f32_{n}"] = {"ms": round(ms, 4), "TFLOP/s": round(tflops, 2),
                                "roofline": roofline("mfma", tflops, fp32_peak, "TFLOP/s")}
        log(f"[bench] gemm_f32 {n}^3: {ms:.3f} ms -> {tflops:.1f} TFLOP/s ({100 * tflops / fp32_peak:.1f}% of fp32 MFMA)")
        if cpu_cores:
            out[f"gemm_f32_{n}"]["cpu_baseline"] = gemm_cpu_baseline(n, cpu_cores, log)
        if n == sizes[-1]:
            ab = ctx.empty((n, n), np.uint16)
            bb = ctx.empty((n, n), np.uint16)
            ctx.convert_f32_to_bf16(a, ab)
            ctx.convert_f32_to_bf16(b, bb)
            g = lambda: ctx.gemm_bf16(ab, bb, c, n, n, n)
            g()
            ctx.synchronize()
            ms = time_launches(ctx, g, 10)
            tflops = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
            out[f"gemm_bf16_{n}"] = {"ms": round(ms, 4), "TFLOP/s": round(tflops, 2),
                                     "roofline": roofline("mfma", tflops, bf16_peak, "TFLOP/s"),
                                     "cpu_baseline": None,
                                     "cpu_baseline_note": "the reference has no bf16 CPU GEMM to restate"}
            log(f"[bench] gemm_bf16 {n}^3: {ms:.3f} ms -> {tflops:.1f} TFLOP/s ({100 * tflops / bf16_peak:.1f}% of bf16)")
            ctx.free(ab)
            ctx.free(bb)
        for x in (a, b, c):
            ctx.free(x)
    return out


def vendor_times(warm_ms: float, gemm_sizes=(1024, 4096, 8192), n_stream: int = 1 << 28) -> list:
    """The same operations composed from torch's own ops, which run ROCm's vendor kernels (hipBLASLt
    for torch.mm, torch's HIP kernels for the rest), as a reference point for this library's
    kernels: torch.mm on the GEMM legs' shapes (fp32, and bf16 inputs with an fp32 result at the
    largest size), and at n_stream float32 elements (uniform [-1, 1)) `x[x > 0] * 2 + 1` (the
    headline ToArray; the boolean index waits for its count on the host, as torch's must),
    `x.sum()`, `torch.where(x > 0, x * 2 + 1, 0).sum()` and `torch.add(a, b, out=c)`. Timed like
    the legs: untimed calls until the device has been busy for `warm_ms`, then HIP events around
    back-to-back calls on torch's stream. The results are not checked (they are not this
    library's). Runs in a process of its own (see vendor_run)."""
    import torch

    torch.backends.cuda.matmul.allow_tf32 = False
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(42)

    def timed(fn, iters):
        t0 = time.perf_counter()
        for _ in range(1000):
            fn()
            torch.cuda.synchronize()
            if (time.perf_counter() - t0) * 1e3 >= warm_ms:
                break
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) / iters

    res = []
    for n in gemm_sizes:
        a = torch.rand(n, n, device=dev, generator=g)
        b = torch.rand(n, n, device=dev, generator=g)
        c = torch.empty(n, n, device=dev)
        cases = [(f"gemm_f32_{n}", lambda: torch.mm(a, b, out=c), "torch.mm fp32")]
        if n == gemm_sizes[-1]:
            ab, bb = a.bfloat16(), b.bfloat16()
            cases.append((f"gemm_bf16_{n}", lambda: torch.mm(ab, bb, out_dtype=torch.float32),
                          "torch.mm bf16 inputs, out_dtype float32"))
        for leg, fn, what in cases:
            ms = timed(fn, 20 if n <= 4096 else 10)
            res.append({"leg": leg, "call": what, "torch": torch.__version__, "ms": round(ms, 4),
                        "TFLOP/s": round(2.0 * n ** 3 / (ms * 1e-3) / 1e12, 2)})
        del a, b, c
    n = n_stream
    x = torch.rand(n, device=dev, generator=g).mul_(2.0).sub_(1.0)
    kept = int((x > 0).sum().item())
    y = torch.rand(n, device=dev, generator=g)
    z = torch.empty(n, device=dev)
    for leg, fn, what, nbytes in (
            ("headline", lambda: x[x > 0] * 2 + 1, "x[x > 0] * 2 + 1", 4 * n + 4 * kept),
            ("sum_f32_256M", lambda: x.sum(), "x.sum()", 4 * n),
            ("where_select_sum_f32_256M", lambda: torch.where(x > 0, x * 2 + 1, 0).sum(),
             "torch.where(x > 0, x * 2 + 1, 0).sum()", 4 * n),
            ("vector_add_f32_256M", lambda: torch.add(x, y, out=z), "torch.add(a, b, out=c)", 12 * n)):
        ms = timed(fn, 20)
        res.append({"leg": leg, "call": what, "torch": torch.__version__, "ms": round(ms, 4),
                    "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1)})
    del x, y, z
    torch.cuda.synchronize()
    return res


def vendor_run(warm_ms: float) -> list:
    """vendor_times in a child process (this file run as a script) that the caller starts before it
    touches the GPU itself: torch brings its own HIP runtime, which does not find the device once
    this library's runtime holds it in the same process."""
    import json
    import subprocess
    import sys

    cmd = [sys.executable, os.path.abspath(__file__), "--vendor", str(warm_ms)]
    p = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    if p.returncode != 0:
        raise RuntimeError(f"vendor timing failed (exit {p.returncode}): {p.stderr[-2000:]}")
    return json.loads(p.stdout.strip().splitlines()[-1])


def attach_vendor(out: dict, res: list, log) -> None:
    """Record each vendor time beside its leg of `out` as `vendor` (this_over_vendor_time < 1: this
    library is faster); the `headline` entry is left to the caller."""
    for v in res:
        v = dict(v)
        leg = v.pop("leg")
        if leg in out:
            v["this_over_vendor_time"] = round(out[leg]["ms"] / v["ms"], 3)
            out[leg]["vendor"] = v
        rate = f"{v['TFLOP/s']:.1f} TFLOP/s" if "TFLOP/s" in v else f"{v['GB/s']:.0f} GB/s"
        log(f"[bench] vendor {leg}: {v['ms']:.3f} ms -> {rate} ({v['call']})")


def spmv_cpu_baseline(rp, col, val, rows: int, iters: int, per_iter_bytes: int, log) -> dict:
    """SparseMatrix.Multiply's row loop followed by the L1 normalisation (oracle restatement, one
    thread) on the same CSR matrix and start vector. Above 10M non-zeros one iteration is timed and
    the x`iters` time extrapolated (every iteration does the same work)."""
    import oracle

    x0 = oracle.gen_uniform_f32(rows, 42, 5, unit_interval=True)
    n_it = iters if val.size < 10_000_000 else 1
    t, reps = cpu_median(lambda: oracle.spmv_power_f32(rp, col, val, x0, n_it), 3, 2.0)
    full_s = t * iters / n_it
    gbs = iters * per_iter_bytes / full_s / 1e9
    sample = (f"{n_it} iteration{'s' if n_it > 1 else ''}" + (f", x{iters} extrapolated" if n_it < iters else "")
              + f"; {runs(reps)} of the oracle's single-thread CSR row loop + L1 normalisation")
    log(f"[bench] cpu spmv x{iters} rows={rows}: {gbs:.2f} GB/s ({full_s * 1e3:.0f} ms, {sample})")
    return cpu_baseline(gbs, "GB/s", 1, sample, ms=round(full_s * 1e3, 1))


def bench_spmv(ctx, log, time_launches, roofline, hbm_peak, sizes=(1_000_000, 16_000_000), iters=20,
               cpu: bool = False) -> dict:
    from dotcompute_amd import hip

    out = {}
    for rows in sizes:
        rp, col, val = hip.gen_zipf_csr(rows, 42)
        nnz = int(rp[-1])
        drp, dcol, dval = ctx.to_device(rp), ctx.to_device(col), ctx.to_device(val)
        x0 = ctx.empty(rows, np.float32)
        x = ctx.empty(rows, np.float32)
        y = ctx.empty(rows, np.float32)
        ctx.fill_uniform_f32(x0, seed=42, stream=5, unit_interval=True)

        def run():
            hip.check(hip.load().dc_hip_memcpy_d2d_async(ctx.handle, x.ptr, x0.ptr, 4 * rows), "d2d")
            ctx.spmv_power_iterate_f32(drp, dcol, dval, x, y, rows, nnz, iters)

        run()
        ctx.synchronize()
        ms = time_launches(ctx, run, 3)
        # algorithmic bytes per iteration: values + columns, row pointers, x gathers (once per
        # distinct column, lower bound 4*cols), y write, then the L1 normalisation (read y twice,
        # write x)
        per_iter = 8 * nnz + 4 * (rows + 1) + 4 * rows + 4 * rows + 12 * rows
        gbs = iters * per_iter / (ms * 1e-3) / 1e9
        single = lambda: ctx.spmv_csr_f32(drp, dcol, dval, x, y, rows, rows, nnz)
        ms1 = time_launches(ctx, single, 10)
        spmv_bytes = 8 * nnz + 4 * (rows + 1) + 4 * rows + 4 * rows
        gbs1 = spmv_bytes / (ms1 * 1e-3) / 1e9
        # the tiled plan: analysis once, then SpMV through it
        t_build = ctx.event(), ctx.event()
        t_build[0].record()
        plan = ctx.spmv_plan(drp, dcol, dval, rows, rows, nnz)
        t_build[1].record()
        t_build[1].synchronize()
        ms_build = t_build[0].elapsed_ms(t_build[1])
        for e in t_build:
            e.destroy()
        slices, slice_cols, plan_bytes = plan.info()
        plan.execute(x, y)
        ctx.synchronize()
        ms_plan = time_launches(ctx, lambda: plan.execute(x, y), 20)
        gbs_plan = spmv_bytes / (ms_plan * 1e-3) / 1e9
        plan.destroy()
        out[f"spmv_power20_{rows // 1_000_000}M"] = {
            "ms": round(ms, 4), "nnz": nnz, "mean_degree": round(nnz / rows, 3), "GB/s": round(gbs, 1),
            "iter_ms": round(ms / iters, 4),
            "roofline": roofline("hbm", gbs, hbm_peak, "GB/s"),
            "single_spmv_ms": round(ms1, 4), "single_spmv_GB/s": round(gbs1, 1),
            "plan_build_ms": round(ms_build, 4), "plan_slices": slices, "plan_slice_cols": slice_cols,
            "plan_device_bytes": plan_bytes, "plan_spmv_ms": round(ms_plan, 4), "plan_spmv_GB/s": round(gbs_plan, 1)}
        log(f"[bench] spmv x{iters} rows={rows} nnz={nnz}: {ms:.3f} ms ({ms / iters * 1e3:.1f} us/iter) -> {gbs:.0f} GB/s;"
            f" single SpMV {ms1 * 1e3:.1f} us -> {gbs1:.0f} GB/s; plan build {ms_build * 1e3:.0f} us ({slices} slices),"
            f" plan SpMV {ms_plan * 1e3:.1f} us -> {gbs_plan:.0f} GB/s")
        for a in (drp, dcol, dval, x0, x, y):
            ctx.free(a)
        if cpu:
            out[f"spmv_power20_{rows // 1_000_000}M"]["cpu_baseline"] = spmv_cpu_baseline(
                rp, col, val, rows, iters, per_iter, log)
    return out


def stream_cpu_baselines(extra: dict, hx: np.ndarray, cores: int, log) -> None:
    """CPU baselines of the 256M streaming legs (Sum, fused Where->Select->Sum/Min/Max, VectorAdd),
    added to the legs already in `extra`. `hx` is the 256M headline input generated on the host."""
    import oracle

    n = hx.size
    mib = n * 4 // (1 << 20)
    if "sum_f32_256M" in extra:
        t, r = cpu_median(lambda: oracle.sum_f32_partitioned(hx, cores), 5, 1.0, warm=True)
        t1, r1 = cpu_median(lambda: oracle.sum_f32_enumerable(hx), 3, 1.0)
        extra["sum_f32_256M"]["cpu_baseline"] = cpu_baseline(
            4 * n / t / 1e9, "GB/s", cores, f"full input ({mib} MiB), {runs(r)} of OptimizedReductionKernel's "
            f"one-double-partial-per-thread sum over {cores} threads", ms=round(t * 1e3, 2))
        extra["sum_f32_256M"]["cpu_baseline_sequential"] = cpu_baseline(
            4 * n / t1 / 1e9, "GB/s", 1, f"full input, {runs(r1)} of Enumerable.Sum's sequential double "
            f"accumulator", ms=round(t1 * 1e3, 2))
        log(f"[bench] cpu sum_f32: {4 * n / t / 1e9:.1f} GB/s on {cores} threads, {4 * n / t1 / 1e9:.1f} GB/s sequential")
    if "sum_i32_256M" in extra:
        xi = oracle.gen_uniform_i32(n, 43, 1)
        t, r = cpu_median(lambda: oracle.sum_i32_bcl(xi), 3, 1.0)
        extra["sum_i32_256M"]["cpu_baseline"] = cpu_baseline(
            4 * n / t / 1e9, "GB/s", 1, f"full input, {runs(r)} of checked Enumerable.Sum(int) (the BCL's "
            f"8-lane overflow-tracked loop, restated in scalar C)", ms=round(t * 1e3, 2))
        log(f"[bench] cpu sum_i32: {4 * n / t / 1e9:.1f} GB/s")
        del xi
    if "where_select_sum_f32_256M" in extra:
        res = []
        t, r = cpu_median(lambda: res.append(oracle.where_gt0_select_2x_plus_1_sum(hx)), 3, 2.0)
        leg = extra["where_select_sum_f32_256M"]
        leg["cpu_baseline"] = cpu_baseline(
            4 * n / t / 1e9, "GB/s", 1, f"full input, {runs(r)} of LINQ-to-objects "
            f"Where(x>0f).Select(x*2f+1f).Sum() with the lambdas written out", ms=round(t * 1e3, 2),
            count_matches_gpu=bool(res[-1][2] == leg["count"]))
        log(f"[bench] cpu where_select_sum: {4 * n / t / 1e9:.2f} GB/s")
    for name in ("min", "max"):
        label = f"where_select_{name}_f32_256M"
        if label not in extra:
            continue
        res = []
        t, r = cpu_median(lambda: res.append(oracle.where_gt0_select_2x_plus_1_minmax(hx, name)), 3, 2.0)
        leg = extra[label]
        leg["cpu_baseline"] = cpu_baseline(
            4 * n / t / 1e9, "GB/s", 1, f"full input, {runs(r)} of LINQ-to-objects "
            f"Where(x>0f).Select(x*2f+1f).{name.capitalize()}() with the lambdas written out",
            ms=round(t * 1e3, 2), value_matches_gpu=bool(np.float32(leg["value"]) == res[-1][0]))
        log(f"[bench] cpu where_select_{name}: {4 * n / t / 1e9:.2f} GB/s")
    for nv, full, label, reps in ((100_000, 100_000, "vector_add_f32_100K", 200),
                                  (32 << 20, n, "vector_add_f32_256M", 3)):
        if label not in extra:
            continue
        a = hx[:nv]
        b = oracle.gen_uniform_f32(nv, 42, 1)  # the device leg's second operand (seed 42, stream 1)
        o = np.empty(nv, np.float32)
        t, r = cpu_median(lambda: oracle.vector_add_f32(a, b, o), reps, 0.5, warm=True)
        sample = (f"full input, {runs(r)}" if nv == full else
                  f"first {nv >> 20}M of the {full >> 20}M elements, {runs(r)}") + \
            " of the generated scalar [Kernel] CPU invoker loop into a preallocated result"
        extra[label]["cpu_baseline"] = cpu_baseline(12 * nv / t / 1e9, "GB/s", 1, sample,
                                                    ms=round(t * full / nv * 1e3, 4))
        log(f"[bench] cpu {label}: {12 * nv / t / 1e9:.2f} GB/s")


def bench_orchestrator(log, cpu: bool = True) -> dict:
    """The README quick start end to end: IComputeOrchestrator.ExecuteAsync("VectorAdd", "HIP", a, b,
    result) on host arrays of 100,000 floats through the C++ orchestrator (pooled device buffers; the
    two inputs copied in, the result copied back), and ExecuteWithBuffersAsync on device-resident
    buffers. Runs dotcompute_amd/lib/dc_orchestrator_bench in a child process."""
    import json
    import subprocess

    exe = os.path.join(os.path.dirname(os.path.abspath(__file__)), "dotcompute_amd", "lib", "dc_orchestrator_bench")
    r = subprocess.run([exe, "100000", "300"], capture_output=True, text=True, timeout=120)
    if r.returncode != 0:
        log(f"[bench] orchestrator bench failed ({r.returncode}): {r.stderr.strip()[-300:]}")
        return {}
    d = json.loads(r.stdout.strip().splitlines()[-1])
    us = d["execute_async_us"]["median"]
    leg = {"us_per_call": us, "GB/s_host_arrays": round(12 * d["n"] / (us * 1e-6) / 1e9, 2),
           "device_resident_us_per_call": d["execute_with_buffers_us"]["median"],
           "launch_and_wait_us": d["launch_and_wait_us"]["median"], "idle_wait_us": d["idle_wait_us"],
           "h2d_input_us": d["h2d_input_us"], "d2h_result_us": d["d2h_result_us"], "bit_exact": d["bit_exact"],
           "note": "host arrays: 2 inputs in (the result is never read by the kernel, so it is not copied in), "
                   "launch, result out, synchronised per call; PCIe-bound, not an HBM roofline. "
                   "launch_and_wait_us: the same compiled kernel launched directly with a prebuilt argument "
                   "block and waited for, the floor under the device-resident call"}
    log(f"[bench] orchestrator VectorAdd 100K: {us:.1f} us per ExecuteAsync (device-resident "
        f"{leg['device_resident_us_per_call']:.1f} us, of which launch and wait {leg['launch_and_wait_us']:.1f} us; "
        f"h2d {d['h2d_input_us']:.1f} us, d2h {d['d2h_result_us']:.1f} us)")
    if cpu:
        import oracle

        a = oracle.gen_uniform_f32(100_000, 42, 0)
        b = oracle.gen_uniform_f32(100_000, 42, 1)
        o = np.empty(100_000, np.float32)
        t, reps = cpu_median(lambda: oracle.vector_add_f32(a, b, o), 300, 0.5, warm=True)
        leg["cpu_baseline"] = cpu_baseline(t * 1e6, "us per call", 1, f"{runs(reps)} of the generated scalar [Kernel] "
                                           "CPU invoker loop over the same host arrays (the reference's CPU path "
                                           "adds a Task.Run around it)", higher_is_better=False)
    return {"vector_add_100K_orchestrator_e2e": leg}


if __name__ == "__main__":
    import json
    import sys

    if len(sys.argv) == 3 and sys.argv[1] == "--vendor":
        print(json.dumps(vendor_times(float(sys.argv[2]))))
    else:
        sys.exit("usage: bench_extras.py --vendor WARM_MS (bench.py --vendor runs it)")
