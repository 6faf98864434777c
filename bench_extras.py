"""GEMM and SpMV legs of bench.py (inputs generated on device, resident before timing)."""
from __future__ import annotations

import numpy as np


def bench_gemm(ctx, log, time_launches, roofline, fp32_peak, bf16_peak, sizes=(1024, 4096, 8192)) -> dict:
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
                                     "roofline": roofline("mfma", tflops, bf16_peak, "TFLOP/s")}
            log(f"[bench] gemm_bf16 {n}^3: {ms:.3f} ms -> {tflops:.1f} TFLOP/s ({100 * tflops / bf16_peak:.1f}% of bf16)")
            ctx.free(ab)
            ctx.free(bb)
        for x in (a, b, c):
            ctx.free(x)
    return out


def bench_spmv(ctx, log, time_launches, roofline, hbm_peak, sizes=(1_000_000, 16_000_000), iters=20) -> dict:
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
        # the column-sliced plan: analysis once, then SpMV through it
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
    return out
