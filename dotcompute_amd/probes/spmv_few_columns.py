"""Measurement program: the tiled SpMV plan on matrices with few columns (one or two x slices, so
the row pass's per-block run table has one or two runs). Times plan.execute with HIP events on
the context's stream and prints one line per matrix. Run from the repository root on a gfx950
box after the library is built: python3 dotcompute_amd/probes/spmv_few_columns.py"""
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))

import numpy as np  # noqa: E402

from bench import time_launches  # noqa: E402
from dotcompute_amd import hip  # noqa: E402


def main() -> None:
    ctx = hip.Context(0)
    for rows, cols in ((4_000_000, 4096), (4_000_000, 1000), (4_000_000, 65536)):
        rp, col, val = hip.gen_zipf_csr(rows, 11, max_degree=min(4096, cols - 1), cols=cols)
        x = hip.gen_uniform_f32(cols, 11, 5, True)
        drp, dcol, dval = ctx.to_device(rp), ctx.to_device(col), ctx.to_device(val)
        dx, dy = ctx.to_device(x), ctx.empty(rows, np.float32)
        with ctx.spmv_plan(drp, dcol, dval, rows, cols, col.size, 0) as plan:
            slices, width, _ = plan.info()
            run = lambda: plan.execute(dx, dy)  # noqa: E731
            run()
            ctx.synchronize()
            ms = time_launches(ctx, run, 20, warm_ms=100)
        gbs = (8 * col.size + 4 * (rows + 1) + 4 * rows + 4 * cols) / (ms * 1e-3) / 1e9
        print(f"rows {rows} cols {cols} nnz {col.size} slices {slices} width {width}: {ms * 1e3:.1f} us per SpMV "
              f"({gbs:.0f} GB/s of CSR + x + y)", flush=True)
        for a in (drp, dcol, dval, dx, dy):
            ctx.free(a)
    ctx.close()


if __name__ == "__main__":
    main()
