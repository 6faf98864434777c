"""GPU parity: the column-sliced SpMV plan (dc_hip_spmv_plan_*), which the power iteration uses.

Reference semantics: SparseOps.SpMV (SparseMatrix.cs:669-692), a sequential float32 row sum. The
plan sums each row slice by slice: partial_s = sequential sum of the row's products whose column
falls in slice s (index order) for segments of at most 32 products (longer ones: a fixed-order
wave reduction), then y = 0.0f + partial_0 + partial_1 + ... in slice order. Two checks per case:
  - parity: |y - y64| <= 1e-4 * sum_i |v_i x_c(i)| per row, y64 the float64 row sum;
  - exactness of the order: rows whose segments are all at most 32 nonzeros must equal, bit for
    bit, the same slice-ordered sum composed from the oracle's sequential float32 SpMV applied to
    each slice's sub-matrix (a different order than one sequential pass would be caught).
"""
import numpy as np
import pytest

import oracle
from dotcompute_amd import hip

pytestmark = pytest.mark.gpu

REL = 1e-4
SEQ_SEG = 32  # segments up to this length are summed sequentially on the GPU


def upload_csr(ctx, rp, col, val):
    return ctx.to_device(rp), ctx.to_device(col if col.size else np.zeros(1, np.int32)), \
        ctx.to_device(val if val.size else np.zeros(1, np.float32))


def row_scale(rp, col, val, x):
    return oracle.spmv_csr_f64(rp, col, np.abs(val), np.abs(x).astype(np.float64))


def sliced_reference(rp, col, val, x, width):
    """Slice-ordered float32 sum from the oracle's sequential SpMV on each slice's sub-matrix; also
    returns, per row, whether any of its segments is longer than SEQ_SEG (tree-summed on the GPU)."""
    rows = rp.size - 1
    slices = (int(x.size) + width - 1) // width
    row_of = np.repeat(np.arange(rows), np.diff(rp))
    y = np.zeros(rows, np.float32)
    has_long = np.zeros(rows, bool)
    for s in range(slices):
        keep = (col // width) == s
        counts = np.bincount(row_of[keep], minlength=rows).astype(np.int64)
        sub_rp = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
        part = oracle.spmv_csr_f32(sub_rp, np.ascontiguousarray(col[keep]), np.ascontiguousarray(val[keep]), x)
        y = (y + part).astype(np.float32)
        has_long |= counts > SEQ_SEG
    return y, has_long


def run_plan(ctx, rp, col, val, x, slice_cols_max=0, repeat=2):
    rows = rp.size - 1
    drp, dcol, dval = upload_csr(ctx, rp, col, val)
    dx = ctx.to_device(x)
    dy = ctx.empty(max(rows, 1), np.float32)
    with ctx.spmv_plan(drp, dcol, dval, rows, x.size, col.size, slice_cols_max) as plan:
        info = plan.info()
        ys = []
        for _ in range(repeat):
            plan.execute(dx, dy)
            ctx.synchronize()
            ys.append(dy.to_host(rows))
    for a in (drp, dcol, dval, dx, dy):
        ctx.free(a)
    for y in ys[1:]:
        assert np.array_equal(y.view(np.uint32), ys[0].view(np.uint32)), "plan execution is not deterministic"
    return ys[0], info


def check(rp, col, val, x, y, width):
    ref64 = oracle.spmv_csr_f64(rp, col, val, x.astype(np.float64))
    assert np.all(np.abs(y - ref64) <= REL * row_scale(rp, col, val, x) + 1e-30)
    ref32, has_long = sliced_reference(rp, col, val, x, width)
    ok = ~has_long
    assert np.array_equal(y[ok].view(np.uint32), ref32[ok].view(np.uint32))


# (rows, cols, slice_cols_max) -> expected number of slices. Default width (0): one slice up to
# 512 KB of x, else 2 / 4 / 8 slices up to 1 / 2 / 4 MB (an XCD's share of x at most 512 KB).
SHAPES = [
    (5000, 5000, 0, 1),
    (200_000, 200_000, 0, 2),
    (600_000, 600_000, 0, 8),
    (5000, 5000, 2500, 2),
    (5000, 5000, 1250, 4),
    (5000, 5000, 625, 8),
    (5000, 5000, 300, 24),
    (20000, 20000, 100, 32),     # capped at 32 slices: wider than asked
    (3000, 70000, 4000, 24),     # rectangular, more columns than rows
    (1, 1, 0, 1),
    (64, 64, 16, 4),
]


@pytest.mark.parametrize("rows,cols,width,slices", SHAPES)
def test_plan_slices_vs_oracle(ctx, rows, cols, width, slices):
    seed = rows + cols + width
    if cols == 1:  # a 1x1 matrix: the generator avoids self-loops, so give the row its one entry
        rp, col, val = np.array([0, 1], np.int32), np.zeros(1, np.int32), np.ones(1, np.float32)
    else:
        rp, col, val = oracle.gen_zipf_csr(rows, seed, max_degree=min(4096, cols - 1), cols=cols)
    x = oracle.gen_uniform_f32(cols, seed, 5, unit_interval=True)
    y, (s, w, nbytes) = run_plan(ctx, rp, col, val, x, width)
    assert s == slices and w == (cols + s - 1) // s and nbytes > 0
    check(rp, col, val, x, y, w)


def test_plan_signed_values_and_long_segments(ctx):
    """Negative values, rows of 0 / 1 / 4096 / 3000 nonzeros; segments summed sequentially (up to
    32), by the whole wave (33-256) and by a workgroup (longer), at each threshold; empty rows
    exactly zero."""
    lens = [0, 1, 4096, 0, 3000, 7, 129, 128, 0, 600, 257, 256, 513, 512, 32, 33, 31, 64, 65]
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cols = 5000
    col = (np.arange(rp[-1]) * 7919 % cols).astype(np.int32)
    val = oracle.gen_uniform_f32(int(rp[-1]), 9, 0)
    x = oracle.gen_uniform_f32(cols, 9, 1)
    for width, slices in ((0, 1), (2500, 2), (625, 8)):
        y, (s, w, _) = run_plan(ctx, rp, col, val, x, width)
        assert s == slices
        check(rp, col, val, x, y, w)
        assert y[0] == 0 and y[3] == 0 and y[8] == 0


def test_plan_one_slice_equals_sequential_reference(ctx):
    """One slice (asked for with a slice width of all the columns): every row is one segment, so
    rows of at most 32 nonzeros (about 99% of the rows of this graph) are the sequential float32
    row sum of SparseOps.SpMV bit for bit."""
    rows = 300_000
    rp, col, val = oracle.gen_zipf_csr(rows, 7)
    x = oracle.gen_uniform_f32(rows, 7, 5, unit_interval=True)
    y, (s, _, _) = run_plan(ctx, rp, col, val, x, rows, repeat=1)
    assert s == 1
    ref = oracle.spmv_csr_f32(rp, col, val, x)
    short = np.diff(rp) <= SEQ_SEG
    assert short.sum() > 0.98 * rows
    assert np.array_equal(y[short].view(np.uint32), ref[short].view(np.uint32))


@pytest.mark.parametrize("width,slices", [(1 << 16, 16), (1 << 15, 32), (1 << 18, 4)])
def test_plan_1m_many_slices(ctx, width, slices):
    rows = 1_000_000
    rp, col, val = oracle.gen_zipf_csr(rows, 42)
    x = oracle.gen_uniform_f32(rows, 42, 5, unit_interval=True)
    y, (s, w, _) = run_plan(ctx, rp, col, val, x, width, repeat=2)
    assert s == slices
    check(rp, col, val, x, y, w)


@pytest.mark.parametrize("width", [0, 1 << 16])
def test_plan_power_iteration_1m_vs_oracle(ctx, width):
    rows, iters = 1_000_000, 20
    rp, col, val = oracle.gen_zipf_csr(rows, 42)
    x0 = oracle.gen_uniform_f32(rows, 42, 5, unit_interval=True)
    drp, dcol, dval = upload_csr(ctx, rp, col, val)
    dx = ctx.to_device(x0)
    dy = ctx.empty(rows, np.float32)
    s = ctx.empty(1, np.float64)
    with ctx.spmv_plan(drp, dcol, dval, rows, rows, col.size, width) as plan:
        # the plan owns a copy of the matrix: the CSR arrays can go once the build has run
        ctx.synchronize()
        for a in (drp, dcol, dval):
            ctx.free(a)
        plan.power_iterate(dx, dy, iters, s)
        ctx.synchronize()
    x = dx.to_host()
    ref_x, ref_s = oracle.spmv_power_f32(rp, col, val, x0, iters)
    assert abs(s.to_host()[0] - ref_s) <= REL * abs(ref_s)
    assert np.all(np.abs(x - ref_x) <= REL * np.abs(ref_x) + 1e-12)
    assert abs(float(np.sum(x, dtype=np.float64)) - 1.0) < 1e-4
    for a in (dx, dy, s):
        ctx.free(a)


def test_plan_empty_matrices(ctx):
    # rows but no nonzeros: y must be all zeros
    rows = 1000
    rp = np.zeros(rows + 1, np.int32)
    x = np.ones(rows, np.float32)
    y, (s, _, _) = run_plan(ctx, rp, np.zeros(0, np.int32), np.zeros(0, np.float32), x, 0, repeat=1)
    assert s == 1 and np.all(y == 0)


def test_plan_argument_errors(ctx):
    L = hip.load()
    rp = ctx.to_device(np.array([0, 1], np.int32))
    col = ctx.to_device(np.array([0], np.int32))
    val = ctx.to_device(np.array([1.0], np.float32))
    import ctypes as C

    h = C.c_void_p()
    assert L.dc_hip_spmv_plan_create(ctx.handle, rp.ptr, col.ptr, val.ptr, 1, 1, 1, -1, C.byref(h)) == hip.DC_ERR_INVALID_ARGUMENT
    assert L.dc_hip_spmv_plan_create(ctx.handle, rp.ptr, col.ptr, val.ptr, 1, 0, 1, 0, C.byref(h)) == hip.DC_ERR_INVALID_ARGUMENT
    assert L.dc_hip_spmv_plan_create(ctx.handle, rp.ptr, col.ptr, val.ptr, 1, 1, 1, 0, None) == hip.DC_ERR_INVALID_ARGUMENT
    # a 1x2 matrix is not square: the power iteration refuses it before any work is queued
    with ctx.spmv_plan(rp, col, val, 1, 2, 1) as plan:
        x = ctx.empty(2, np.float32)
        y = ctx.empty(1, np.float32)
        st = L.dc_hip_spmv_plan_power_iterate_f32(ctx.handle, plan.handle, x.ptr, y.ptr, 1, None)
        assert st == hip.DC_ERR_DIMENSION
        ctx.free(x)
        ctx.free(y)
    ctx.synchronize()
    for a in (rp, col, val):
        ctx.free(a)
