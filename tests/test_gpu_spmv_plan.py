"""GPU parity: the tiled SpMV plan (dc_hip_spmv_plan_*), which the power iteration uses.

Reference semantics: SparseOps.SpMV (SparseMatrix.cs:669-692), a sequential float32 row sum. The
plan forms every product val * x[col] once (x tiles of up to 32768 columns in LDS) and stages each
row block's products at their CSR positions, so a row of at most 32 nonzeros is summed by one lane
in index order (0.0f + p_0 + p_1 + ...), whatever the number of column slices; longer rows are
summed by a wave (lane k adds products k, k + 64, ... in order, then a fixed tree). Two checks per
case:
  - parity: |y - y64| <= 1e-4 * sum_i |v_i x_c(i)| per row, y64 the float64 row sum;
  - exactness of the order: rows of at most 32 nonzeros equal the oracle's sequential float32
    SpMV bit for bit (a product formed twice, dropped, misplaced or summed out of order fails it).
"""
import numpy as np
import pytest

import oracle
from dotcompute_amd import hip

pytestmark = pytest.mark.gpu

REL = 1e-4
SEQ_ROW = 32          # rows up to this length are summed sequentially on the GPU
TILE_COLS = 32768     # widest slice (one x tile in LDS)
GIANT_ROW = 4096      # longer rows are summed with their products formed from x directly


def upload_csr(ctx, rp, col, val):
    return ctx.to_device(rp), ctx.to_device(col if col.size else np.zeros(1, np.int32)), \
        ctx.to_device(val if val.size else np.zeros(1, np.float32))


def row_scale(rp, col, val, x):
    return oracle.spmv_csr_f64(rp, col, np.abs(val), np.abs(x).astype(np.float64))


def expected_slices(cols, width, nnz=0, rows=None):
    """(slices, columns per slice) the plan picks: slice_cols_max capped at 32768, or by default
    the widest power of two in [4096, 32768] with w <= nnz / (2 * CUs), widened while more than
    span / 8 slices would be needed (span: the plan's block span, 4096 nonzeros when that gives
    fewer than 4 blocks per CU, else 8192); then widened when more than 32768 slices would be
    needed."""
    if width > 0:
        w = min(width, TILE_COLS)
    else:
        cus = max(1, hip.device_info(0).compute_units)
        rows = cols if rows is None else rows
        span = 4096 if nnz // 8192 + max(rows - 1, 0) // 16384 + 1 < 4 * cus else 8192
        w = 4096
        while w < TILE_COLS and (2 * w <= nnz // (2 * cus) or -(-cols // w) > span // 8):
            w *= 2
    if -(-cols // w) > 32768:
        w = -(-cols // 32768)
    return max(1, -(-cols // w)), w


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


def check(rp, col, val, x, y):
    ref64 = oracle.spmv_csr_f64(rp, col, val, x.astype(np.float64))
    assert np.all(np.abs(y - ref64) <= REL * row_scale(rp, col, val, x) + 1e-30)
    ref32 = oracle.spmv_csr_f32(rp, col, val, x)
    ok = np.diff(rp) <= SEQ_ROW
    assert np.array_equal(y[ok].view(np.uint32), ref32[ok].view(np.uint32))


# (rows, cols, slice_cols_max) -> expected number of slices: ceil(cols / w), w = slice_cols_max
# capped at 32768 columns, widened when more than 32768 slices would be needed (None: the
# default width, which depends on the number of nonzeros and of CUs; see expected_slices).
SHAPES = [
    (5000, 5000, 0, None),
    (200_000, 200_000, 0, None),
    (600_000, 600_000, 0, None),
    (100_000, 100_000, 1 << 20, 4),   # wider than one x tile: capped at 32768 columns
    (5000, 5000, 2500, 2),
    (5000, 5000, 1250, 4),
    (5000, 5000, 625, 8),
    (5000, 5000, 300, 17),
    (20000, 20000, 100, 200),
    (20000, 20000, 7, 2858),          # more slices than the row pass's LDS chunk table holds
    (70000, 70000, 1, 23334),         # more than 32768 slices asked for: widened to 3 columns
    (3000, 70000, 4000, 18),          # rectangular, more columns than rows
    (1, 1, 0, None),
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
    assert (s, w) == expected_slices(cols, width, col.size, rows) and s == (slices or s) and nbytes > 0
    check(rp, col, val, x, y)


def test_plan_signed_values_long_and_giant_rows(ctx):
    """Negative values; rows of 0 / 1 / 31-33 / 4096 / 3000 nonzeros; rows at the giant threshold
    (4096 nonzeros: staged; 4097 and 40000: summed from x directly), each followed by more rows;
    empty rows exactly zero."""
    lens = [0, 1, 4096, 0, 3000, 7, 129, 128, 0, 600, 257, 256, 513, 512, 32, 33, 31, 64, 65,
            GIANT_ROW, 5, GIANT_ROW + 1, 0, 3, 40000, 2, 1, 0, 17]
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cols = 5000
    col = (np.arange(rp[-1]) * 7919 % cols).astype(np.int32)
    val = oracle.gen_uniform_f32(int(rp[-1]), 9, 0)
    x = oracle.gen_uniform_f32(cols, 9, 1)
    for width in (0, 2500, 625, 3):
        y, (s, w, _) = run_plan(ctx, rp, col, val, x, width)
        assert (s, w) == expected_slices(cols, width, col.size, rp.size - 1)
        check(rp, col, val, x, y)
        assert y[0] == 0 and y[3] == 0 and y[8] == 0 and y[22] == 0 and y[27] == 0


def test_plan_many_row_blocks_of_empty_rows(ctx):
    """Blocks are also cut every 16384 rows: 100,000 rows, mostly empty, a few short rows spread
    among them."""
    rows, cols = 100_000, 1000
    lens = np.zeros(rows, np.int64)
    lens[::997] = 3
    lens[50_000:50_010] = 40
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    col = (np.arange(rp[-1]) * 613 % cols).astype(np.int32)
    val = oracle.gen_uniform_f32(int(rp[-1]), 3, 0)
    x = oracle.gen_uniform_f32(cols, 3, 1)
    y, _ = run_plan(ctx, rp, col, val, x, 0)
    check(rp, col, val, x, y)
    assert np.all(y[lens == 0] == 0)


def test_plan_equals_sequential_reference(ctx):
    """Rows of at most 32 nonzeros (about 99% of the rows of this graph) are the sequential
    float32 row sum of SparseOps.SpMV bit for bit, with the default slices (tens of them)."""
    rows = 300_000
    rp, col, val = oracle.gen_zipf_csr(rows, 7)
    x = oracle.gen_uniform_f32(rows, 7, 5, unit_interval=True)
    y, (s, w, _) = run_plan(ctx, rp, col, val, x, 0, repeat=1)
    assert (s, w) == expected_slices(rows, 0, col.size) and s > 1
    ref = oracle.spmv_csr_f32(rp, col, val, x)
    short = np.diff(rp) <= SEQ_ROW
    assert short.sum() > 0.98 * rows
    assert np.array_equal(y[short].view(np.uint32), ref[short].view(np.uint32))


def random_structure(kind, rows, cols, seed):
    """CSR matrices of other shapes than the Zipf graph: uniform degrees, rows whose columns cluster
    (several products of a row in one run), hub columns, and rows that are all hubs."""
    rng = np.random.default_rng(seed)
    if kind == "uniform":
        deg = rng.integers(0, 65, rows)
    else:
        deg = rng.integers(0, 41, rows)
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    nnz = int(rp[-1])
    if kind == "uniform":
        col = rng.integers(0, cols, nnz)
    elif kind == "clustered":
        centre = np.repeat(rng.integers(0, cols, rows), deg)
        col = np.clip(centre + rng.integers(-500, 501, nnz), 0, cols - 1)
    else:  # hubs: 30% of the nonzeros point at 10 columns
        col = rng.integers(0, cols, nnz)
        hub = rng.random(nnz) < 0.3
        col[hub] = rng.integers(0, 10, int(hub.sum())) * (cols // 10)
    val = (rng.standard_normal(nnz)).astype(np.float32)
    return rp, col.astype(np.int32), val


@pytest.mark.parametrize("kind,rows,cols", [("uniform", 100_000, 300_000), ("clustered", 200_000, 200_000),
                                            ("hubs", 150_000, 1_000_000)])
def test_plan_random_structures(ctx, kind, rows, cols):
    rp, col, val = random_structure(kind, rows, cols, rows + cols)
    x = oracle.gen_uniform_f32(cols, 11, 2)
    for width in (0, 2048):
        y, (s, w, _) = run_plan(ctx, rp, col, val, x, width)
        assert (s, w) == expected_slices(cols, width, col.size, rows)
        check(rp, col, val, x, y)


def test_plan_large_blocks_equal_sequential_reference(ctx):
    """A matrix with enough nonzeros for 8192-nonzero blocks and 1024-thread row-pass workgroups
    (2M rows of the Zipf graph, 10.8M nonzeros): rows of at most 32 nonzeros are the sequential
    float32 row sum bit for bit, the rest within the tolerance."""
    rows = 2_000_000
    rp, col, val = oracle.gen_zipf_csr(rows, 5)
    cus = max(1, hip.device_info(0).compute_units)
    assert col.size // 8192 + (rows - 1) // 16384 + 1 >= 4 * cus, "the case must take the 8192 span"
    x = oracle.gen_uniform_f32(rows, 5, 5, unit_interval=True)
    y, (s, w, _) = run_plan(ctx, rp, col, val, x, 0)
    assert (s, w) == expected_slices(rows, 0, col.size, rows)
    check(rp, col, val, x, y)


@pytest.mark.parametrize("width,slices", [(0, None), (1 << 15, 31), (1 << 12, 245), (1000, 1000)])
def test_plan_1m_many_slices(ctx, width, slices):
    rows = 1_000_000
    rp, col, val = oracle.gen_zipf_csr(rows, 42)
    x = oracle.gen_uniform_f32(rows, 42, 5, unit_interval=True)
    y, (s, w, _) = run_plan(ctx, rp, col, val, x, width, repeat=2)
    assert (s, w) == expected_slices(rows, width, col.size) and s == (slices or s)
    check(rp, col, val, x, y)


@pytest.mark.parametrize("width", [0, 1 << 15])
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
    for rows in (1000, 40_000):
        rp = np.zeros(rows + 1, np.int32)
        x = np.ones(rows, np.float32)
        y, (s, w, _) = run_plan(ctx, rp, np.zeros(0, np.int32), np.zeros(0, np.float32), x, 0, repeat=1)
        assert (s, w) == expected_slices(rows, 0, 0) and np.all(y == 0)


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
