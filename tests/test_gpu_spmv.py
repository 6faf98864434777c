"""GPU parity: CSR SpMV and the 20-iteration normalised power iteration (SpMV benchmark).

Reference semantics: SparseOps.SpMV (SparseMatrix.cs:669-692), a sequential float32 row sum; the
HIP kernels sum each row in a different (fixed) order, so the bar is rel 1e-4 per element,
measured against sum_i |v_i * x_c(i)| of the row (the row's condition scale). Small graphs are
also checked against a dense float64 brute force. Graphs: Zipf(alpha=2.0) out-degrees on
[1, 4096], uniform columns without self-loops, values 1/out-degree.
"""
import numpy as np
import pytest

import oracle
from dotcompute_amd import hip

pytestmark = pytest.mark.gpu

REL = 1e-4


def upload_csr(ctx, rp, col, val):
    return ctx.to_device(rp), ctx.to_device(col if col.size else np.zeros(1, np.int32)), \
        ctx.to_device(val if val.size else np.zeros(1, np.float32))


def spmv_gpu(ctx, rp, col, val, x):
    rows = rp.size - 1
    drp, dcol, dval = upload_csr(ctx, rp, col, val)
    dx = ctx.to_device(x)
    dy = ctx.empty(max(rows, 1), np.float32)
    ctx.spmv_csr_f32(drp, dcol, dval, dx, dy, rows, x.size, col.size)
    ctx.synchronize()
    y = dy.to_host(rows)
    for a in (drp, dcol, dval, dx, dy):
        ctx.free(a)
    return y


def row_scale(rp, col, val, x):
    """sum_i |v_i x_c(i)| per row, float64."""
    return oracle.spmv_csr_f64(rp, col, np.abs(val), np.abs(x).astype(np.float64))


@pytest.mark.parametrize("rows,seed", [(1, 1), (2, 2), (64, 3), (257, 4), (5000, 5)])
def test_spmv_small_vs_dense_bruteforce(ctx, rows, seed):
    rp, col, val = oracle.gen_zipf_csr(max(rows, 2), seed, max_degree=min(4096, max(rows, 2) - 1))
    rp = rp[: rows + 1]
    col, val = col[: rp[-1]], val[: rp[-1]]
    x = oracle.gen_uniform_f32(max(rows, 2), seed, 5, unit_interval=True)
    y = spmv_gpu(ctx, rp, col, val, x)
    dense = np.zeros((rows, x.size))
    for r in range(rows):
        for i in range(rp[r], rp[r + 1]):
            dense[r, col[i]] += val[i]
    ref = dense @ x.astype(np.float64)
    scale = row_scale(rp, col, val, x)
    assert np.all(np.abs(y - ref) <= REL * scale + 1e-30)


def test_spmv_long_rows_and_empty_rows(ctx):
    """Rows of 0, 1, 4096 and 3000 nonzeros (long-row pass and the empty-row case)."""
    lens = [0, 1, 4096, 0, 3000, 7, 129, 128, 0]
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cols = 5000
    col = (np.arange(rp[-1]) * 7919 % cols).astype(np.int32)
    val = oracle.gen_uniform_f32(int(rp[-1]), 9, 0)
    x = oracle.gen_uniform_f32(cols, 9, 1)
    y = spmv_gpu(ctx, rp, col, val, x)
    ref = oracle.spmv_csr_f64(rp, col, val, x.astype(np.float64))
    assert np.all(np.abs(y - ref) <= REL * row_scale(rp, col, val, x) + 1e-30)
    assert y[0] == 0 and y[3] == 0 and y[8] == 0


@pytest.mark.parametrize("rows", [1_000_000])
def test_spmv_1m_vs_oracle(ctx, rows):
    rp, col, val = oracle.gen_zipf_csr(rows, 42)
    x = oracle.gen_uniform_f32(rows, 42, 5, unit_interval=True)
    y = spmv_gpu(ctx, rp, col, val, x)
    ref = oracle.spmv_csr_f32(rp, col, val, x)
    assert np.all(np.abs(y - ref) <= REL * row_scale(rp, col, val, x) + 1e-30)


def test_power_iteration_1m_vs_oracle(ctx):
    rows, iters = 1_000_000, 20
    rp, col, val = oracle.gen_zipf_csr(rows, 42)
    x0 = oracle.gen_uniform_f32(rows, 42, 5, unit_interval=True)
    drp, dcol, dval = upload_csr(ctx, rp, col, val)
    dx = ctx.to_device(x0)
    dy = ctx.empty(rows, np.float32)
    s = ctx.empty(1, np.float64)
    ctx.spmv_power_iterate_f32(drp, dcol, dval, dx, dy, rows, col.size, iters, s)
    ctx.synchronize()
    x = dx.to_host()
    ref_x, ref_s = oracle.spmv_power_f32(rp, col, val, x0, iters)
    assert abs(s.to_host()[0] - ref_s) <= REL * abs(ref_s)
    assert np.all(np.abs(x - ref_x) <= REL * np.abs(ref_x) + 1e-12)
    assert abs(float(np.sum(x, dtype=np.float64)) - 1.0) < 1e-4
    for a in (drp, dcol, dval, dx, dy, s):
        ctx.free(a)


@pytest.mark.slow
def test_power_iteration_16m_vs_oracle(ctx):
    """Config C5 at 16M rows: the 20-iteration power iteration (489 column slices; rows of more
    than 32 nonzeros are tree-summed, every other row is the sequential float32 sum) against the
    oracle's sequential float32 restatement
    (oracle.spmv_power_f32, about 7 s on the host): every element of x_20 and the last L1 norm within
    rel 1e-4. Also the iteration's invariants (x >= 0, sum x = 1) and one step re-derived in float64
    on sampled rows."""
    from dotcompute_amd import hip

    rows, iters = 16_000_000, 20
    rp, col, val = hip.gen_zipf_csr(rows, 42)
    x0 = oracle.gen_uniform_f32(rows, 42, 5, unit_interval=True)
    drp, dcol, dval = upload_csr(ctx, rp, col, val)
    dx = ctx.to_device(x0)
    dy = ctx.empty(rows, np.float32)
    s = ctx.empty(1, np.float64)
    ctx.spmv_power_iterate_f32(drp, dcol, dval, dx, dy, rows, col.size, iters - 1, s)
    ctx.synchronize()
    x19 = dx.to_host()
    ctx.spmv_power_iterate_f32(drp, dcol, dval, dx, dy, rows, col.size, 1, s)
    ctx.synchronize()
    x20 = dx.to_host()
    s20 = s.to_host()[0]
    for a in (drp, dcol, dval, dx, dy, s):
        ctx.free(a)
    assert np.all(x20 >= 0) and abs(float(np.sum(x20, dtype=np.float64)) - 1.0) < 1e-4
    sample = np.random.default_rng(0).integers(0, rows, 2000)
    for r in sample:
        b, e = rp[r], rp[r + 1]
        yr = float(np.dot(val[b:e].astype(np.float64), x19[col[b:e]].astype(np.float64)))
        assert abs(x20[r] - yr / s20) <= REL * abs(yr / s20) + 1e-12
    ref_x, ref_s = oracle.spmv_power_f32(rp, col, val, x0, iters)
    assert abs(s20 - ref_s) <= REL * abs(ref_s)
    bad = np.abs(x20 - ref_x) > REL * np.abs(ref_x) + 1e-12
    assert not bad.any(), (int(bad.sum()), np.flatnonzero(bad)[:10])


def test_spmv_short_rows_bit_exact_with_sequential_reference(ctx):
    """Rows of at most 512 nonzeros are summed by one thread in index order from products rounded
    once each, exactly as SparseOps.SpMV does: bit-identical to the sequential float32 oracle."""
    rows = 300_000
    rp, col, val = oracle.gen_zipf_csr(rows, 7)
    x = oracle.gen_uniform_f32(rows, 7, 5, unit_interval=True)
    y = spmv_gpu(ctx, rp, col, val, x)
    ref = oracle.spmv_csr_f32(rp, col, val, x)
    short = np.diff(rp) <= 512
    assert short.sum() > 0.99 * rows
    assert np.array_equal(y[short].view(np.uint32), ref[short].view(np.uint32))


# ---- SparseOps.SpMV<T> for T = double and int (the reference is generic over INumber<T>) ----------
def spmv_gpu_typed(ctx, rp, col, val, x):
    rows = rp.size - 1
    drp, dcol = ctx.to_device(rp), ctx.to_device(col if col.size else np.zeros(1, np.int32))
    dval = ctx.to_device(val if val.size else np.zeros(1, val.dtype))
    dx = ctx.to_device(x)
    dy = ctx.empty(max(rows, 1), val.dtype)
    ctx.spmv_csr(drp, dcol, dval, dx, dy, rows, x.size, col.size)
    ctx.synchronize()
    y = dy.to_host(rows)
    for a in (drp, dcol, dval, dx, dy):
        ctx.free(a)
    return y


@pytest.mark.parametrize("rows", [5000, 1_000_000])
def test_spmv_double_rows_match_sequential_reference(ctx, rows):
    """SpMV<double>: rows of at most 512 nonzeros bit-identical to the reference loop (0.0 plus each
    product in index order), the long rows (a fixed-order tree) within 1e-12 of it."""
    rp, col, _ = oracle.gen_zipf_csr(rows, 61)
    val = oracle.gen_uniform_f32(int(rp[-1]), 62, 0).astype(np.float64) * np.pi
    x = oracle.gen_uniform_f32(rows, 63, 1).astype(np.float64) / 3.0
    y = spmv_gpu_typed(ctx, rp, col, val, x)
    ref = oracle.spmv_csr_f64d(rp, col, val, x)
    deg = np.diff(rp)
    short = deg <= 512
    assert np.array_equal(y[short].view(np.uint64), ref[short].view(np.uint64))
    scale = oracle.spmv_csr_f64d(rp, col, np.abs(val), np.abs(x))
    assert np.all(np.abs(y - ref) <= 1e-12 * scale + 1e-300)
    assert (~short).any() or rows < 1_000_000  # the 1M graph has rows past the long-row threshold


@pytest.mark.parametrize("rows", [5000, 1_000_000])
def test_spmv_int_wraps_like_csharp(ctx, rows):
    """SpMV<int>: every row bit-identical to the reference loop, long rows included (wrapping adds
    give the same bits in any order); values chosen so products and sums overflow int32."""
    rp, col, _ = oracle.gen_zipf_csr(rows, 64)
    val = oracle.gen_uniform_i32(int(rp[-1]), 65, 1, -2_000_000_000, 2_000_000_000)
    x = oracle.gen_uniform_i32(rows, 66, 2, -70_000, 70_000)
    y = spmv_gpu_typed(ctx, rp, col, val, x)
    ref = oracle.spmv_csr_i32(rp, col, val, x)
    assert np.array_equal(y, ref)


def test_spmv_typed_dimension_check(ctx):
    rp = np.array([0, 1], np.int32)
    col = np.array([0], np.int32)
    for dt in (np.float64, np.int32):
        drp, dcol, dval = ctx.to_device(rp), ctx.to_device(col), ctx.to_device(np.ones(1, dt))
        dx, dy = ctx.to_device(np.ones(1, dt)), ctx.empty(1, dt)
        with pytest.raises(hip.HipError) as e:
            ctx.spmv_csr(drp, dcol, dval, dx, dy, -1, 1, 1)
        assert e.value.status == hip.DC_ERR_INVALID_ARGUMENT
        for a in (drp, dcol, dval, dx, dy):
            ctx.free(a)
