"""GPU parity: dense row-major GEMM on the matrix cores (fp32 and bf16-in / fp32-accumulate).

Tolerance (written once, used everywhere): normwise ||C - C64||_F / ||C64||_F <= 1e-4 and, per
entry, |C - C64| <= 1e-4 * (|A|·|B|)_ij, against a float64 GEMM of the same inputs (for bf16, of
the bf16-rounded inputs). Element-relative error is ill-posed where C_ij ~ 0, hence the |A||B|
scaling. Large sizes are checked on sampled full rows plus a Freivalds product over all of C.
The reference's own case is CudaRealWorldAlgorithmTests.cs:56-96 (m=512, n=768, k=384, seeds 42/43,
abs 1e-3 vs a CPU fp32 triple loop), reproduced below against the oracle's fp32 loop.
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

REL = 1e-4


def make_inputs(m, n, k, seed_a=42, seed_b=43):
    a = oracle.gen_uniform_f32(m * k, seed_a, 0).reshape(m, k)
    b = oracle.gen_uniform_f32(k * n, seed_b, 0).reshape(k, n)
    return a, b


def run_gemm(ctx, a, b, kind="f32"):
    m, k = a.shape
    _, n = b.shape
    c = ctx.empty((m, n), np.float32)
    if kind == "f32":
        da, db = ctx.to_device(a), ctx.to_device(b)
        ctx.gemm_f32(da, db, c, m, n, k)
    else:
        da, db = ctx.to_device(oracle.f32_to_bf16(a)), ctx.to_device(oracle.f32_to_bf16(b))
        ctx.gemm_bf16(da, db, c, m, n, k)
    ctx.synchronize()
    out = c.to_host()
    for x in (da, db, c):
        ctx.free(x)
    return out


def check_rows(c, a, b, rows):
    ref, absref = oracle.gemm_f64_rows(np.ascontiguousarray(a), np.ascontiguousarray(b), rows)
    got = c[rows].astype(np.float64)
    err = np.abs(got - ref)
    assert np.all(err <= REL * absref + 1e-30), f"max per-entry ratio {np.max(err / np.maximum(absref, 1e-30)):.3e}"
    normwise = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert normwise <= REL, normwise
    return normwise


def freivalds(c, a, b, seed=0):
    """C·r vs A·(B·r) in float64 with r in {-1,+1}^n; bound 1e-4 * (|A|·(|B|·1))."""
    rng = np.random.default_rng(seed)
    n = b.shape[1]
    r = rng.choice([-1.0, 1.0], size=n)
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    lhs = c.astype(np.float64) @ r
    rhs = a64 @ (b64 @ r)
    bound = np.abs(a64) @ (np.abs(b64) @ np.ones(n))
    assert np.all(np.abs(lhs - rhs) <= REL * bound)


@pytest.mark.parametrize("shape", [(128, 128, 128), (256, 384, 640), (512, 768, 384), (1024, 1024, 1024)])
def test_gemm_f32_full_tiles(ctx, shape):
    m, n, k = shape
    a, b = make_inputs(m, n, k)
    c = run_gemm(ctx, a, b)
    check_rows(c, a, b, np.arange(m))


# Full-tile shapes run the direct-to-LDS kernel (64-tiles below 2 * CUs 128-tiles, else 128-tiles);
# these cover one, two and an odd number of 32-wide k tiles for both tile sizes.
@pytest.mark.parametrize("shape", [(128, 128, 32), (192, 320, 96), (256, 64, 64), (4096, 2048, 32),
                                   (2048, 4096, 64), (4096, 2048, 96)])
def test_gemm_f32_k_tile_counts(ctx, shape):
    m, n, k = shape
    a, b = make_inputs(m, n, k)
    c = run_gemm(ctx, a, b)
    check_rows(c, a, b, np.arange(m))


def test_gemm_f32_reference_case_vs_fp32_loop(ctx):
    """CudaRealWorldAlgorithmTests.cs:56-96: m=512, n=768, k=384, abs tol 1e-3 vs the fp32 triple loop."""
    m, n, k = 512, 768, 384
    a, b = make_inputs(m, n, k)
    c = run_gemm(ctx, a, b)
    expected = oracle.gemm_f32_naive(a, b, threads=8)
    assert np.max(np.abs(c - expected)) <= 1e-3


# Shapes with fewer than 2 * CUs tiles of 128x128 run 64x64 tiles; (4000, 2100, 37) has 544 of them
# and takes the bounds-checked 128x128 kernel.
@pytest.mark.parametrize("shape", [(1, 1, 1), (3, 5, 7), (100, 37, 53), (129, 130, 131), (257, 64, 1000),
                                   (4000, 2100, 37)])
def test_gemm_f32_ragged(ctx, shape):
    m, n, k = shape
    a, b = make_inputs(m, n, k, 7, 8)
    c = run_gemm(ctx, a, b)
    check_rows(c, a, b, np.arange(m))


def test_gemm_f32_k_zero_gives_zeros(ctx):
    c = ctx.empty((4, 5), np.float32)
    a = ctx.empty(1, np.float32)
    ctx.gemm_f32(a, a, c, 4, 5, 0)
    ctx.synchronize()
    assert np.all(c.to_host() == 0)
    ctx.free(c)
    ctx.free(a)


def test_gemm_identity_and_permutation_exact(ctx):
    n = 256
    a, _ = make_inputs(n, n, n)
    eye = np.eye(n, dtype=np.float32)
    assert np.array_equal(run_gemm(ctx, a, eye), a)  # one nonzero term per entry: exact
    perm = np.eye(n, dtype=np.float32)[np.random.default_rng(1).permutation(n)]
    assert np.array_equal(run_gemm(ctx, perm, a), perm @ a)


@pytest.mark.slow
@pytest.mark.parametrize("n", [4096, 8192])
def test_gemm_f32_large_sampled(ctx, n):
    a, b = make_inputs(n, n, n)
    c = run_gemm(ctx, a, b)
    rows = np.unique(np.concatenate([[0, n - 1], np.random.default_rng(n).integers(0, n, 30)]))
    check_rows(c, a, b, rows)
    freivalds(c, a, b)


# (256-multiples of m and n with k a multiple of 64 take the 256x256-tile kernel, which reads
# row-major B through transposing LDS reads, with 1, 2, 3, 6 and more 64-wide k tiles; the other
# shapes the 128x128 kernels)
@pytest.mark.parametrize("shape", [(128, 128, 64), (512, 768, 384), (100, 37, 53), (256, 256, 64),
                                   (1024, 512, 1024), (768, 1280, 192), (256, 512, 4096), (384, 256, 64),
                                   (512, 256, 128)])
def test_gemm_bf16(ctx, shape):
    m, n, k = shape
    a, b = make_inputs(m, n, k)
    c = run_gemm(ctx, a, b, kind="bf16")
    ar = oracle.bf16_to_f32(oracle.f32_to_bf16(a)).reshape(m, k)
    br = oracle.bf16_to_f32(oracle.f32_to_bf16(b)).reshape(k, n)
    check_rows(c, ar, br, np.arange(m))


@pytest.mark.slow
def test_gemm_bf16_8192_sampled(ctx):
    n = 8192
    a, b = make_inputs(n, n, n)
    c = run_gemm(ctx, a, b, kind="bf16")
    ar = oracle.bf16_to_f32(oracle.f32_to_bf16(a)).reshape(n, n)
    br = oracle.bf16_to_f32(oracle.f32_to_bf16(b)).reshape(n, n)
    rows = np.unique(np.concatenate([[0, n - 1], np.random.default_rng(5).integers(0, n, 16)]))
    check_rows(c, ar, br, rows)
    freivalds(c, ar, br)  # every entry, through C·r against A·(B·r) on the bf16-rounded inputs


def test_convert_f32_to_bf16_bit_exact(ctx):
    x = np.concatenate([oracle.gen_uniform_f32(100_000, 3, 0) * 1000,
                        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, 3.3895314e38, 1.0039062], np.float32)])
    d = ctx.to_device(x)
    o = ctx.empty(x.size, np.uint16)
    ctx.convert_f32_to_bf16(d, o)
    ctx.synchronize()
    got = o.to_host()
    ref = oracle.f32_to_bf16(x)
    assert np.array_equal(got, ref)
    ctx.free(d)
    ctx.free(o)
