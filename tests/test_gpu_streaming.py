"""GPU parity: VectorAdd, the seeded generators and the sum reductions vs the CPU oracle.

Mirrors the reference's checks (MultiBackendIntegrationTests.cs:130-176 VectorAdd;
CudaRealWorldAlgorithmTests.cs:100-131 reduction vs a double sum) at the configuration sizes,
with the tolerances the HIP path promises: VectorAdd and int32 sums bit-exact, fp32 sums within
rel 1e-5*log2(N) of a float64 host sum.
"""
import math

import numpy as np
import pytest

import oracle
from dotcompute_amd import hip

pytestmark = pytest.mark.gpu


def fp32_sum_tol(n: int) -> float:
    return 1e-5 * max(1.0, math.log2(max(n, 2)))


# ---------------------------------------------------------------- generators
@pytest.mark.parametrize("n", [1, 1000, 100_003])
def test_device_generators_match_oracle(ctx, n):
    d = ctx.empty(n, np.float32)
    ctx.fill_uniform_f32(d, seed=42, stream=0)
    assert np.array_equal(d.to_host().view(np.uint32), oracle.gen_uniform_f32(n, 42, 0).view(np.uint32))
    ctx.fill_uniform_f32(d, seed=7, stream=2, unit_interval=True)
    assert np.array_equal(d.to_host().view(np.uint32), oracle.gen_uniform_f32(n, 7, 2, True).view(np.uint32))
    di = ctx.empty(n, np.int32)
    ctx.fill_uniform_i32(di, seed=43, stream=1, lo=-1000, hi=1000)
    assert np.array_equal(di.to_host(), oracle.gen_uniform_i32(n, 43, 1, -1000, 1000))
    ctx.free(d)
    ctx.free(di)


# ---------------------------------------------------------------- VectorAdd
@pytest.mark.parametrize("n", [0, 1, 3, 5, 1000, 100_000, 1_000_003])
def test_vector_add_bit_exact(ctx, n):
    a = oracle.gen_uniform_f32(n, 42, 0)
    b = oracle.gen_uniform_f32(n, 42, 1)
    da, db, dr = ctx.to_device(a), ctx.to_device(b), ctx.empty(max(n, 1), np.float32)
    ctx.vector_add_f32(da, db, dr, n)
    ctx.synchronize()
    got = dr.to_host(n)
    assert np.array_equal(got.view(np.uint32), oracle.vector_add_f32(a, b).view(np.uint32))
    for x in (da, db, dr):
        ctx.free(x)


def test_vector_add_misaligned_pointers(ctx):
    n = 4099
    a = oracle.gen_uniform_f32(n + 1, 1, 0)
    b = oracle.gen_uniform_f32(n + 1, 1, 1)
    da, db, dr = ctx.to_device(a), ctx.to_device(b), ctx.empty(n + 1, np.float32)
    # offset every pointer by one float: the kernel must take its unaligned path
    sub = lambda d: hip.DeviceArray(ctx, d.ptr + 4, d.nbytes - 4, d.dtype, (n,))
    ctx.vector_add_f32(sub(da), sub(db), sub(dr), n)
    ctx.synchronize()
    got = dr.to_host()[1:]
    assert np.array_equal(got, oracle.vector_add_f32(a[1:].copy(), b[1:].copy()))
    for x in (da, db, dr):
        ctx.free(x)


def test_vector_add_through_code_object(ctx):
    """The generic ICompiledKernel path: load dc_kernels_gfx950.hsaco and launch the `VectorAdd`
    the generator translated from the README [Kernel] — buffers (a, b, result), then the
    dc_gen_launch block (work, epoch, error words, buffer lengths) — block 256, grid ceil(N/256).
    A short `b` makes the kernel report IndexOutOfRange through the error words."""
    import ctypes as C

    L = hip.load()
    path = L.dc_hip_default_module_path()
    assert path, "dc_kernels_gfx950.hsaco not found next to the library"
    mod = C.c_void_p()
    hip.check(L.dc_hip_module_load(ctx.handle, path, C.byref(mod)), "module_load")
    fn = C.c_void_p()
    hip.check(L.dc_hip_module_get_function(mod, b"VectorAdd", C.byref(fn)), "get_function")
    assert L.dc_hip_module_get_function(mod, b"NoSuchKernel", C.byref(C.c_void_p())) == hip.DC_ERR_NOT_FOUND
    err_host = C.c_void_p()
    hip.check(L.dc_hip_malloc_host(ctx.handle, 16, C.byref(err_host)), "malloc_host")
    C.memset(err_host, 0, 16)
    err_dev = C.c_void_p()
    hip.check(L.dc_hip_host_device_pointer(ctx.handle, err_host, C.byref(err_dev)), "host_device_pointer")
    words = (C.c_uint32 * 4).from_address(err_host.value)
    n = 100_000
    a = oracle.gen_uniform_f32(n, 42, 0)
    b = oracle.gen_uniform_f32(n, 42, 1)
    da, db, dr = ctx.to_device(a), ctx.to_device(b), ctx.empty(n, np.float32)
    for epoch, len_b in ((7, n), (8, n - 10)):
        pa, pb, pr = C.c_void_p(da.ptr), C.c_void_p(db.ptr), C.c_void_p(dr.ptr)
        block = hip.GenLaunch(work=n, epoch=epoch, error=err_dev.value)
        block.len[0], block.len[1], block.len[2] = n, len_b, n
        args = (C.c_void_p * 4)(C.addressof(pa), C.addressof(pb), C.addressof(pr), C.addressof(block))
        hip.check(L.dc_hip_launch_kernel(ctx.handle, fn, (n + 255) // 256, 1, 1, 256, 1, 1, 0,
                                         C.cast(args, C.POINTER(C.c_void_p))), "launch")
        ctx.synchronize()
        if len_b == n:
            assert np.array_equal(dr.to_host(), oracle.vector_add_f32(a, b))
            assert words[hip.DC_GEN_ERR_INDEX] != epoch
        else:
            assert words[hip.DC_GEN_ERR_INDEX] == epoch  # b[n-10] and after are out of range
    hip.check(L.dc_hip_module_unload(mod), "unload")
    hip.check(L.dc_hip_free_host(ctx.handle, err_host), "free_host")
    for x in (da, db, dr):
        ctx.free(x)


# ---------------------------------------------------------------- Sum f32
@pytest.mark.parametrize("n", [0, 1, 7, 1000, 65_537, 1_000_000, 16_000_000])
def test_sum_f32_within_tolerance_and_deterministic(ctx, n):
    x = oracle.gen_uniform_f32(n, 42, 0)
    dx = ctx.to_device(x) if n else ctx.empty(1, np.float32)
    out = ctx.empty(1, np.float64)
    ctx.reduce_sum_f32(dx, out, n)
    ctx.synchronize()
    got = out.to_host()[0]
    ref = oracle.sum_f32_compensated(x)
    f32_ref, seq_double = oracle.sum_f32_enumerable(x)
    tol = fp32_sum_tol(n)
    assert abs(got - ref) <= tol * max(abs(ref), 1e-30) + 1e-12
    # the float result the managed caller returns equals Enumerable.Sum's (double accumulator)
    assert abs(np.float32(got) - f32_ref) <= tol * max(abs(ref), 1e-30) + 1e-6
    ctx.reduce_sum_f32(dx, out, n)
    ctx.synchronize()
    assert out.to_host()[0] == got, "reduction is not run-to-run deterministic"
    ctx.free(dx)
    ctx.free(out)


def test_sum_f32_known_answers(ctx):
    # ComputeQueryProviderTests.cs:602-612 (Sum 1..5 = 15), LinqBackendIntegrationTests.cs:164-176
    # (Sum 1..1000 = 500500): exact in float.
    for vals, expect in ((np.arange(1, 6, dtype=np.float32), 15.0), (np.arange(1, 1001, dtype=np.float32), 500500.0)):
        d = ctx.to_device(vals)
        out = ctx.empty(1, np.float64)
        ctx.reduce_sum_f32(d, out)
        ctx.synchronize()
        assert out.to_host()[0] == expect
        ctx.free(d)
        ctx.free(out)


def test_sum_f32_unit_interval_1m_rel_1e3(ctx):
    # CudaRealWorldAlgorithmTests.cs:100-131: 1M values in [0,1), rel 1e-3 vs a double sum.
    n = 1_000_000
    x = oracle.gen_uniform_f32(n, 42, 0, unit_interval=True)
    d = ctx.to_device(x)
    out = ctx.empty(1, np.float64)
    ctx.reduce_sum_f32(d, out)
    ctx.synchronize()
    ref = float(np.sum(x, dtype=np.float64))
    assert abs(out.to_host()[0] - ref) / ref < 1e-3
    assert abs(out.to_host()[0] - ref) / ref < fp32_sum_tol(n)
    ctx.free(d)
    ctx.free(out)


# ---------------------------------------------------------------- Sum i32
@pytest.mark.parametrize("n", [0, 1, 5, 1000, 1_000_000, 16_000_000])
def test_sum_i32_bit_exact(ctx, n):
    x = oracle.gen_uniform_i32(n, 43, 1, -1000, 1000)
    dx = ctx.to_device(x) if n else ctx.empty(1, np.int32)
    out = ctx.empty(1, np.int64)
    ovf = ctx.empty(1, np.int32)
    ctx.reduce_sum_i32(dx, out, ovf, n)
    ctx.synchronize()
    assert out.to_host()[0] == oracle.sum_i32_exact(x)
    assert out.to_host()[0] == oracle.sum_i32_bcl(x)
    assert ovf.to_host()[0] == 0
    for a in (dx, out, ovf):
        ctx.free(a)


def gpu_sum_i32(ctx, x, offset=0):
    """Runs dc_hip_reduce_sum_i32 on x placed `offset` ints into its allocation; returns (exact
    int64 total, overflow flag)."""
    n = x.size
    d = ctx.empty(n + offset + 1, np.int32)
    if n:
        hip.check(hip.load().dc_hip_memcpy_h2d_async(ctx.handle, d.ptr + 4 * offset, x.ctypes.data, x.nbytes), "h2d")
    src = hip.DeviceArray(ctx, d.ptr + 4 * offset, 4 * max(n, 1), np.dtype(np.int32), (n,))
    out = ctx.empty(1, np.int64)
    ovf = ctx.empty(1, np.int32)
    ctx.reduce_sum_i32(src, out, ovf, n)
    ctx.synchronize()
    r = int(out.to_host()[0]), int(ovf.to_host()[0])
    for a in (d, out, ovf):
        ctx.free(a)
    return r


def bcl_overflows(x):
    try:
        oracle.sum_i32_bcl(x)
        return 0
    except OverflowError:
        return 1


def test_sum_i32_overflow_follows_the_bcl_rule(ctx):
    """Checked Sum throws where the .NET BCL's 8-lane vector path (or, below 32 elements, its
    sequential loop) would: the overflow flag matches the oracle's restatement of that algorithm
    on inputs where a prefix overflows but the total fits, and the reverse cases."""
    big = 2**31 - 1

    def vec(n, **at):
        x = np.zeros(n, np.int32)
        for k, v in at.items():
            x[int(k[1:])] = v
        return x

    cases = [
        np.full(4, 2**30, np.int32),            # total 2^32: throws
        np.array([big, 0, 0], np.int32),        # largest total, fits
        np.array([big, 1, -1], np.int32),       # short input: a running total overflows
        vec(32, i0=big, i1=1, i8=-1),           # sequential prefix overflows, lanes do not: no throw
        vec(32, i0=big, i1=-5, i8=1),           # lane 0 overflows, sequential prefixes fit: throws
        vec(32, i8=big, i1=1, i2=-10),          # lane totals overflow in lane order: throws
        vec(40, i0=big, i1=-1, i32=1),          # x32 in the scalar tail: fits
        vec(41, i0=big, i1=-1, i32=1),          # x32 in lane 0: throws
        vec(40, i32=big, i33=1, i34=-1),        # tail prefix overflows: throws
    ]
    for x in cases:
        for offset in (0, 1, 2, 3):
            total, ovf = gpu_sum_i32(ctx, x, offset)
            assert total == int(x.astype(np.int64).sum())
            assert ovf == bcl_overflows(x), (x[:12], x.size, offset)


@pytest.mark.parametrize("n", [1_000_000, 16_000_000])
def test_sum_i32_bcl_rule_on_large_inputs(ctx, n):
    """Planted values near the int32 limit in a 1M / 16M input: the chunks holding them fail the
    fast screen and take the exact per-lane prefix check. One lane's running total comes within
    10^7 of 2^31 and back (no throw); then the same with 2^31 - 1 (its running total crosses unless
    the lane's earlier prefix is negative, so the oracle decides); then lane totals whose
    lane-order sum overflows."""
    base = oracle.gen_uniform_i32(n, 44, 1, -1000, 1000)
    i0 = (n // 3) & ~7
    near = 2**31 - 1 - 10**7
    x1 = base.copy()
    x1[i0 + 8], x1[i0 + 8 * 1000] = near, -near        # lane 0, 1000 elements of its lane apart
    x2 = base.copy()
    x2[i0 + 3], x2[i0 + 3 + 8 * 5000] = 2**31 - 1, -(2**31 - 1)
    x3 = base.copy()
    x3[5 * 8 + 1] = near                                # lane 1 total ~ near, lane 2 total ~ near
    x3[7 * 8 + 2] = near
    for x in (x1, x2, x3):
        for offset in (0, 1):
            total, ovf = gpu_sum_i32(ctx, x, offset)
            assert total == int(x.astype(np.int64).sum())
            assert ovf == bcl_overflows(x), (n, offset)
    assert bcl_overflows(x1) == 0 and bcl_overflows(x3) == 1


@pytest.mark.parametrize("n", [1 << 20, 1 << 22])
def test_sum_i32_screen_limits(ctx, n):
    """Constant inputs at the edge of the whole-input screen (n * largest and n * smallest within
    int32: no prefix can overflow): just inside it the total is returned with no overflow; one step
    outside the exact lane check decides, and the BCL rule then throws on the lane totals' sum.
    n = 2^20 runs the one-launch form (which screens), 2^22 the two-launch form (exact lane check
    only)."""
    lim = (2**31 - 1) // n
    for v in (lim, lim + 1, -(lim + 1), -(lim + 2)):
        x = np.full(n, v, np.int32)
        total, ovf = gpu_sum_i32(ctx, x)
        assert total == v * n
        assert ovf == bcl_overflows(x), (n, v)
        assert ovf == (0 if -2**31 <= v * n <= 2**31 - 1 else 1)


def test_sum_misaligned_inputs(ctx):
    """Inputs that start 1-3 elements past a 16-byte boundary run the vector path on the aligned
    part (no single-workgroup fallback): same results as the aligned input."""
    n = 3_000_001
    xi = oracle.gen_uniform_i32(n, 45, 1, -1000, 1000)
    xf = oracle.gen_uniform_f32(n, 45, 0)
    ref_f = oracle.sum_f32_compensated(xf)
    for offset in (1, 2, 3):
        assert gpu_sum_i32(ctx, xi, offset) == (int(xi.astype(np.int64).sum()), 0)
        d = ctx.empty(n + offset + 1, np.float32)
        hip.check(hip.load().dc_hip_memcpy_h2d_async(ctx.handle, d.ptr + 4 * offset, xf.ctypes.data, xf.nbytes), "h2d")
        src = hip.DeviceArray(ctx, d.ptr + 4 * offset, 4 * n, np.dtype(np.float32), (n,))
        out = ctx.empty(1, np.float64)
        ctx.reduce_sum_f32(src, out, n)
        ctx.synchronize()
        assert abs(out.to_host()[0] - ref_f) <= fp32_sum_tol(n) * abs(ref_f)
        ctx.free(d)
        ctx.free(out)


@pytest.mark.slow
def test_sum_256m_f32_and_i32(ctx):
    n = 256 * 1024 * 1024
    dx = ctx.empty(n, np.float32)
    ctx.fill_uniform_f32(dx, seed=42, stream=0)
    out = ctx.empty(1, np.float64)
    ctx.reduce_sum_f32(dx, out)
    ctx.synchronize()
    x = oracle.gen_uniform_f32(n, 42, 0)
    ref = oracle.sum_f32_compensated(x)
    assert abs(out.to_host()[0] - ref) <= fp32_sum_tol(n) * abs(ref)
    ctx.free(dx)
    di = ctx.empty(n, np.int32)
    ctx.fill_uniform_i32(di, seed=43, stream=1)
    oi = ctx.empty(1, np.int64)
    ovf = ctx.empty(1, np.int32)
    ctx.reduce_sum_i32(di, oi, ovf)
    ctx.synchronize()
    xi = oracle.gen_uniform_i32(n, 43, 1)
    assert oi.to_host()[0] == oracle.sum_i32_exact(xi)
    assert ovf.to_host()[0] == 0 and oracle.sum_i32_bcl(xi) == int(oracle.sum_i32_exact(xi))
    # the BCL's lane rule at full size: elements 0, 8 and 16 (lane 0) push lane 0 past
    # int.MaxValue and back, while the total stays small: OverflowException by the rule, not by the total
    planted = {0: 1000, 8: 2**31 - 500, 16: -(2**31 - 500)}
    for i, v in planted.items():
        xi[i] = v
        hip.check(hip.load().dc_hip_memcpy_h2d_async(ctx.handle, di.ptr + 4 * i, xi[i:i + 1].ctypes.data, 4), "h2d")
    ctx.reduce_sum_i32(di, oi, ovf)
    ctx.synchronize()
    assert oi.to_host()[0] == oracle.sum_i32_exact(xi)
    with pytest.raises(OverflowError):
        oracle.sum_i32_bcl(xi)
    assert ovf.to_host()[0] == 1
    for a in (out, di, oi, ovf):
        ctx.free(a)


# ---------------------------------------------------------------- streaming probes (bench ceilings)
@pytest.mark.parametrize("n", [0, 8, 4096, 1_000_000])
def test_stream_probes(ctx, n):
    """The measurement-only probes the bench reports as ceilings do what they claim: a copy, the
    sum of the two halves, and a read that writes nothing."""
    x = oracle.gen_uniform_f32(n, 5, 0)
    dx, dd = ctx.to_device(x), ctx.empty(max(n, 8), np.float32)
    sentinel = np.full(max(n, 8), 7.0, np.float32)
    dd.copy_from(sentinel)
    ctx.stream_probe(hip.PROBE_COPY, dx, dd, n)
    ctx.synchronize()
    assert np.array_equal(dd.to_host(n).view(np.uint32), x.view(np.uint32))
    ctx.stream_probe(hip.PROBE_READ2_WRITE1, dx, dd, n)
    ctx.synchronize()
    h = n // 2
    assert np.array_equal(dd.to_host(h), (x[:h] + x[h:]).astype(np.float32))
    before = dd.to_host()
    ctx.stream_probe(hip.PROBE_READ, dx, dd, n)
    ctx.synchronize()
    assert np.array_equal(dd.to_host().view(np.uint32), before.view(np.uint32))
    for x_ in (dx, dd):
        ctx.free(x_)


def test_stream_probe_arguments(ctx):
    dx, dd = ctx.empty(16, np.float32), ctx.empty(16, np.float32)
    lib = hip.load_bench()
    assert lib.dc_bench_stream_probe(ctx.handle, hip.PROBE_COPY, dx.ptr, dd.ptr, 12) == hip.DC_ERR_INVALID_ARGUMENT
    assert lib.dc_bench_stream_probe(ctx.handle, 3, dx.ptr, dd.ptr, 8) == hip.DC_ERR_INVALID_ARGUMENT
    assert lib.dc_bench_stream_probe(ctx.handle, hip.PROBE_COPY, dx.ptr + 4, dd.ptr, 8) == hip.DC_ERR_MISALIGNED
    for x_ in (dx, dd):
        ctx.free(x_)
