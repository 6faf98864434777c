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
    """The generic ICompiledKernel path: load dc_kernels_gfx950.hsaco, launch `VectorAdd` with
    the reference's generated signature (a, b, result, __length), block 256, grid ceil(N/256)."""
    import ctypes as C

    L = hip.load()
    path = L.dc_hip_default_module_path()
    assert path, "dc_kernels_gfx950.hsaco not found next to the library"
    mod = C.c_void_p()
    hip.check(L.dc_hip_module_load(ctx.handle, path, C.byref(mod)), "module_load")
    fn = C.c_void_p()
    hip.check(L.dc_hip_module_get_function(mod, b"VectorAdd", C.byref(fn)), "get_function")
    assert L.dc_hip_module_get_function(mod, b"NoSuchKernel", C.byref(C.c_void_p())) == hip.DC_ERR_NOT_FOUND
    n = 100_000
    a = oracle.gen_uniform_f32(n, 42, 0)
    b = oracle.gen_uniform_f32(n, 42, 1)
    da, db, dr = ctx.to_device(a), ctx.to_device(b), ctx.empty(n, np.float32)
    pa, pb, pr = C.c_void_p(da.ptr), C.c_void_p(db.ptr), C.c_void_p(dr.ptr)
    ln = C.c_uint32(n)
    args = (C.c_void_p * 4)(C.addressof(pa), C.addressof(pb), C.addressof(pr), C.addressof(ln))
    hip.check(L.dc_hip_launch_kernel(ctx.handle, fn, (n + 255) // 256, 1, 1, 256, 1, 1, 0,
                                     C.cast(args, C.POINTER(C.c_void_p))), "launch")
    ctx.synchronize()
    assert np.array_equal(dr.to_host(), oracle.vector_add_f32(a, b))
    hip.check(L.dc_hip_module_unload(mod), "unload")
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
    assert out.to_host()[0] == oracle.sum_i32_checked(x)
    assert ovf.to_host()[0] == 0
    for a in (dx, out, ovf):
        ctx.free(a)


def test_sum_i32_overflow_is_reported(ctx):
    x = np.full(4, 2**30, np.int32)  # 2^32 does not fit int32: checked Sum throws
    with pytest.raises(OverflowError):
        oracle.sum_i32_checked(x)
    d = ctx.to_device(x)
    out = ctx.empty(1, np.int64)
    ovf = ctx.empty(1, np.int32)
    ctx.reduce_sum_i32(d, out, ovf)
    ctx.synchronize()
    assert out.to_host()[0] == 2**32 and ovf.to_host()[0] == 1
    x2 = np.array([2**31 - 1, 0, 0], np.int32)  # largest representable total: no overflow
    d2 = ctx.to_device(x2)
    ctx.reduce_sum_i32(d2, out, ovf)
    ctx.synchronize()
    assert out.to_host()[0] == 2**31 - 1 and ovf.to_host()[0] == 0
    for a in (d, d2, out, ovf):
        ctx.free(a)


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
    for a in (out, di, oi, ovf):
        ctx.free(a)
