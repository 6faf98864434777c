"""GPU: dc_hip_linq_where_select_sum_f32_noalloc, the allocation-free variant of the LINQ Sum
entry point (its partials live in a static device array resolved at context creation), against
dc_hip_linq_where_select_sum_f32 through the C ABI: two calls in a row, the second on a smaller
input, each bit-identical in sum and count to the allocating entry point (same kernels and grid,
so the same summation order), and within the fp32 sum tolerance of the oracle."""
import ctypes as C
import math

import numpy as np
import pytest

import oracle
from dotcompute_amd import hip

pytestmark = pytest.mark.gpu


def run(ctx, fn, chain, dx, n):
    s = ctx.empty(1, np.float64)
    c = ctx.empty(1, np.int64)
    hip.check(getattr(hip.load(), fn)(ctx.handle, C.byref(chain), dx.ptr, n, s.ptr, c.ptr), fn)
    ctx.synchronize()
    r = float(s.to_host()[0]), int(c.to_host()[0])
    ctx.free(s)
    ctx.free(c)
    return r


def test_noalloc_sum_matches_allocating_entry_point(ctx):
    chain = hip.where_gt0_select_2x_plus_1()
    for n in (20_000_003, 1_000_001, 0, 4097):  # the second call is smaller than the first
        x = oracle.gen_uniform_f32(n, 46, 0)
        dx = ctx.to_device(x) if n else ctx.empty(1, np.float32)
        got = run(ctx, "dc_hip_linq_where_select_sum_f32_noalloc", chain, dx, n)
        ref = run(ctx, "dc_hip_linq_where_select_sum_f32", chain, dx, n)
        assert got[1] == ref[1]
        assert np.float64(got[0]).view(np.uint64) == np.float64(ref[0]).view(np.uint64), (n, got, ref)
        f, d, cnt = oracle.where_gt0_select_2x_plus_1_sum(x)
        assert got[1] == cnt
        assert abs(got[0] - d) <= 1e-5 * max(1.0, math.log2(max(n, 2))) * abs(d) + 1e-12
        ctx.free(dx)


def test_noalloc_sum_general_chain_and_errors(ctx):
    """An interpreted chain (not the affine fast path) and argument errors: the same checks as
    the allocating entry point, with no device work on a rejected call."""
    chain = hip.LinqChain.assemble([(hip.LOAD, hip.SRC_ELEM, 0), (hip.MUL, hip.SRC_ELEM, 0),
                                    (hip.CMP_GT, hip.SRC_IMM, 0.25), (hip.FILTER, 0, 0),
                                    (hip.LOAD, hip.SRC_ELEM, 0), (hip.ABS, 0, 0), (hip.SQRT, 0, 0),
                                    (hip.MAP, 0, 0)])
    n = 3_000_000
    x = oracle.gen_uniform_f32(n, 47, 0)
    dx = ctx.to_device(x)
    a = run(ctx, "dc_hip_linq_where_select_sum_f32_noalloc", chain, dx, n)
    b = run(ctx, "dc_hip_linq_where_select_sum_f32", chain, dx, n)
    assert a == b
    L = hip.load()
    s = ctx.empty(1, np.float64)
    assert L.dc_hip_linq_where_select_sum_f32_noalloc(ctx.handle, C.byref(chain), dx.ptr, -1, s.ptr, None) \
        == hip.DC_ERR_INVALID_ARGUMENT
    assert L.dc_hip_linq_where_select_sum_f32_noalloc(ctx.handle, C.byref(chain), None, 5, s.ptr, None) \
        == hip.DC_ERR_INVALID_ARGUMENT
    ctx.free(s)
    ctx.free(dx)


def test_noalloc_calls_from_two_contexts_do_not_race(ctx):
    """Two contexts on one GPU share the static partials: calls enqueued back to back from both,
    without synchronising in between, each return their own input's sum (the library orders each
    call behind the other context's previous one)."""
    chain = hip.where_gt0_select_2x_plus_1()
    other = hip.Context(0)
    try:
        xa = oracle.gen_uniform_f32(8_000_003, 48, 0)
        xb = oracle.gen_uniform_f32(6_000_001, 49, 0)
        da, db = ctx.to_device(xa), other.to_device(xb)
        ref_a = run(ctx, "dc_hip_linq_where_select_sum_f32", chain, da, xa.size)
        ref_b = run(other, "dc_hip_linq_where_select_sum_f32", chain, db, xb.size)
        outs = []
        L = hip.load()
        for it in range(6):
            for c, d, n in ((ctx, da, xa.size), (other, db, xb.size)):
                s, k = c.empty(1, np.float64), c.empty(1, np.int64)
                hip.check(L.dc_hip_linq_where_select_sum_f32_noalloc(c.handle, C.byref(chain), d.ptr, n, s.ptr, k.ptr),
                          "noalloc")
                outs.append((c, s, k))
        ctx.synchronize()
        other.synchronize()
        for i, (c, s, k) in enumerate(outs):
            want = ref_a if i % 2 == 0 else ref_b
            assert (float(s.to_host()[0]), int(k.to_host()[0])) == want, i
            c.free(s)
            c.free(k)
        ctx.free(da)
        other.free(db)
    finally:
        other.close()
