"""GPU parity: fused Where/Select chains over int32 sources (AsComputeQueryable over an int[]).

C# int semantics (ComputeQueryableExtensions.cs:249-259 types any unmanaged T; the reference's
generator maps `int` and `%`, CudaKernelGenerator.cs:1351,1399-1416): + - * wrap, / and % truncate,
a zero divisor throws DivideByZeroException and int.MinValue / -1 OverflowException (reported as the
first throwing element's 4 * index + kind), and Sum() after Where/Select throws OverflowException as
soon as the checked running total leaves int32 (Enumerable.Sum over an iterator). Every result is
compared with the oracle's restatement on the same seeded inputs: bit-exact counts, elements, sums,
overflow flags and fault words.
"""
import numpy as np
import pytest

import oracle
from dotcompute_amd import hip
from dotcompute_amd.hip import (ABS, ADD, CMP_EQ, CMP_GT, CMP_LT, CMP_NE, DIV, FILTER, LOAD, MAP, MUL, NEG, REM,
                                RDIV, SRC_ELEM, SRC_IMM, SRC_S0, STORE_S0, SUB, LinqChain)

pytestmark = pytest.mark.gpu

I32_MIN, I32_MAX = -2**31, 2**31 - 1


def chain(instrs):
    return LinqChain.assemble(instrs, int32=True)


# Range(1, 100).Where(x => x % 2 == 0).Select(x => x * x)   (LinqBackendIntegrationTests.cs:309-325)
EVEN_SQUARES = chain([(LOAD, SRC_ELEM, 0), (REM, SRC_IMM, 2), (CMP_EQ, SRC_IMM, 0), (FILTER, SRC_IMM, 0),
                      (LOAD, SRC_ELEM, 0), (MUL, SRC_ELEM, 0), (MAP, SRC_IMM, 0)])
# Where(x => x % 3 != 0).Select(x => x * x - 7 * x)
POLY = chain([(LOAD, SRC_ELEM, 0), (REM, SRC_IMM, 3), (CMP_NE, SRC_IMM, 0), (FILTER, SRC_IMM, 0),
              (LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 7), (STORE_S0, SRC_IMM, 0),
              (LOAD, SRC_ELEM, 0), (MUL, SRC_ELEM, 0), (SUB, SRC_S0, 0), (MAP, SRC_IMM, 0)])
# Select(x => x)
IDENTITY = chain([(LOAD, SRC_ELEM, 0), (MAP, SRC_IMM, 0)])
# Select(x => 100000 / x): throws for x == 0
DIV_BY_X = chain([(LOAD, SRC_ELEM, 0), (RDIV, SRC_IMM, 100000), (MAP, SRC_IMM, 0)])
# Where(x => x != 0).Select(x => 100000 / x): never throws in C# (the Where drops the zeros)
GUARDED_DIV = chain([(LOAD, SRC_ELEM, 0), (CMP_NE, SRC_IMM, 0), (FILTER, SRC_IMM, 0),
                     (LOAD, SRC_ELEM, 0), (RDIV, SRC_IMM, 100000), (MAP, SRC_IMM, 0)])


def put(ctx, x, offset=0):
    """Device copy of int32 `x` placed `offset` elements into its allocation (for misaligned
    starts); returns (allocation, view)."""
    n = x.size
    d = ctx.empty(n + offset + 1, np.int32)
    if n:
        hip.check(hip.load().dc_hip_memcpy_h2d_async(ctx.handle, d.ptr + 4 * offset, x.ctypes.data, x.nbytes), "h2d")
    return d, hip.DeviceArray(ctx, d.ptr + 4 * offset, 4 * n, np.dtype(np.int32), (n,))


def run_to_array(ctx, ch, x, offset=0):
    """ToArray on the kernel the library picks and on the lookback grid (flag
    LINQ_FLAG_ORDERED_GRID): the same first exception and, without one, the same elements."""
    n = x.size
    d, src = put(ctx, x, offset)
    out, cnt, fault = ctx.empty(n + 1, np.int32), ctx.empty(1, np.int64), ctx.empty(1, np.int64)
    res = []
    for c in (ch, type(ch).from_buffer_copy(ch)):
        if res:
            c.flags |= hip.LINQ_FLAG_ORDERED_GRID
        ctx.where_select_i32(c, src, out, cnt, fault, n)
        ctx.synchronize()
        k = int(cnt.to_host()[0])
        f = int(fault.to_host()[0])
        assert k >= 0 or f >= 0, "resident grid reported a wait that gave up"
        res.append((out.to_host(k) if k > 0 and f < 0 else np.empty(0, np.int32), k, f))
    for a in (d, out, cnt, fault):
        ctx.free(a)
    (g0, k0, f0), (g1, k1, f1) = res
    assert f0 == f1
    if f0 < 0:
        assert k0 == k1 and np.array_equal(g0, g1)
    return g0, k0, f0


def run_sum(ctx, ch, x, offset=0):
    n = x.size
    d, src = put(ctx, x, offset)
    s, c, o, f = ctx.empty(1, np.int64), ctx.empty(1, np.int64), ctx.empty(1, np.int32), ctx.empty(1, np.int64)
    ctx.where_select_sum_i32(ch, src, s, c, o, f, n)
    ctx.synchronize()
    res = int(s.to_host()[0]), int(c.to_host()[0]), bool(o.to_host()[0]), int(f.to_host()[0])
    for a in (d, s, c, o, f):
        ctx.free(a)
    return res


def run_minmax(ctx, ch, x, op):
    n = x.size
    d, src = put(ctx, x)
    v, c, f = ctx.empty(1, np.int32), ctx.empty(1, np.int64), ctx.empty(1, np.int64)
    ctx.where_select_minmax_i32(ch, src, op, v, c, f, n)
    ctx.synchronize()
    res = int(v.to_host()[0]), int(c.to_host()[0]), int(f.to_host()[0])
    for a in (d, v, c, f):
        ctx.free(a)
    return res


def test_reference_golden_vectors_as_written(ctx):
    """The reference's LINQ known answers on int sources with int lambdas."""
    r100 = np.arange(1, 101, dtype=np.int32)
    got, k, f = run_to_array(ctx, EVEN_SQUARES, r100)
    assert f == -1 and k == 50 and got[0] == 4 and got[-1] == 10000
    assert run_sum(ctx, EVEN_SQUARES, r100) == (171700, 50, False, -1)  # 4 * (1^2 + ... + 50^2)
    s15 = np.arange(1, 6, dtype=np.int32)
    where_gt = lambda t: [(LOAD, SRC_ELEM, 0), (CMP_GT, SRC_IMM, t), (FILTER, SRC_IMM, 0)]
    times = lambda m: [(LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, m), (MAP, SRC_IMM, 0)]
    # ComputeQueryProviderTests.cs:341-365
    assert run_to_array(ctx, chain(where_gt(3)), s15)[0].tolist() == [4, 5]
    assert run_to_array(ctx, chain(times(2)), np.arange(1, 4, dtype=np.int32))[0].tolist() == [2, 4, 6]
    # LinqBackendIntegrationTests.cs:51-66, :139-161
    assert run_to_array(ctx, chain(where_gt(2) + times(2)), s15)[0].tolist() == [6, 8, 10]
    r10 = np.arange(1, 11, dtype=np.int32)
    assert run_to_array(ctx, chain(where_gt(3) + times(3)), r10)[0].tolist() == [12, 15, 18, 21, 24, 27, 30]
    # :164-176 (Sum over Range(1, 1000)) and ComputeQueryProviderTests.cs:602-612 (Sum of {1..5})
    assert run_sum(ctx, IDENTITY, np.arange(1, 1001, dtype=np.int32))[0] == 500500
    assert run_sum(ctx, IDENTITY, s15)[0] == 15


@pytest.mark.parametrize("n", [0, 1, 3, 63, 4097, 1_000_000, 16_000_000])
@pytest.mark.parametrize("name", ["even_squares", "poly"])
def test_to_array_bit_exact(ctx, n, name):
    ch = {"even_squares": EVEN_SQUARES, "poly": POLY}[name]
    x = oracle.gen_uniform_i32(n, 46, 1, -1000, 1000)
    got, k, f = run_to_array(ctx, ch, x)
    ref, rf = oracle.linq_where_select_i32(ch, x)
    assert f == rf == -1 and k == ref.size and np.array_equal(got, ref)


@pytest.mark.parametrize("offset", [1, 2, 3])
def test_to_array_misaligned(ctx, offset):
    x = oracle.gen_uniform_i32(2_000_003, 47, 1, -50000, 50000)
    got, k, f = run_to_array(ctx, POLY, x, offset)
    ref, _ = oracle.linq_where_select_i32(POLY, x)
    assert f == -1 and np.array_equal(got, ref)


@pytest.mark.parametrize("offset", [1, 2, 3])
def test_to_array_round_robin_misaligned(ctx, offset):
    # large enough for the round-robin grid after the 3-1 peeled head elements, with faults in the
    # head and in the body reported at their sequence index
    n = 4 * min(hip.device_info(0).compute_units, 256) * 8192 + 7
    x = oracle.gen_uniform_i32(n, 57, 1, -1000, 1000)
    d, src = put(ctx, x, offset)
    assert ctx.to_array_strategy(src, n) == hip.STRATEGY_ROUNDS
    ctx.free(d)
    got, k, f = run_to_array(ctx, POLY, x, offset)
    ref, rf = oracle.linq_where_select_i32(POLY, x)
    assert f == rf == -1 and k == ref.size and np.array_equal(got, ref)
    for zero in (4 - offset - 1, n - 5):  # the last head element, then an element near the end
        y = x.copy()
        y[y == 0] = 1
        y[zero] = 0
        assert run_to_array(ctx, DIV_BY_X, y, offset)[2] == 4 * zero + hip.LINQ_FAULT_DIVIDE_BY_ZERO


def test_to_array_256m_bit_exact(ctx):
    n = 256 * 1024 * 1024
    x = oracle.gen_uniform_i32(n, 48, 1, -1000, 1000)
    d = ctx.to_device(x)
    assert ctx.to_array_strategy(d, n) == hip.STRATEGY_ROUNDS  # the resident round-robin grid
    ctx.free(d)
    got, k, f = run_to_array(ctx, EVEN_SQUARES, x)
    ref, rf = oracle.linq_where_select_i32(EVEN_SQUARES, x)
    assert f == rf == -1 and k == ref.size and np.array_equal(got, ref)
    total, cnt, ovf, f = run_sum(ctx, POLY, x)
    rt, rc, ro, rf = oracle.linq_where_select_sum_i32(POLY, x)
    assert (total, cnt, ovf, f) == (rt, rc, ro, rf) and ovf


@pytest.mark.parametrize("n", [0, 1, 5, 31, 32, 33, 1_000_000, 16_000_000])
def test_sum_count_minmax_match_oracle(ctx, n):
    x = oracle.gen_uniform_i32(n, 49, 1, -1000, 1000)
    for ch in (EVEN_SQUARES, POLY, IDENTITY, GUARDED_DIV):
        assert run_sum(ctx, ch, x) == oracle.linq_where_select_sum_i32(ch, x)
        for op, name in ((hip.LINQ_MIN, "min"), (hip.LINQ_MAX, "max")):
            v, c, f = run_minmax(ctx, ch, x, op)
            rv, rc, rf = oracle.linq_where_select_minmax_i32(ch, x, name)
            assert (c, f) == (rc, rf) and (c == 0 or v == rv)


def big_with(n, seed, values: dict):
    """Small random values with `values` planted; the element before the first planted one brings
    the running total back to exactly 0 there, so the planted values alone decide the overflow."""
    x = oracle.gen_uniform_i32(n, seed, 1, -100, 100)
    first = min(values)
    if first >= 1:
        x[first - 1] = 0
        x[first - 1] = -int(x[:first].astype(np.int64).sum())
    for i, v in values.items():
        x[i] = v
    return x


@pytest.mark.parametrize("where", [0, 1, 2, 5_000_000, 16_000_000 - 4])
def test_sum_overflow_inside_a_chunk_is_found(ctx, where):
    """The running total crosses int.MaxValue and comes back within a few elements: the chunk's end
    is in range, so the overflow is found only by the exact in-order check of that chunk."""
    n = 16_000_000
    x = big_with(n, 50, {where: I32_MAX - 100, where + 1: 1000, where + 2: -1000, where + 3: -(I32_MAX - 100)})
    total, cnt, ovf, f = run_sum(ctx, IDENTITY, x)
    assert (total, cnt, ovf, f) == oracle.linq_where_select_sum_i32(IDENTITY, x)
    assert ovf and total == int(x.astype(np.int64).sum())


@pytest.mark.parametrize("where", [0, 3, 5_000_000, 16_000_000 - 3])
def test_sum_near_the_limit_without_overflow(ctx, where):
    """Bounds that straddle int.MaxValue while the actual running total never leaves int32."""
    n = 16_000_000
    x = big_with(n, 51, {where: I32_MAX - 1000, where + 1: -2000, where + 2: 1000 - (I32_MAX - 1000)})
    total, cnt, ovf, f = run_sum(ctx, IDENTITY, x)
    ref = oracle.linq_where_select_sum_i32(IDENTITY, x)
    assert (total, cnt, ovf, f) == ref and not ovf, ref


def test_sum_overflow_depends_on_the_kept_elements(ctx):
    """Where(x != 7).Select(x): a dropped element does not enter the running total."""
    n = 4_000_000
    x = big_with(n, 52, {100: I32_MAX - 10, 101: 7, 102: 7, 103: -(I32_MAX - 10)})
    x[104:][x[104:] == 7] = 8
    ch = chain([(LOAD, SRC_ELEM, 0), (CMP_NE, SRC_IMM, 7), (FILTER, SRC_IMM, 0), (LOAD, SRC_ELEM, 0), (MAP, SRC_IMM, 0)])
    assert run_sum(ctx, ch, x) == oracle.linq_where_select_sum_i32(ch, x)
    assert not run_sum(ctx, ch, x)[2]        # without the two 7s the total stays at MaxValue - 10 + ...
    assert run_sum(ctx, IDENTITY, x)[2]      # with them it passes MaxValue


@pytest.mark.parametrize("offset", [0, 1, 2, 3])
def test_sum_misaligned_head_and_tail(ctx, offset):
    n = 1_000_005
    x = big_with(n, 53, {0: I32_MAX - 5, 1: 10, 2: -20, n - 2: 5})
    assert run_sum(ctx, IDENTITY, x, offset) == oracle.linq_where_select_sum_i32(IDENTITY, x)


@pytest.mark.parametrize("n", [1000, 1_000_000, 16_000_000])
def test_faults_report_the_first_throwing_element(ctx, n):
    x = oracle.gen_uniform_i32(n, 54, 1, 1, 1000)  # no zeros
    zeros = [n - 1, n // 2 + 17, n // 3]
    for z in zeros:
        x[z] = 0
    first = 4 * min(zeros) + hip.LINQ_FAULT_DIVIDE_BY_ZERO
    assert hip.can_fault_i32(DIV_BY_X) and not hip.can_fault_i32(EVEN_SQUARES)
    _, _, f = run_to_array(ctx, DIV_BY_X, x)
    assert f == first == oracle.linq_where_select_i32(DIV_BY_X, x)[1]
    assert run_sum(ctx, DIV_BY_X, x)[3] == first
    assert run_minmax(ctx, DIV_BY_X, x, hip.LINQ_MAX)[2] == first
    # the Where drops the zeros: no exception, and the results are the oracle's
    got, k, f = run_to_array(ctx, GUARDED_DIV, x)
    ref, rf = oracle.linq_where_select_i32(GUARDED_DIV, x)
    assert f == rf == -1 and np.array_equal(got, ref)
    assert run_sum(ctx, GUARDED_DIV, x) == oracle.linq_where_select_sum_i32(GUARDED_DIV, x)


def test_overflow_faults(ctx):
    """int.MinValue / -1 and Math.Abs(int.MinValue) throw OverflowException; unchecked -x wraps."""
    x = np.array([5, -3, I32_MIN, 7, I32_MIN] + [1] * 10000, np.int32)
    div_m1 = chain([(LOAD, SRC_ELEM, 0), (DIV, SRC_IMM, -1), (MAP, SRC_IMM, 0)])
    absx = chain([(LOAD, SRC_ELEM, 0), (ABS, SRC_IMM, 0), (MAP, SRC_IMM, 0)])
    neg = chain([(LOAD, SRC_ELEM, 0), (NEG, SRC_IMM, 0), (MAP, SRC_IMM, 0)])
    for ch in (div_m1, absx):
        _, _, f = run_to_array(ctx, ch, x)
        assert f == 4 * 2 + hip.LINQ_FAULT_OVERFLOW == oracle.linq_where_select_i32(ch, x)[1]
    got, k, f = run_to_array(ctx, neg, x)
    assert f == -1 and got[2] == I32_MIN and got[0] == -5
    # a Where before the division skips the elements it drops
    safe = chain([(LOAD, SRC_ELEM, 0), (CMP_GT, SRC_IMM, I32_MIN), (FILTER, SRC_IMM, 0),
                  (LOAD, SRC_ELEM, 0), (DIV, SRC_IMM, -1), (MAP, SRC_IMM, 0)])
    got, k, f = run_to_array(ctx, safe, x)
    assert f == -1 and np.array_equal(got, oracle.linq_where_select_i32(safe, x)[0])


def test_fault_entry_points_need_a_fault_word(ctx):
    x = ctx.empty(16, np.int32)
    out, cnt = ctx.empty(16, np.int32), ctx.empty(1, np.int64)
    st = hip.load().dc_hip_linq_where_select_i32(ctx.handle, hip.C.byref(DIV_BY_X), x.ptr, 16, out.ptr, cnt.ptr, None)
    assert st == hip.DC_ERR_INVALID_ARGUMENT
    sq = chain([(LOAD, SRC_ELEM, 0), (hip.SQRT, SRC_IMM, 0), (MAP, SRC_IMM, 0)])
    st = hip.load().dc_hip_linq_where_select_i32(ctx.handle, hip.C.byref(sq), x.ptr, 16, out.ptr, cnt.ptr, None)
    assert st == hip.DC_ERR_UNSUPPORTED
    for a in (x, out, cnt):
        ctx.free(a)


def test_random_int_programs_match_oracle(ctx):
    """Random straight-line int programs (wrapping + - *, % and / by constants, min/max/neg/abs,
    comparisons) over values that hit the wrap-around, checked element for element."""
    rng = np.random.default_rng(55)
    x = oracle.gen_uniform_i32(300_000, 56, 1, -2_000_000_000, 2_000_000_000)
    x[:6] = [0, 1, -1, I32_MIN, I32_MAX, I32_MIN + 1]
    value_ops = [ADD, SUB, MUL, REM, DIV, hip.MIN, hip.MAX]
    for trial in range(12):
        code = []
        for stage in range(int(rng.integers(1, 4))):
            code.append((LOAD, SRC_ELEM, 0))
            for _ in range(int(rng.integers(1, 4))):
                op = value_ops[int(rng.integers(len(value_ops)))]
                c = int(rng.integers(2, 100000)) * (1 if rng.random() < 0.5 else -1)
                code.append((op, SRC_IMM, c) if op in (REM, DIV) or rng.random() < 0.7 else (op, SRC_ELEM, 0))
            if rng.random() < 0.3:
                code.append((NEG if rng.random() < 0.5 else ABS, SRC_IMM, 0))
            if rng.random() < 0.5:
                code += [(CMP_LT if rng.random() < 0.5 else CMP_GT, SRC_IMM, int(rng.integers(-10**9, 10**9))),
                         (FILTER, SRC_IMM, 0)]
            else:
                code.append((MAP, SRC_IMM, 0))
        ch = chain(code)
        got, k, f = run_to_array(ctx, ch, x)
        ref, rf = oracle.linq_where_select_i32(ch, x)
        assert f == rf, (trial, code)
        if f < 0:
            assert np.array_equal(got, ref), (trial, code)
        s_ref = oracle.linq_where_select_sum_i32(ch, x)
        s_got = run_sum(ctx, ch, x)
        assert s_got == s_ref if s_ref[3] < 0 else s_got[3] == s_ref[3], (trial, code)


DIVISORS = [2, 3, 7, -7, 10, 1000, -65536, 2**30 + 1, I32_MAX, I32_MIN, -2, 641]


@pytest.mark.parametrize("d", DIVISORS)
def test_division_by_constants_on_every_terminal(ctx, d):
    """x / d and x % d for constants the kernels divide by multiply-high (the constants are computed
    on the host once per launch): ToArray (both grids), checked Sum and Min/Max against the oracle,
    over values that include int.MinValue, int.MaxValue, 0 and +-1."""
    x = oracle.gen_uniform_i32(300_001, 70, 1, I32_MIN, I32_MAX)
    x[:7] = [I32_MIN, I32_MAX, 0, 1, -1, d, -d if d != I32_MIN else 5]
    for op in (DIV, REM):
        ch = chain([(LOAD, SRC_ELEM, 0), (op, SRC_IMM, d), (MAP, SRC_IMM, 0)])
        got, k, f = run_to_array(ctx, ch, x)
        ref, rf = oracle.linq_where_select_i32(ch, x)
        assert f == rf == -1 and k == ref.size and np.array_equal(got, ref), (op, d)
        assert run_sum(ctx, ch, x) == oracle.linq_where_select_sum_i32(ch, x), (op, d)
        for mop, name in ((hip.LINQ_MIN, "min"), (hip.LINQ_MAX, "max")):
            v, c, f = run_minmax(ctx, ch, x, mop)
            rv, rc, rf = oracle.linq_where_select_minmax_i32(ch, x, name)
            assert (v, c, f) == (rv, rc, rf), (op, d, name)


def test_division_constants_when_the_program_is_full(ctx):
    """A program of 47 instructions with 23 divisions by constants: the constants no longer fit as
    extra instructions (48 at most), and the kernels derive them themselves; results still match."""
    code = [(LOAD, SRC_ELEM, 0)]
    for i in range(22):
        code.append((REM if i % 2 else DIV, SRC_IMM, 3 + 2 * i))
        code.append((ADD, SRC_ELEM, 0))
    code.append((DIV, SRC_IMM, 5))
    code.append((MAP, SRC_IMM, 0))
    assert len(code) == 47
    ch = chain(code)
    x = oracle.gen_uniform_i32(100_003, 71, 1, -10**6, 10**6)
    got, k, f = run_to_array(ctx, ch, x)
    ref, rf = oracle.linq_where_select_i32(ch, x)
    assert f == rf == -1 and np.array_equal(got, ref)
    assert run_sum(ctx, ch, x) == oracle.linq_where_select_sum_i32(ch, x)
