"""GPU parity: LINQ programs compiled at run time (hipRTC) against the interpreter and the oracle.

A ToArray of at least LINQ_COMPILE_MIN_ELEMENTS elements whose program has no prebuilt kernel runs on
a round-robin kernel compiled for that program (the reference compiles every query with NVRTC and
caches it: CudaRuntimeKernelCompiler.cs:80-138). The compiled kernel must return exactly what the
interpreter returns (the same elements bit for bit, the same count, the same first exception), and
both what the oracle's restatement of LINQ-to-objects returns. LINQ_FLAG_INTERPRET forces the
interpreter on the same input for the comparison.
"""
import numpy as np
import pytest

import oracle
from dotcompute_amd import hip
from dotcompute_amd.hip import (ABS, ADD, CMP_AND, CMP_GE, CMP_GT, CMP_LE, CMP_LT, CMP_NE, CMP_OR, DIV, FILTER, LOAD,
                                MAP, MAX, MIN, MUL, NEG, PAND_Q, PNOT, POR_Q, PSTORE, RDIV, REM, RSUB, SQRT, SRC_ELEM,
                                SRC_IMM, SRC_S0, SRC_S1, STORE_S0, STORE_S1, SUB, LinqChain)

pytestmark = [pytest.mark.gpu,
              pytest.mark.skip(reason="ToArray does not launch compiled kernels: a compiled kernel for a filtered "
                                      "division faulted the device and its cause is not found yet")]

N_MIN = hip.LINQ_COMPILE_MIN_ELEMENTS


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def interpreted(chain):
    ch = type(chain).from_buffer_copy(chain)
    ch.flags |= hip.LINQ_FLAG_INTERPRET
    return ch


def float_program(rng):
    """Random float program: filters (with predicate combinations) and maps over every value op,
    operands from constants, the element and the save registers."""
    code = []
    for _ in range(int(rng.integers(1, 4))):
        if rng.integers(0, 2):
            code.append((LOAD, SRC_ELEM, 0))
            code.append((int(rng.choice([CMP_GT, CMP_GE, CMP_LT, CMP_LE, CMP_NE])), SRC_IMM, float(rng.uniform(-1, 1))))
            if rng.integers(0, 2):
                code += [(PSTORE, SRC_IMM, 0), (LOAD, SRC_ELEM, 0), (ABS, SRC_IMM, 0),
                         (CMP_LT, SRC_IMM, float(rng.uniform(0.2, 1.0)), int(rng.choice([CMP_AND, CMP_OR]))),
                         (int(rng.choice([PAND_Q, POR_Q])), SRC_IMM, 0)]
            if rng.integers(0, 4) == 0:
                code.append((PNOT, SRC_IMM, 0))
            code.append((FILTER, SRC_IMM, 0))
        else:
            code.append((LOAD, SRC_ELEM, 0))
            for _ in range(int(rng.integers(1, 5))):
                op = int(rng.choice([ADD, SUB, RSUB, MUL, DIV, RDIV, MIN, MAX, NEG, ABS, SQRT, REM]))
                if rng.integers(0, 3) == 0:
                    code.append((STORE_S0, SRC_IMM, 0))
                    code.append((op, SRC_S0, float(rng.uniform(-2, 2))))
                else:
                    code.append((op, SRC_ELEM if rng.integers(0, 4) == 0 else SRC_IMM, float(rng.uniform(-2, 2))))
            if rng.integers(0, 2):
                code += [(STORE_S1, SRC_IMM, 0), (ADD, SRC_S1, 0)]
            code.append((MAP, SRC_IMM, 0))
    return LinqChain.assemble(code)


def int_program(rng):
    """Random int program: wrapping + - *, / and % by constants (multiply-high) and by the element
    (which throws on zeros), min/max/neg/abs, comparisons."""
    value_ops = [ADD, SUB, MUL, REM, DIV, MIN, MAX]
    code = []
    for _ in range(int(rng.integers(1, 4))):
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
    return LinqChain.assemble(code, int32=True)


def run(ctx, chain, x, offset, is_int):
    """(elements, count, fault) of ToArray over x placed `offset` elements into its allocation."""
    n = x.size
    dt = np.int32 if is_int else np.float32
    d = ctx.empty(n + offset + 1, dt)
    hip.check(hip.load().dc_hip_memcpy_h2d_async(ctx.handle, d.ptr + 4 * offset, x.ctypes.data, x.nbytes), "h2d")
    src = hip.DeviceArray(ctx, d.ptr + 4 * offset, 4 * n, np.dtype(dt), (n,))
    out, cnt, fault = ctx.empty(n + 1, dt), ctx.empty(1, np.int64), ctx.empty(1, np.int64)
    if is_int:
        ctx.where_select_i32(chain, src, out, cnt, fault, n)
    else:
        ctx.where_select_f32(chain, src, out, cnt, n)
    ctx.synchronize()
    k = int(cnt.to_host()[0])
    f = int(fault.to_host()[0]) if is_int else -1
    got = out.to_host(k) if k > 0 and f < 0 else np.empty(0, dt)
    for a in (d, out, cnt, fault):
        ctx.free(a)
    return got, k, f


@pytest.mark.parametrize("seed", range(8))
def test_compiled_float_programs(ctx, seed):
    rng = np.random.default_rng(900 + seed)
    prog = float_program(rng)
    x = oracle.gen_uniform_f32(N_MIN + 1237 * seed, 700 + seed, 0)
    offset = seed % 4
    launches, failures = ctx.compile_stats()
    got, k, _ = run(ctx, prog, x, offset, False)
    assert ctx.compile_stats() == (launches + 1, failures), "the program did not run compiled"
    ref_i, ki, _ = run(ctx, interpreted(prog), x, offset, False)
    assert ctx.compile_stats()[0] == launches + 1, "LINQ_FLAG_INTERPRET still compiled"
    assert k == ki and np.array_equal(bits(got), bits(ref_i)), seed
    ref = oracle.linq_where_select(prog, x)
    assert k == ref.size and np.array_equal(bits(got), bits(ref)), seed


@pytest.mark.parametrize("seed", range(8))
def test_compiled_int_programs(ctx, seed):
    rng = np.random.default_rng(1900 + seed)
    prog = int_program(rng)
    x = oracle.gen_uniform_i32(N_MIN + 911 * seed, 800 + seed, 1, -2_000_000_000, 2_000_000_000)
    x[:6] = [1, 2, -1, -2**31, 2**31 - 1, -2**31 + 1]
    if seed % 2:  # zeros late in the input: programs that divide by the element throw there
        x[N_MIN - 5000 + seed] = 0
        x[-3] = 0
    offset = (seed * 3) % 4
    launches, failures = ctx.compile_stats()
    got, k, f = run(ctx, prog, x, offset, True)
    assert ctx.compile_stats() == (launches + 1, failures), "the program did not run compiled"
    gi, ki, fi = run(ctx, interpreted(prog), x, offset, True)
    ref, rf = oracle.linq_where_select_i32(prog, x)
    assert f == fi == rf, seed
    if f < 0:
        assert k == ki == ref.size and np.array_equal(got, gi) and np.array_equal(got, ref), seed


def test_compiled_fault_is_the_first_throwing_element(ctx):
    """Select(x => 100000 / x) with zeros at several places: the compiled kernel reports the first
    one (DivideByZeroException), like the interpreter and LINQ-to-objects."""
    prog = LinqChain.assemble([(LOAD, SRC_ELEM, 0), (RDIV, SRC_IMM, 100000), (MAP, SRC_IMM, 0)], int32=True)
    x = oracle.gen_uniform_i32(N_MIN + 77, 31, 1, 1, 1000)
    for i in (N_MIN - 1, 3_000_001, 123_457):
        x[i] = 0
    got, k, f = run(ctx, prog, x, 0, True)
    assert f == 4 * 123_457 + hip.LINQ_FAULT_DIVIDE_BY_ZERO
    assert run(ctx, interpreted(prog), x, 0, True)[2] == f


def test_small_inputs_and_affine_chains_are_not_compiled(ctx):
    """Below LINQ_COMPILE_MIN_ELEMENTS the interpreter runs (a compile costs more than it saves),
    and affine chains keep their prebuilt kernels at any size."""
    sq = LinqChain.assemble([(LOAD, SRC_ELEM, 0), (MUL, SRC_ELEM, 0), (MAP, SRC_IMM, 0)])
    affine = LinqChain.assemble([(LOAD, SRC_ELEM, 0), (CMP_GT, SRC_IMM, 0.0), (FILTER, SRC_IMM, 0),
                                 (LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 2.0), (ADD, SRC_IMM, 1.0), (MAP, SRC_IMM, 0)])
    launches, _ = ctx.compile_stats()
    x = oracle.gen_uniform_f32(N_MIN - 1, 5, 0)
    got, k, _ = run(ctx, sq, x, 0, False)
    assert np.array_equal(bits(got), bits(x * x))
    x = oracle.gen_uniform_f32(N_MIN + 10, 6, 0)
    got, k, _ = run(ctx, affine, x, 0, False)
    assert np.array_equal(bits(got), bits(oracle.where_gt0_select_2x_plus_1(x)))
    assert ctx.compile_stats()[0] == launches


def test_compiled_kernel_is_reused(ctx):
    """The second run of a program uses the cached kernel: same result, no failure, one launch each."""
    prog = LinqChain.assemble([(LOAD, SRC_ELEM, 0), (REM, SRC_IMM, 7), (CMP_NE, SRC_IMM, 0), (FILTER, SRC_IMM, 0),
                               (LOAD, SRC_ELEM, 0), (MUL, SRC_ELEM, 0), (MAP, SRC_IMM, 0)], int32=True)
    x = oracle.gen_uniform_i32(N_MIN + 1, 9, 1, -40000, 40000)
    launches, failures = ctx.compile_stats()
    a = run(ctx, prog, x, 0, True)
    b = run(ctx, prog, x, 0, True)
    assert ctx.compile_stats() == (launches + 2, failures)
    assert a[1] == b[1] and a[2] == b[2] == -1 and np.array_equal(a[0], b[0])
    ref, _ = oracle.linq_where_select_i32(prog, x)
    assert np.array_equal(a[0], ref)
