"""GPU parity: MathF.Pow in Where/Select lambdas (the reference maps Pow to the CUDA pow,
CudaKernelGenerator.cs:1380; LINQ-to-objects calls MathF.Pow, which is the C runtime's powf).

pow is not correctly rounded in either library: the device's powf and the C runtime's are each
within 1 ulp of the exact value, so the tolerance is 2 ulp between the two, stated per test. Special
values (NaN, infinities, signed zeros, exact cases) must match bit for bit, and so must the kept
count and the order of the kept elements. Programs with POW run on their own interpreter variant
(kernels with the library call compiled in); both ToArray grids are checked against each other.
"""
import math

import numpy as np
import pytest

import oracle
from dotcompute_amd import hip
from dotcompute_amd.hip import (ADD, CMP_GT, CMP_LT, FILTER, LOAD, MAP, MUL, POW, RPOW, SRC_ELEM, SRC_IMM, SRC_S0,
                                STORE_S0, LinqChain)

from test_gpu_linq import run_minmax, run_sum, run_to_array

pytestmark = pytest.mark.gpu

ULP_TOL = 2  # device powf vs C runtime powf: each within 1 ulp of the exact value

SPECIALS = np.array([0.0, -0.0, 1.0, -1.0, 2.0, -2.0, 0.5, -0.5, np.inf, -np.inf, np.nan, 1e-45, -1e-45,
                     3.4e38, -3.4e38, 1e-38, 16.0, -27.0, 0.25, 1e10], np.float32)


def inputs(n, seed):
    x = oracle.gen_uniform_f32(n, seed, 0) * np.float32(6.0)
    x[: min(n, SPECIALS.size)] = SPECIALS[: min(n, SPECIALS.size)]
    return x


def ordered_bits(a):
    """Float32 bit patterns mapped to integers in the order of the floats they encode."""
    i = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    return np.where(i < 0, -(i & 0x7FFFFFFF), i)


def assert_pow_close(got, want):
    """Same length; NaN where the oracle has NaN; infinities and zeros (with their sign) bit for
    bit; every finite value within ULP_TOL ulp."""
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    assert got.shape == want.shape
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    exact = ~nan & (np.isinf(want) | (want == 0))
    assert np.array_equal(got[exact].view(np.uint32), want[exact].view(np.uint32))
    d = np.abs(ordered_bits(got[~nan]) - ordered_bits(want[~nan]))
    assert d.size == 0 or int(d.max()) <= ULP_TOL, (int(d.max()), got[~nan][d.argmax()], want[~nan][d.argmax()])


# Select-only programs: x => MathF.Pow(x, c), c => MathF.Pow(c, x), x => MathF.Pow(x, x), and
# x => MathF.Pow(x + 1f, x * 0.5f) (both operands computed: the exponent goes through a save register).
SELECT_PROGRAMS = {
    "x^2": [(LOAD, SRC_ELEM, 0), (POW, SRC_IMM, 2.0), (MAP, SRC_IMM, 0)],
    "x^0.5": [(LOAD, SRC_ELEM, 0), (POW, SRC_IMM, 0.5), (MAP, SRC_IMM, 0)],
    "x^-1.5": [(LOAD, SRC_ELEM, 0), (POW, SRC_IMM, -1.5), (MAP, SRC_IMM, 0)],
    "x^3": [(LOAD, SRC_ELEM, 0), (POW, SRC_IMM, 3.0), (MAP, SRC_IMM, 0)],
    "x^(1/3)": [(LOAD, SRC_ELEM, 0), (POW, SRC_IMM, 1.0 / 3.0), (MAP, SRC_IMM, 0)],
    "2^x": [(LOAD, SRC_ELEM, 0), (RPOW, SRC_IMM, 2.0), (MAP, SRC_IMM, 0)],
    "(-1.5)^x": [(LOAD, SRC_ELEM, 0), (RPOW, SRC_IMM, -1.5), (MAP, SRC_IMM, 0)],
    "x^x": [(LOAD, SRC_ELEM, 0), (POW, SRC_ELEM, 0), (MAP, SRC_IMM, 0)],
    "(x+1)^(x/2)": [(LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 0.5), (STORE_S0, SRC_IMM, 0), (LOAD, SRC_ELEM, 0),
                    (ADD, SRC_IMM, 1.0), (POW, SRC_S0, 0), (MAP, SRC_IMM, 0)],
}


@pytest.mark.parametrize("n", [1, 20, 4097, 1_000_000, 4_000_003])
@pytest.mark.parametrize("name", sorted(SELECT_PROGRAMS))
def test_pow_select_matches_csharp_within_2ulp(ctx, name, n):
    chain = LinqChain.assemble(SELECT_PROGRAMS[name])
    x = inputs(n, 80 + n % 7)
    got = run_to_array(ctx, chain, x)  # also checks the lookback grid against the round-robin one
    assert_pow_close(got, oracle.linq_where_select(chain, x))


def test_pow_select_integer_exponents_are_exact_on_small_integers(ctx):
    """Results that are representable and far from any rounding boundary: small integers raised
    to small integer powers (3^7 = 2187, (-2)^5 = -32, 10^-2 is not exact and is left out)."""
    base = np.tile(np.arange(-12, 13, dtype=np.float32), 400)
    for e, ref in ((2.0, base ** 2), (3.0, base ** 3), (5.0, base ** 5), (0.0, np.ones_like(base))):
        chain = LinqChain.assemble([(LOAD, SRC_ELEM, 0), (POW, SRC_IMM, e), (MAP, SRC_IMM, 0)])
        got = run_to_array(ctx, chain, base)
        assert np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32)), e


def unambiguous(x, exponent, threshold):
    """The elements whose pow lies more than 8 ulp from the threshold in float64: the two libraries
    (each within 1 ulp) then agree on the comparison."""
    with np.errstate(all="ignore"):
        p = np.power(np.abs(x.astype(np.float64)), exponent)
    ulp = np.spacing(np.float32(threshold)).astype(np.float64)
    return x[~(np.abs(p - threshold) <= 8 * ulp)]


@pytest.mark.parametrize("n", [1000, 1_000_000, 4_000_003])
def test_pow_in_predicate_keeps_the_same_elements(ctx, n):
    """Where(x => MathF.Pow(x, 2.5f) > 3f).Select(x => MathF.Pow(x, 0.75f)): the kept elements and
    their order exactly (no element within 8 ulp of the threshold), the values within 2 ulp."""
    x = np.abs(oracle.gen_uniform_f32(n + n // 4, 91, 0)) * np.float32(3.0)
    x = unambiguous(x, 2.5, 3.0)[:n]
    chain = LinqChain.assemble([(LOAD, SRC_ELEM, 0), (POW, SRC_IMM, 2.5), (CMP_GT, SRC_IMM, 3.0), (FILTER, SRC_IMM, 0),
                                (LOAD, SRC_ELEM, 0), (POW, SRC_IMM, 0.75), (MAP, SRC_IMM, 0)])
    got = run_to_array(ctx, chain, x)
    want = oracle.linq_where_select(chain, x)
    assert got.size == want.size and 0 < want.size < x.size
    assert_pow_close(got, want)


@pytest.mark.parametrize("n", [1000, 1_000_000, 16_000_000])
def test_pow_sum_count_and_min_max(ctx, n):
    """Where(x => x > 0f).Select(x => MathF.Pow(x, 1.5f)) then Sum, Min and Max: the count exactly,
    the sum within the float Sum tolerance of the float64 sequential sum, Min/Max within 2 ulp."""
    x = oracle.gen_uniform_f32(n, 93, 0) * np.float32(4.0)
    chain = LinqChain.assemble([(LOAD, SRC_ELEM, 0), (CMP_GT, SRC_IMM, 0.0), (FILTER, SRC_IMM, 0),
                                (LOAD, SRC_ELEM, 0), (POW, SRC_IMM, 1.5), (MAP, SRC_IMM, 0)])
    got, cnt = run_sum(ctx, chain, x)
    _, seq_double, ref_cnt = oracle.linq_where_select_sum(chain, x)
    assert cnt == ref_cnt > 0
    tol = 1e-5 * max(1.0, math.log2(n))  # the float Sum tolerance; 2 ulp per term is 2.4e-7 relative
    assert abs(got - seq_double) <= tol * abs(seq_double)
    for op, name in ((hip.LINQ_MIN, "min"), (hip.LINQ_MAX, "max")):
        v, c = run_minmax(ctx, chain, x, op)
        rv, rc = oracle.linq_where_select_minmax(chain, x, name)
        assert c == rc
        assert_pow_close(np.array([v]), np.array([rv]))


def test_pow_in_a_filter_of_nan_producing_bases(ctx):
    """Where(x => MathF.Pow(x, 0.5f) < 1f).Select(x => MathF.Pow(x, 0.5f)): negative bases give NaN,
    and NaN < 1f is false, so they are dropped as LINQ-to-objects drops them; -0 and +0 give +0
    (not -0, which sqrt(-0) would give) and are kept; 0.25 gives 0.5 exactly."""
    x = np.array([-4.0, -0.0, 0.0, 0.25, 0.99, 1.0, 4.0, np.nan, -np.inf, np.inf, -1e-45], np.float32)
    x = np.tile(x, 1000)
    chain = LinqChain.assemble([(LOAD, SRC_ELEM, 0), (POW, SRC_IMM, 0.5), (CMP_LT, SRC_IMM, 1.0),
                                (FILTER, SRC_IMM, 0), (MAP, SRC_IMM, 0)])
    got = run_to_array(ctx, chain, x)
    want = oracle.linq_where_select(chain, x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert want.size == 4000
    assert want[:3].view(np.uint32).tolist() == [0, 0, np.float32(0.5).view(np.uint32)]
