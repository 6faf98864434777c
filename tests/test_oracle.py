"""Pins the CPU oracle (oracle/liboracle.so) before it is trusted as the GPU checker.

Each oracle function is checked against something independent of it: the reference's own known
answers, the published SplitMix64 outputs, golden vectors computed with NumPy / math.fsum
(tests/golden/hot_path_golden.json, written by tests/golden/make_golden.py without the oracle),
closed forms (Zipf mean degree, identity matrices, stochastic-matrix invariants) and brute force
on small inputs. A few tests plant a mistake in a copy of an oracle result and check that the
comparison used by the GPU tests catches it.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "hot_path_golden.json")))
KA = GOLDEN["reference_known_answers"]


def from_bits(bits):
    return np.array(bits, np.uint32).view(np.float32)


# ------------------------------------------------------------------ generators
def test_splitmix64_published_outputs():
    # First three outputs of SplitMix64 started from state 0 (Steele/Lea/Flood; Vigna's splitmix64.c).
    expected = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    state = 0
    for e in expected:
        assert oracle.splitmix64(state) == e
        state = (state + 0x9E3779B97F4A7C15) & (2**64 - 1)
    assert [int(h, 16) for h in GOLDEN["splitmix64_from_zero"]] == expected


def test_uniform_generators_match_golden():
    inp = GOLDEN["inputs"]
    assert np.array_equal(oracle.gen_uniform_f32(4096, 42, 0).view(np.uint32), np.array(inp["f32_seed42_stream0_bits"], np.uint32))
    assert np.array_equal(oracle.gen_uniform_f32(4096, 42, 1).view(np.uint32), np.array(inp["f32_seed42_stream1_bits"], np.uint32))
    assert np.array_equal(oracle.gen_uniform_f32(64, 42, 5, True).view(np.uint32),
                          np.array(inp["f32_unit_seed42_stream5_bits"], np.uint32))
    assert oracle.gen_uniform_i32(4096, 43, 1, -1000, 1000).tolist() == inp["i32_seed43_stream1"]


def test_uniform_distribution_properties():
    x = oracle.gen_uniform_f32(1_000_000, 7, 0)
    assert x.min() >= -1.0 and x.max() < 1.0
    assert np.all((x.astype(np.float64) + 1.0) * 2**23 == np.round((x.astype(np.float64) + 1.0) * 2**23))  # 2^-23 grid
    assert abs(float(x.mean())) < 3e-3 and abs(float((x > 0).mean()) - 0.5) < 2e-3
    u = oracle.gen_uniform_f32(1_000_000, 7, 0, True)
    assert u.min() >= 0.0 and u.max() < 1.0 and abs(float(u.mean()) - 0.5) < 2e-3
    i = oracle.gen_uniform_i32(1_000_000, 7, 1, -1000, 1000)
    assert i.min() == -1000 and i.max() == 1000 and abs(float(i.mean())) < 2.0


def test_zipf_graph_closed_form_and_invariants():
    rows = 1_000_000
    rp, col, val = oracle.gen_zipf_csr(rows, 42, alpha=2.0, max_degree=4096)
    deg = np.diff(rp)
    # E[deg] for Zipf(2) on [1, 4096] = H_4096 / H_4096^(2)
    k = np.arange(1, 4097, dtype=np.float64)
    mean = (1.0 / k).sum() / (k ** -2.0).sum()
    assert abs(mean - 5.4) < 0.02
    assert abs(deg.mean() - mean) / mean < 0.02
    assert deg.min() >= 1 and deg.max() <= 4096
    p1 = 1.0 / (k ** -2.0).sum()  # P(deg = 1)
    assert abs(float((deg == 1).mean()) - p1) < 3e-3
    assert np.all(np.diff(rp) >= 1) and rp[0] == 0 and rp[-1] == col.size
    rows_of = np.repeat(np.arange(rows), deg)
    assert not np.any(col == rows_of), "self-loop"
    assert col.min() >= 0 and col.max() < rows
    assert np.array_equal(val, (np.float32(1.0) / deg.astype(np.float32))[rows_of])


# ------------------------------------------------------------------ VectorAdd
def test_vector_add_known_answer_and_golden():
    r = KA["README.md:46-57 VectorAdd"]
    assert oracle.vector_add_f32(np.array(r["a"], np.float32), np.array(r["b"], np.float32)).tolist() == r["result"]
    a = from_bits(GOLDEN["inputs"]["f32_seed42_stream0_bits"])
    b = from_bits(GOLDEN["inputs"]["f32_seed42_stream1_bits"])
    assert np.array_equal(oracle.vector_add_f32(a, b).view(np.uint32), np.array(GOLDEN["vector_add_bits"], np.uint32))


# ------------------------------------------------------------------ Sum
def test_sum_known_answers():
    assert oracle.sum_f32_enumerable(np.arange(1, 6, dtype=np.float32))[0] == KA["ComputeQueryProviderTests.cs:602-612 Sum 1..5"]
    assert oracle.sum_f32_enumerable(np.arange(1, 1001, dtype=np.float32))[0] == KA["LinqBackendIntegrationTests.cs:164-176 Sum 1..1000"]
    assert oracle.sum_f32_enumerable(np.zeros(0, np.float32))[0] == 0.0


def test_sum_f32_against_exact_sum():
    a = from_bits(GOLDEN["inputs"]["f32_seed42_stream0_bits"])
    exact = GOLDEN["sum_f32_exact"]
    assert oracle.sum_f32_compensated(a) == pytest.approx(exact, rel=1e-15, abs=1e-12)
    f, d = oracle.sum_f32_enumerable(a)
    assert abs(d - exact) <= 1e-12 * max(abs(exact), 1)
    assert f == np.float32(d)
    big = oracle.gen_uniform_f32(2_000_000, 9, 0)
    fs = math.fsum(big.astype(np.float64))
    assert abs(oracle.sum_f32_compensated(big) - fs) <= 1e-12 * abs(fs) + 1e-9
    fp, dp = oracle.sum_f32_partitioned(big, 8)
    assert abs(dp - fs) <= 1e-10 * abs(fs) + 1e-6
    # the sum is invariant under permutation up to rounding
    perm = np.random.default_rng(1).permutation(big)
    assert abs(oracle.sum_f32_compensated(perm) - fs) <= 1e-12 * abs(fs) + 1e-9


def test_sum_i32_exact_and_checked_semantics():
    x = np.array(GOLDEN["inputs"]["i32_seed43_stream1"], np.int32)
    assert oracle.sum_i32_exact(x) == GOLDEN["sum_i32_exact"] == oracle.sum_i32_checked(x)
    with pytest.raises(OverflowError):
        oracle.sum_i32_checked(np.array([2**31 - 1, 1], np.int32))
    with pytest.raises(OverflowError):  # a running total that leaves int32 throws even if the end fits
        oracle.sum_i32_checked(np.array([2**31 - 1, 1, -1], np.int32))
    assert oracle.sum_i32_checked(np.array([2**31 - 1, -1, 1], np.int32)) == 2**31 - 1
    assert oracle.sum_i32_checked(np.array([-(2**31), 0], np.int32)) == -(2**31)


def _seq_checked(x):
    """Sequential checked int32 running total with Python ints (the BCL's scalar loop, written
    independently of the oracle): None where it throws."""
    s = 0
    for v in x.tolist():
        s += v
        if not -(2**31) <= s < 2**31:
            return None
    return s


def _bcl(x, lanes=8):
    try:
        return oracle.sum_i32_bcl(np.asarray(x, np.int32), lanes)
    except OverflowError:
        return None


def test_sum_i32_bcl_short_inputs_are_the_sequential_checked_loop():
    rng = np.random.default_rng(3)
    big = 2**31 - 1
    for n in range(0, 32):
        for _ in range(20):
            x = rng.choice([big, -big - 1, 1, -1, 0, big // 2, -(big // 2)], size=n).astype(np.int32)
            assert _bcl(x) == _seq_checked(x)
    assert _bcl([big, 1, -1]) is None          # a running total that leaves int32 throws
    assert _bcl([big, -1, 1]) == big


def test_sum_i32_bcl_no_overflow_is_the_exact_sum():
    for n in (32, 33, 39, 40, 41, 63, 64, 65, 1000, 4097, 100_003):
        x = oracle.gen_uniform_i32(n, 17, 1, -1000, 1000)
        assert _bcl(x) == int(x.astype(np.int64).sum())


def test_sum_i32_bcl_lane_structure():
    """Inputs that tell the BCL's vector path (8 lanes of element classes i mod 8, lane totals added
    in lane order, then the tail from V) apart from a sequential running total."""
    big = 2**31 - 1

    def vec(n, **at):
        x = np.zeros(n, np.int32)
        for k, v in at.items():
            x[int(k[1:])] = v
        return x

    # sequential overflows (big + 1), but lane 0 holds big - 1 and lane 1 holds 1: no throw
    x = vec(32, i0=big, i1=1, i8=-1)
    assert _seq_checked(x) is None and _bcl(x) == big
    # lane 0's running total reaches 2^31 although every sequential prefix fits
    x = vec(32, i0=big, i1=-5, i8=1)
    assert _seq_checked(x) == big - 4 and _bcl(x) is None
    # lane totals (big, 1, -10, ...) overflow when added in lane order; sequentially x1 + x2 comes first
    x = vec(32, i8=big, i1=1, i2=-10)
    assert _seq_checked(x) == big - 9 and _bcl(x) is None
    # where the vector loops stop: n = 40 leaves [32, 40) to the scalar tail (lane 0 = {x0..x24}),
    # n = 41 puts x32 into lane 0 (V = 40)
    x40 = vec(40, i0=big, i1=-1, i32=1)
    x41 = vec(41, i0=big, i1=-1, i32=1)
    assert _bcl(x40) == big and _bcl(x41) is None
    # a tail prefix that overflows although the final total fits
    assert _bcl(vec(40, i32=big, i33=1, i34=-1)) is None
    # the lane count matters: with 4 lanes (Arm64) x0 and x4 share a lane
    x = vec(32, i0=big, i4=1, i1=-1)
    assert _bcl(x, lanes=8) == big and _bcl(x, lanes=4) is None


# ------------------------------------------------------------------ LINQ
def _chain(code):
    from dotcompute_amd.hip import LinqChain
    return LinqChain.assemble(code)


def test_where_select_known_answers_through_interpreter():
    from dotcompute_amd.hip import CMP_GT, FILTER, LOAD, MAP, MUL, SRC_ELEM, SRC_IMM
    w3 = _chain([(LOAD, SRC_ELEM, 0), (CMP_GT, SRC_IMM, 3), (FILTER, SRC_IMM, 0)])
    assert oracle.linq_where_select(w3, np.arange(1, 6, dtype=np.float32)).tolist() == KA[
        "ComputeQueryProviderTests.cs:341-365 Where(x>3) over 1..5"]
    s2 = _chain([(LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 2), (MAP, SRC_IMM, 0)])
    assert oracle.linq_where_select(s2, np.array([1, 2, 3], np.float32)).tolist() == KA[
        "ComputeQueryProviderTests.cs:341-365 Select(x*2) over 1,2,3"]
    ws = _chain([(LOAD, SRC_ELEM, 0), (CMP_GT, SRC_IMM, 2), (FILTER, SRC_IMM, 0),
                 (LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 2), (MAP, SRC_IMM, 0)])
    assert oracle.linq_where_select(ws, np.arange(1, 6, dtype=np.float32)).tolist() == KA[
        "LinqBackendIntegrationTests.cs:51-66 Where(x>2).Select(x*2) over 1..5"]


def test_benchmark_chain_matches_numpy_golden_and_interpreter():
    from dotcompute_amd import hip

    a = from_bits(GOLDEN["inputs"]["f32_seed42_stream0_bits"])
    ref = np.array(GOLDEN["where_gt0_select_2x_plus_1_bits"], np.uint32)
    hand = oracle.where_gt0_select_2x_plus_1(a)
    assert np.array_equal(hand.view(np.uint32), ref)
    interp = oracle.linq_where_select(hip.where_gt0_select_2x_plus_1(), a)
    assert np.array_equal(interp.view(np.uint32), ref)
    f, d, cnt = oracle.where_gt0_select_2x_plus_1_sum(a)
    assert cnt == ref.size and abs(d - GOLDEN["where_gt0_select_2x_plus_1_sum_exact"]) <= 1e-12 * abs(d)
    # +0 and -0 are dropped, NaN is dropped, inf maps to inf
    edge = np.array([0.0, -0.0, np.nan, np.inf, 1e-45, -1.0], np.float32)
    assert oracle.where_gt0_select_2x_plus_1(edge).tolist() == [np.inf, np.float32(1e-45) * 2 + 1]


def _ichain(code):
    from dotcompute_amd.hip import LinqChain
    return LinqChain.assemble(code, int32=True)


def test_int_chains_reference_known_answers():
    """The reference's LINQ known answers on int sources (LinqBackendIntegrationTests.cs:51-66,
    :164-176, :309-325): the oracle's int interpreter against closed forms."""
    from dotcompute_amd.hip import CMP_EQ, CMP_GT, FILTER, LOAD, MAP, MUL, REM, SRC_ELEM, SRC_IMM
    even_sq = _ichain([(LOAD, SRC_ELEM, 0), (REM, SRC_IMM, 2), (CMP_EQ, SRC_IMM, 0), (FILTER, SRC_IMM, 0),
                       (LOAD, SRC_ELEM, 0), (MUL, SRC_ELEM, 0), (MAP, SRC_IMM, 0)])
    r100 = np.arange(1, 101, dtype=np.int32)
    out, fault = oracle.linq_where_select_i32(even_sq, r100)
    assert fault == -1 and out.tolist() == [(2 * k) ** 2 for k in range(1, 51)]
    total, k, ovf, fault = oracle.linq_where_select_sum_i32(even_sq, r100)
    assert (total, k, ovf, fault) == (4 * 50 * 51 * 101 // 6, 50, False, -1)  # 4 * sum of k^2 = 171700
    ws = _ichain([(LOAD, SRC_ELEM, 0), (CMP_GT, SRC_IMM, 2), (FILTER, SRC_IMM, 0),
                  (LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 2), (MAP, SRC_IMM, 0)])
    assert oracle.linq_where_select_i32(ws, np.arange(1, 6, dtype=np.int32))[0].tolist() == [6, 8, 10]
    ident = _ichain([(LOAD, SRC_ELEM, 0), (MAP, SRC_IMM, 0)])
    assert oracle.linq_where_select_sum_i32(ident, np.arange(1, 1001, dtype=np.int32))[0] == 500500


def test_int_chains_match_numpy_wrapping_arithmetic():
    """Where(x % 3 != 0).Select(x * x - 7 * x) over the whole int range: numpy's int32 arithmetic
    wraps as C#'s unchecked int does, and np.fmod truncates as C#'s % does (not Python's %)."""
    from dotcompute_amd.hip import CMP_NE, FILTER, LOAD, MAP, MUL, REM, SRC_ELEM, SRC_IMM, SRC_S0, STORE_S0, SUB
    poly = _ichain([(LOAD, SRC_ELEM, 0), (REM, SRC_IMM, 3), (CMP_NE, SRC_IMM, 0), (FILTER, SRC_IMM, 0),
                    (LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 7), (STORE_S0, SRC_IMM, 0),
                    (LOAD, SRC_ELEM, 0), (MUL, SRC_ELEM, 0), (SUB, SRC_S0, 0), (MAP, SRC_IMM, 0)])
    x = oracle.gen_uniform_i32(200_000, 60, 1, -2_147_483_647, 2_147_483_647)
    x[:4] = [-2**31, 2**31 - 1, -7, -8]
    with np.errstate(over="ignore"):
        keep = np.fmod(x, np.int32(3)) != 0
        y = x[keep] * x[keep] - np.int32(7) * x[keep]
    got, fault = oracle.linq_where_select_i32(poly, x)
    assert fault == -1 and np.array_equal(got, y)
    # the checked running total: the first prefix outside int32, from an int64 cumulative sum
    small = oracle.gen_uniform_i32(300_000, 61, 1, -1000, 1000)
    with np.errstate(over="ignore"):
        ys = (small[np.fmod(small, 3) != 0].astype(np.int64) ** 2) - 7 * small[np.fmod(small, 3) != 0]
    cs = np.cumsum(ys)
    total, k, ovf, fault = oracle.linq_where_select_sum_i32(poly, small)
    assert (total, k, fault) == (int(cs[-1]), ys.size, -1)
    assert ovf == bool((cs > 2**31 - 1).any() or (cs < -2**31).any()) and ovf


def test_int_division_truncates_and_throws_like_csharp():
    """C#: -8 / 7 == -1 and -8 % 7 == -1 (truncation, not floor); a zero divisor throws
    DivideByZeroException and int.MinValue / -1, int.MinValue % -1 and Math.Abs(int.MinValue) throw
    OverflowException (kind 1 and 2 of the fault code 4 * index + kind)."""
    from dotcompute_amd.hip import ABS, DIV, LOAD, MAP, REM, RDIV, SRC_ELEM, SRC_IMM
    div7 = _ichain([(LOAD, SRC_ELEM, 0), (DIV, SRC_IMM, 7), (MAP, SRC_IMM, 0)])
    rem7 = _ichain([(LOAD, SRC_ELEM, 0), (REM, SRC_IMM, 7), (MAP, SRC_IMM, 0)])
    v = np.array([-8, 8, -7, 6, -6, -2**31], np.int32)
    assert oracle.linq_where_select_i32(div7, v)[0].tolist() == [-1, 1, -1, 0, 0, -306783378]
    assert oracle.linq_where_select_i32(rem7, v)[0].tolist() == [-1, 1, 0, 6, -6, -2]
    inv = _ichain([(LOAD, SRC_ELEM, 0), (RDIV, SRC_IMM, 100), (MAP, SRC_IMM, 0)])
    out, fault = oracle.linq_where_select_i32(inv, np.array([3, 50, 0, 0, 1], np.int32))
    assert out.tolist() == [33, 2] and fault == 4 * 2 + 1
    for code in ([(LOAD, SRC_ELEM, 0), (DIV, SRC_IMM, -1), (MAP, SRC_IMM, 0)],
                 [(LOAD, SRC_ELEM, 0), (REM, SRC_IMM, -1), (MAP, SRC_IMM, 0)],
                 [(LOAD, SRC_ELEM, 0), (ABS, SRC_IMM, 0), (MAP, SRC_IMM, 0)]):
        out, fault = oracle.linq_where_select_i32(_ichain(code), np.array([5, -5, -2**31, 9], np.int32))
        assert fault == 4 * 2 + 2 and out.size == 2
    # a planted mistake: a floor-division restatement would be caught by the known answers above
    assert (-8) // 7 == -2 and int(np.fmod(np.int32(-8), np.int32(7))) == -1


def test_float_remainder_and_rounding_closed_forms():
    """C#'s float % is the truncated remainder (C fmodf, exact); MathF.Floor/Ceiling; MathF.Round
    rounds half to even. The interpreter's REM/RREM/FLOOR/CEIL/ROUND against numpy's fmod, floor,
    ceil and rint, bit for bit, over ties, signed zeros, infinities and NaN."""
    from dotcompute_amd.hip import CEIL, FLOOR, LOAD, MAP, REM, ROUND, RREM, SRC_ELEM, SRC_IMM
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 0.0, -0.0, 3.75, -3.75, 1e-40, -7.0, 123456.5,
                  np.inf, -np.inf, np.nan, 0.7499999, -0.75], np.float32)
    x = np.concatenate([x, oracle.gen_uniform_f32(4096, 33, 0) * 50])

    def run(code):
        return np.array([oracle.linq_eval(_chain(code + [(MAP, SRC_IMM, 0)]), float(v))[1] for v in x], np.float32)

    with np.errstate(invalid="ignore", divide="ignore"):
        cases = [([(LOAD, SRC_ELEM, 0), (REM, SRC_IMM, 0.75)], np.fmod(x, np.float32(0.75))),
                 ([(LOAD, SRC_ELEM, 0), (RREM, SRC_IMM, 9.0)], np.fmod(np.float32(9.0), x)),
                 ([(LOAD, SRC_ELEM, 0), (FLOOR, SRC_IMM, 0)], np.floor(x)),
                 ([(LOAD, SRC_ELEM, 0), (CEIL, SRC_IMM, 0)], np.ceil(x)),
                 ([(LOAD, SRC_ELEM, 0), (ROUND, SRC_IMM, 0)], np.rint(x))]
    for code, want in cases:
        got = run(code)
        same = (got.view(np.uint32) == want.astype(np.float32).view(np.uint32)) | (np.isnan(got) & np.isnan(want))
        assert same.all(), (code, x[~same][:4], got[~same][:4], want[~same][:4])
    assert run([(LOAD, SRC_ELEM, 0), (ROUND, SRC_IMM, 0)])[:6].tolist() == [0.0, 2.0, 2.0, -0.0, -2.0, -2.0]


# MathF.Pow special values (IEEE 754-2008 pow, C99 Annex F; .NET Core's MathF.Pow documents the
# same table): (base, exponent, result).
INF, NAN = float("inf"), float("nan")
POW_SPECIALS = [
    (NAN, 0.0, 1.0), (NAN, -0.0, 1.0), (INF, 0.0, 1.0), (-3.5, -0.0, 1.0),    # pow(x, +-0) = 1
    (1.0, NAN, 1.0), (1.0, INF, 1.0), (1.0, -INF, 1.0), (1.0, -2.5, 1.0),    # pow(1, y) = 1
    (-1.0, INF, 1.0), (-1.0, -INF, 1.0),                                     # pow(-1, +-inf) = 1
    (0.0, -3.0, INF), (-0.0, -3.0, -INF), (0.0, -2.0, INF), (-0.0, -2.0, INF), (-0.0, -0.5, INF),
    (0.0, 3.0, 0.0), (-0.0, 3.0, -0.0), (-0.0, 2.0, 0.0), (-0.0, 0.5, 0.0), (-0.0, INF, 0.0),
    (0.5, -INF, INF), (-0.5, -INF, INF), (2.0, -INF, 0.0), (-2.0, -INF, 0.0),
    (0.5, INF, 0.0), (-0.5, INF, 0.0), (2.0, INF, INF), (-2.0, INF, INF),
    (-INF, -3.0, -0.0), (-INF, -2.0, 0.0), (-INF, -0.5, 0.0), (-INF, 3.0, -INF), (-INF, 2.0, INF),
    (-INF, 0.5, INF), (INF, -1.0, 0.0), (INF, 0.5, INF),
    (-8.0, 1.0 / 3.0, NAN), (-2.0, 0.5, NAN), (NAN, 1.0, NAN), (2.0, NAN, NAN),   # NaN results
    (-2.0, 3.0, -8.0), (-2.0, -2.0, 0.25), (2.0, 10.0, 1024.0), (3.0, 2.0, 9.0), (2.0, 3.0, 8.0),
    (0.25, 0.5, 0.5), (1e-30, 2.0, 0.0), (1e30, 2.0, INF), (2.0, -149.0, 2.0 ** -149),
]


def test_float_pow_special_values_and_accuracy():
    """MathF.Pow through the interpreter's POW (v = pow(v, operand)) and RPOW (v = pow(operand, v)):
    every special value of the IEEE/C99 table bit for bit (signed zeros and infinities included),
    operands in the right order (2^3 = 8 but 3^2 = 9), and finite results within 1 ulp of the
    float64 pow rounded to float32 (the C runtime's powf is within 1 ulp of the exact value)."""
    from dotcompute_amd.hip import LOAD, MAP, POW, RPOW, SRC_ELEM, SRC_IMM

    def pow_of(base, exp):  # LOAD base; POW exp
        return oracle.linq_eval(_chain([(LOAD, SRC_IMM, base), (POW, SRC_IMM, exp), (MAP, SRC_IMM, 0)]), 0.0)[1]

    def rpow_of(base, exp):  # the element is the exponent: LOAD e; RPOW base
        return oracle.linq_eval(_chain([(LOAD, SRC_ELEM, 0), (RPOW, SRC_IMM, base), (MAP, SRC_IMM, 0)]), exp)[1]

    for base, exp, want in POW_SPECIALS:
        for got in (pow_of(base, exp), rpow_of(base, exp)):
            w = np.float32(want)
            assert (np.isnan(got) and np.isnan(w)) or np.float32(got).view(np.uint32) == w.view(np.uint32), \
                (base, exp, got, want)
    x = np.abs(oracle.gen_uniform_f32(3000, 71, 0)) * 8.0 + np.float32(1e-3)
    y = oracle.gen_uniform_f32(3000, 72, 0) * 6.0
    for b, e in zip(x.tolist(), y.tolist()):
        ref = np.float32(math.pow(np.float64(np.float32(b)), np.float64(np.float32(e))))
        got = np.float32(pow_of(b, e))
        if np.isinf(ref) or ref == 0.0:
            assert got == ref, (b, e)
        else:
            assert abs(int(got.view(np.int32)) - int(ref.view(np.int32))) <= 1, (b, e, got, ref)


def test_float_fold_min_max_hand_cases_and_numpy():
    """Aggregate((acc, x) => MathF.Min(acc, x)) / MathF.Max, folded in order: -0 below +0 whatever
    the order of the zeros, NaN wherever a NaN is kept (Enumerable.Max would skip it), the
    reference's {5, 2, 8, 1} input (ExpressionTreeVisitorTests.cs:113-147), and numpy min/max of
    the kept, mapped values on NaN-free data without zeros, where the fold and Enumerable agree."""
    from dotcompute_amd.hip import CMP_GT, FILTER, LOAD, MAP, MUL, SRC_ELEM, SRC_IMM
    ident = _chain([])
    f32 = lambda v: np.array(v, np.float32)
    for xs, mn, mx in (([0.0, -0.0], -0.0, 0.0), ([-0.0, 0.0], -0.0, 0.0), ([5.0, 2.0, 8.0, 1.0], 1.0, 8.0),
                       ([3.0, np.nan, 1.0], np.nan, np.nan), ([np.nan], np.nan, np.nan), ([-np.inf, 2.0], -np.inf, 2.0)):
        for op, want in (("min", mn), ("max", mx)):
            got, k = oracle.linq_where_select_fold(ident, f32(xs), op)
            assert k == len(xs)
            assert (np.isnan(got) and np.isnan(want)) or f32(got).view(np.uint32) == f32(want).view(np.uint32), \
                (xs, op, got)
    assert oracle.linq_where_select_fold(ident, f32([]), "min")[1] == 0
    # Enumerable.Max skips the NaN the fold keeps; Enumerable takes the first of equal zeros
    assert oracle.linq_where_select_minmax(ident, f32([3.0, np.nan, 1.0]), "max")[0] == 3.0
    assert oracle.linq_where_select_minmax(ident, f32([0.0, -0.0]), "min")[0].view(np.uint32) == 0
    x = oracle.gen_uniform_f32(50_000, 77, 0)
    x = x[x != 0]
    prog = _chain([(LOAD, SRC_ELEM, 0), (CMP_GT, SRC_IMM, -0.5), (FILTER, SRC_IMM, 0),
                   (LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 3.0), (MAP, SRC_IMM, 0)])
    kept = x[x > np.float32(-0.5)] * np.float32(3.0)
    assert oracle.linq_where_select_fold(prog, x, "min") == (kept.min(), kept.size)
    assert oracle.linq_where_select_fold(prog, x, "max") == (kept.max(), kept.size)


def test_int_min_max_against_numpy():
    """Where/Select then Min/Max over int32: the extreme of the elements ToArray returns, the kept
    count, no value for an empty result, and the first exception when one is thrown."""
    from dotcompute_amd.hip import CMP_GT, FILTER, LOAD, MAP, MUL, RDIV, SRC_ELEM, SRC_IMM
    x = oracle.gen_uniform_i32(100_000, 62, 1, -2_000_000_000, 2_000_000_000)
    prog = _ichain([(LOAD, SRC_ELEM, 0), (CMP_GT, SRC_IMM, -5), (FILTER, SRC_IMM, 0),
                    (LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 3), (MAP, SRC_IMM, 0)])
    kept, fault = oracle.linq_where_select_i32(prog, x)
    assert fault == -1 and kept.size > 0
    assert kept.tolist() == ((x[x > -5].astype(np.int64) * 3 + 2**31) % 2**32 - 2**31).tolist()
    for op, ref in (("min", int(kept.min())), ("max", int(kept.max()))):
        v, k, f = oracle.linq_where_select_minmax_i32(prog, x, op)
        assert (v, k, f) == (ref, kept.size, -1)
    none = _ichain([(LOAD, SRC_ELEM, 0), (CMP_GT, SRC_IMM, 2**31 - 1), (FILTER, SRC_IMM, 0)])
    assert oracle.linq_where_select_minmax_i32(none, x, "max")[1:] == (0, -1)
    inv = _ichain([(LOAD, SRC_ELEM, 0), (RDIV, SRC_IMM, 7), (MAP, SRC_IMM, 0)])
    z = np.array([3, 5, 0, 9, 0], np.int32)
    assert oracle.linq_where_select_minmax_i32(inv, z, "min")[2] == 4 * 2 + 1  # DivideByZero at index 2


def test_planted_mistake_is_caught():
    """The bit comparison the GPU tests use must reject an off-by-one-ulp or reordered result."""
    a = oracle.gen_uniform_f32(10_000, 3, 0)
    good = oracle.where_gt0_select_2x_plus_1(a)
    bad = good.copy()
    bad.view(np.uint32)[17] += 1
    assert not np.array_equal(bad.view(np.uint32), good.view(np.uint32))
    swapped = good.copy()
    swapped[[3, 4]] = swapped[[4, 3]]
    assert not np.array_equal(swapped.view(np.uint32), good.view(np.uint32))


def _f32(bits_list):
    return np.array(bits_list, np.uint32).view(np.float32)


def test_min_max_known_answers_and_empty():
    empty_chain = _chain([])
    ka = KA["FutureExpansionTests.cs:553-570 Sum/Count/Max over Range(1,100)"]
    r100 = np.arange(1, 101, dtype=np.float32)
    assert oracle.linq_where_select_minmax(empty_chain, r100, "max") == (ka["max"], ka["count"])
    assert oracle.linq_where_select_sum(empty_chain, r100)[1] == ka["sum"]
    ka4 = KA["ExpressionTreeVisitorTests.cs:113-147 Min/Max over 5,2,8,1"]
    x4 = np.array(ka4["input"], np.float32)
    assert oracle.linq_where_select_minmax(empty_chain, x4, "min")[0] == ka4["min"]
    assert oracle.linq_where_select_minmax(empty_chain, x4, "max")[0] == ka4["max"]
    # an empty sequence (nothing kept) reports count 0; the host layer throws on it
    from dotcompute_amd.hip import CMP_GT, FILTER, LOAD, SRC_ELEM, SRC_IMM
    none = _chain([(LOAD, SRC_ELEM, 0), (CMP_GT, SRC_IMM, 100.0), (FILTER, SRC_IMM, 0)])
    assert oracle.linq_where_select_minmax(none, x4, "min")[1] == 0
    assert oracle.linq_where_select_minmax(empty_chain, np.empty(0, np.float32), "max")[1] == 0


def test_min_max_signed_zero_and_nan_rules():
    """Hand-worked cases of Enumerable.Min/Max(IEnumerable<float>): ties (+0 == -0) keep the earlier
    element; Min returns the first NaN; Max skips NaNs and returns the last NaN when all are NaN."""
    e = _chain([])
    pz, nz = 0x00000000, 0x80000000
    nan_a, nan_b, nan_c = 0x7FC00001, 0x7FC00002, 0x7FC00003
    mm = lambda bits_list, op: oracle.linq_where_select_minmax(e, _f32(bits_list), op)[0].view(np.uint32)
    assert mm([pz, nz], "min") == pz and mm([nz, pz], "min") == nz
    assert mm([pz, nz], "max") == pz and mm([nz, pz], "max") == nz
    one = np.float32(1).view(np.uint32)
    two = np.float32(2).view(np.uint32)
    assert mm([one, nan_a, pz, nan_b], "min") == nan_a   # first NaN, even after smaller values
    assert mm([nan_a, nan_b], "min") == nan_a
    assert mm([nan_a, nan_b, nan_c], "max") == nan_c     # all NaN: the last one
    assert mm([nan_a, two, nan_b, one], "max") == two    # NaNs skipped
    assert mm([one, two, nan_a], "max") == two


def test_min_max_match_numpy_on_nan_free_data():
    from dotcompute_amd import hip
    a = oracle.gen_uniform_f32(100_003, 12, 0)
    kept = oracle.where_gt0_select_2x_plus_1(a)
    ch = hip.where_gt0_select_2x_plus_1()
    assert oracle.linq_where_select_minmax(ch, a, "min") == (kept.min(), kept.size)
    assert oracle.linq_where_select_minmax(ch, a, "max") == (kept.max(), kept.size)
    # the written-out lambdas (the bench's CPU baseline) agree with numpy and the interpreter,
    # also with NaN, -0, +inf and a tie in the input
    assert oracle.where_gt0_select_2x_plus_1_minmax(a, "min") == (kept.min(), kept.size)
    assert oracle.where_gt0_select_2x_plus_1_minmax(a, "max") == (kept.max(), kept.size)
    b = a.copy()
    b[[5, 70, 900, 901, 4000]] = [np.nan, -0.0, np.inf, a[70], a[4000]]
    for op in ("min", "max"):
        got, ref = oracle.where_gt0_select_2x_plus_1_minmax(b, op), oracle.linq_where_select_minmax(ch, b, op)
        assert got[1] == ref[1] and got[0].view(np.uint32) == ref[0].view(np.uint32)
    assert oracle.where_gt0_select_2x_plus_1_minmax(b, "max")[0] == np.inf
    assert oracle.where_gt0_select_2x_plus_1_minmax(-np.abs(a), "min")[1] == 0
    # a planted mistake (taking the last of equal minima) is visible in the bits
    z = _f32([0x3F800000, 0x80000000, 0x00000000])
    assert oracle.linq_where_select_minmax(_chain([]), z, "min")[0].view(np.uint32) == 0x80000000


# ------------------------------------------------------------------ GEMM
def test_gemm_against_numpy_float64_golden():
    a = from_bits(GOLDEN["inputs"]["f32_seed42_stream0_bits"])[: 16 * 24].reshape(16, 24)
    b = from_bits(GOLDEN["inputs"]["f32_seed42_stream1_bits"])[: 24 * 8].reshape(24, 8)
    ref = np.array(GOLDEN["gemm_16x24x8_f64"]).reshape(16, 8)
    c64, absc = oracle.gemm_f64_rows(a, b, np.arange(16))
    assert np.allclose(c64, ref, rtol=0, atol=1e-12)
    assert np.all(absc >= np.abs(c64) - 1e-12)
    c32 = oracle.gemm_f32_naive(a, b)
    assert np.all(np.abs(c32 - ref) <= 1e-5 * absc)


def test_gemm_blocked_equals_naive_bitwise_and_identity():
    a = oracle.gen_uniform_f32(70 * 130, 1, 0).reshape(70, 130)
    b = oracle.gen_uniform_f32(130 * 90, 1, 1).reshape(130, 90)
    # MatrixOperations.MultiplyBlocked keeps each entry's sequential-k order across 64-blocks
    assert np.array_equal(oracle.gemm_f32_blocked(a, b), oracle.gemm_f32_naive(a, b, threads=4))
    eye = np.eye(130, dtype=np.float32)
    assert np.array_equal(oracle.gemm_f32_naive(a, eye), a)


def test_gemm_rank_one_closed_form():
    u = oracle.gen_uniform_f32(64, 2, 0).reshape(64, 1)
    v = oracle.gen_uniform_f32(64, 2, 1).reshape(1, 64)
    c, _ = oracle.gemm_f64_rows(u, v, np.arange(64))
    assert np.array_equal(c, u.astype(np.float64) @ v.astype(np.float64))


def test_bf16_rounding():
    x = np.array([1.0, 1.0039062, 1.0117188, -2.5, np.inf, np.nan, 3.4028235e38, 3.3895314e38], np.float32)
    h = oracle.f32_to_bf16(x)
    # 1.0039062 = 0x3F808000: exact tie -> even (0x3F80); 1.0117188 = 0x3F818000: tie -> 0x3F82
    assert h[0] == 0x3F80 and h[1] == 0x3F80 and h[2] == 0x3F82 and h[3] == 0xC020
    assert h[4] == 0x7F80 and (h[5] & 0x7FFF) > 0x7F80
    assert np.isinf(oracle.bf16_to_f32(h[6:7])[0])  # FLT_MAX rounds up past the largest finite bf16
    assert h[7] == 0x7F7F  # the largest finite bf16 is exact
    r = oracle.bf16_to_f32(oracle.f32_to_bf16(oracle.gen_uniform_f32(10000, 5, 0)))
    assert np.max(np.abs(r - oracle.gen_uniform_f32(10000, 5, 0))) <= 2.0 ** -9


# ------------------------------------------------------------------ SpMV
def test_spmv_golden_and_dimension_check():
    g = GOLDEN["csr_6x6"]
    rp = np.array(g["row_pointers"], np.int32)
    col = np.array(g["col_indices"], np.int32)
    val = from_bits(g["values_f32_bits"])
    x = np.array(g["x"], np.float32)
    y = oracle.spmv_csr_f32(rp, col, val, x)
    assert np.allclose(y, g["y_f64"], rtol=1e-6, atol=0)
    assert y[1] == 0.0  # empty row
    with pytest.raises(ValueError):
        oracle.spmv_csr_f32(rp, col, val, x, cols=7)


def test_spmv_dense_bruteforce_and_power_invariants():
    rows = 300
    rp, col, val = oracle.gen_zipf_csr(rows, 5, max_degree=rows - 1)
    x = oracle.gen_uniform_f32(rows, 5, 5, True)
    dense = np.zeros((rows, rows))
    for r in range(rows):
        for i in range(rp[r], rp[r + 1]):
            dense[r, col[i]] += val[i]
    assert np.allclose(oracle.spmv_csr_f32(rp, col, val, x), dense @ x.astype(np.float64), rtol=1e-5, atol=0)
    # each row sums its out-degree values 1/deg: A·1 = 1 (row-stochastic)
    assert np.allclose(oracle.spmv_csr_f32(rp, col, val, np.ones(rows, np.float32)), 1.0, rtol=1e-6)
    xp, s = oracle.spmv_power_f32(rp, col, val, x, 20)
    assert np.all(xp >= 0) and abs(float(np.sum(xp, dtype=np.float64)) - 1.0) < 1e-5
    # power iteration of a row-stochastic matrix in float64 converges to the same direction
    xd = x.astype(np.float64)
    for _ in range(20):
        yd = dense @ xd
        xd = yd / yd.sum()
    assert np.allclose(xp, xd, rtol=1e-4, atol=1e-9)


def _dense_int(rp, col, val, rows, cols):
    dense = np.zeros((rows, cols), object)
    for r in range(rows):
        for i in range(rp[r], rp[r + 1]):
            dense[r, col[i]] += int(val[i])
    return dense


def test_spmv_double_exact_on_integers_and_index_order():
    """SpMV<double>: integer-valued operands below 2^20 make every product and partial sum exact, so
    the result equals the integer dense product; a row whose order matters (1e16 + 1 - 1e16) pins
    the index order of the additions."""
    rows = 200
    rp, col, _ = oracle.gen_zipf_csr(rows, 7, max_degree=rows - 1)
    rng = np.random.default_rng(7)
    val = rng.integers(-1000, 1000, col.size).astype(np.float64)
    x = rng.integers(-1000, 1000, rows).astype(np.float64)
    want = _dense_int(rp, col, val, rows, rows) @ np.array([int(v) for v in x], object)
    assert np.array_equal(oracle.spmv_csr_f64d(rp, col, val, x), np.array(want, np.float64))
    # row 0 in index order: 2^53 + 1 ties to 2^53 (even), + 1 again, - 2^53 = 0; the reverse order
    # gives 2 and a pairwise tree 1. Row 2 is row 0 reversed; row 1 is empty.
    rp2 = np.array([0, 4, 4, 8], np.int32)
    col2 = np.array([0, 1, 2, 3, 3, 2, 1, 0], np.int32)
    val2 = np.array([2.0**53, 1.0, 1.0, -2.0**53, -2.0**53, 1.0, 1.0, 2.0**53])
    y = oracle.spmv_csr_f64d(rp2, col2, val2, np.ones(4))
    assert y.tolist() == [0.0, 0.0, 2.0]
    with pytest.raises(ValueError):
        oracle.spmv_csr_f64d(rp2, col2, val2, np.ones(4), cols=5)


def test_spmv_int_wraps_modulo_2_32():
    """SpMV<int>: unchecked C# arithmetic; the dense product in Python integers reduced mod 2^32."""
    rows = 150
    rp, col, _ = oracle.gen_zipf_csr(rows, 8, max_degree=rows - 1)
    val = oracle.gen_uniform_i32(col.size, 8, 1, -2_000_000_000, 2_000_000_000)
    x = oracle.gen_uniform_i32(rows, 9, 2, -70_000, 70_000)
    want = _dense_int(rp, col, val, rows, rows) @ np.array([int(v) for v in x], object)
    wrapped = np.array([((int(v) + 2**31) % 2**32) - 2**31 for v in want], np.int64).astype(np.int32)
    got = oracle.spmv_csr_i32(rp, col, val, x)
    assert np.array_equal(got, wrapped)
    assert any(abs(int(v)) >= 2**31 for v in want)  # the case does overflow
    assert got[np.diff(rp) == 0].tolist() == [0] * int(np.sum(np.diff(rp) == 0))


# ------------------------------------------------------------------ [Kernel] samples
# Each oracle restates a sample kernel body under the CPU invoker's flat-loop semantics; the pins
# below are closed forms computed independently (numpy float32 array arithmetic, Python integers).
def test_kernel_samples_elementwise_closed_forms():
    x = oracle.gen_uniform_f32(1000, 60, 0)
    y = oracle.gen_uniform_f32(1000, 60, 1)
    st, got = oracle.kernel_saxpy(x, y, 1.75)
    assert st == 0 and np.array_equal(got, np.float32(1.75) * x + y)  # two roundings, as numpy does
    st, _ = oracle.kernel_saxpy(x[:999], y, 1.75)
    assert st == 1  # x shorter than the work size: x[999] throws
    keys = np.arange(0, 5000, 7, dtype=np.uint32)
    st, h = oracle.kernel_hash_mix(keys, keys.size, 0x9E3779B9)

    def lowbias32(v):
        v ^= 0x9E3779B9
        v ^= v >> 16
        v = (v * 0x7FEB352D) & 0xFFFFFFFF
        v ^= v >> 15
        v = (v * 0x846CA68B) & 0xFFFFFFFF
        return v ^ (v >> 16)

    assert st == 0 and h.tolist() == [lowbias32(int(k)) for k in keys]
    src = oracle.gen_uniform_f32(64, 61, 0)
    idx = np.array([3, 0, 63, 17], np.int32)
    assert np.array_equal(oracle.kernel_gather(src, idx, 4)[1], src[idx])
    assert oracle.kernel_gather(src, np.array([3, 64], np.int32), 2)[0] == 1
    assert oracle.kernel_gather(src, np.array([-1], np.int32), 1)[0] == 1
    a = np.array([7, -7, 2**31 - 1, 5], np.int32)
    assert oracle.kernel_int_divide(a, np.array([2, 2, -1, 5], np.int32), 4)[1].tolist() == [3, -3, -(2**31 - 1), 1]
    assert oracle.kernel_int_divide(a, np.array([2, 0, 1, 1], np.int32), 4)[0] == 2
    assert oracle.kernel_int_divide(np.array([-(2**31)], np.int32), np.array([-1], np.int32), 1)[0] == 3


def test_kernel_samples_net_semantics():
    nan = float("nan")
    assert oracle.lib().oracle_net_maxf(-0.0, 0.0) == 0.0 and math.copysign(1, oracle.lib().oracle_net_maxf(-0.0, 0.0)) == 1
    assert math.copysign(1, oracle.lib().oracle_net_maxf(0.0, -0.0)) == 1
    assert math.copysign(1, oracle.lib().oracle_net_minf(0.0, -0.0)) == -1
    assert math.copysign(1, oracle.lib().oracle_net_minf(-0.0, 0.0)) == -1
    assert math.isnan(oracle.lib().oracle_net_maxf(nan, 1.0)) and math.isnan(oracle.lib().oracle_net_maxf(1.0, nan))
    assert math.isnan(oracle.lib().oracle_net_minf(nan, 1.0)) and math.isnan(oracle.lib().oracle_net_minf(1.0, nan))
    assert oracle.lib().oracle_net_minf(2.0, 3.0) == 2.0 and oracle.lib().oracle_net_maxf(2.0, 3.0) == 3.0
    f2l = oracle.lib().oracle_net_f2l
    assert f2l(nan) == 0 and f2l(1e30) == 2**63 - 1 and f2l(-1e30) == -(2**63) and f2l(-2.75) == -2
    assert f2l(2.0**63) == 2**63 - 1  # 2^63 is a float32 and saturates
    assert f2l(9.2233715e18) == 9223371487098961920  # the float32 just below 2^63 converts exactly
    # ScaleClamp against numpy where no signed zeros or NaNs occur (numpy's maximum differs there)
    x = oracle.gen_uniform_f32(5000, 62, 0)
    st, out = oracle.kernel_scale_clamp(x, x.size, 3.0, -1.5, 2.0)
    v = x * np.float32(3.0)
    ref = np.where(v > 0, np.minimum(v, np.float32(2.0)),
                   np.where(v < np.float32(-1.5), np.float32(-1.5), np.maximum(v, np.float32(-0.75))))
    assert st == 0 and np.array_equal(out, ref.astype(np.float32))
    # LongMix: shift masked to 6 bits, float -> long saturating, wrapping sum
    a = np.array([1, -3, 2**62, 5], np.int64)
    f = np.array([0.0, 1.0, 4.0, -0.25], np.float32)
    st, b = oracle.kernel_long_mix(a, f, 4, 65)  # shift 65 & 63 = 1
    prod = (f * np.float32(3.0e18))
    sat = [0, int(prod[1]), 2**63 - 1, int(prod[3])]
    want = [((int(a[i]) << 1) + sat[i] + i + 2**63) % 2**64 - 2**63 for i in range(4)]
    assert st == 0 and b.tolist() == want


def test_kernel_samples_grids_closed_forms():
    rows, cols = 37, 53
    inp = oracle.gen_uniform_f32(rows * cols, 63, 0)
    st, out = oracle.kernel_transpose(inp, rows * cols, rows, cols)
    assert st == 0 and np.array_equal(out, inp.reshape(rows, cols).T.ravel())
    m, k, n = 9, 13, 7
    a = oracle.gen_uniform_f32(m * k, 64, 0)
    b = oracle.gen_uniform_f32(k * n, 64, 1)
    st, c = oracle.kernel_matmul_naive(a, b, m * n, k, m, n)
    ref = np.zeros((m, n), np.float32)
    for i in range(m):  # in-order float32 accumulation, one rounding per multiply and per add
        for j in range(n):
            s = np.float32(0)
            for p in range(k):
                s = np.float32(s + np.float32(a[i * k + p] * b[p * n + j]))
            ref[i, j] = s
    assert st == 0 and np.array_equal(c, ref.ravel())
    assert np.allclose(c.reshape(m, n), a.reshape(m, k).astype(np.float64) @ b.reshape(k, n), rtol=1e-5, atol=1e-5)
    d, h, w = 5, 6, 7
    src = oracle.gen_uniform_f32(d * h * w, 65, 0)
    st, dst = oracle.kernel_stencil3d(src, d * h * w, d, h, w)
    s3 = src.reshape(d, h, w)
    left = np.zeros_like(s3)
    left[:, :, 1:] = s3[:, :, :-1]
    below = np.zeros_like(s3)
    below[1:] = s3[:-1]
    ref = s3 * np.float32(2) - left - np.float32(0.5) * below
    assert st == 0 and np.array_equal(dst, ref.ravel())
    assert oracle.kernel_transpose(inp, rows * cols, rows, 0)[0] == 2  # zero extent: __i % 0
