"""GPU parity: fused Where/Select -> ToArray (order-preserving compaction) and -> Sum.

The benchmark chain is src.AsComputeQueryable().Where(x => x > 0f).Select(x => x * 2f + 1f);
count, order and every output bit must equal LINQ-to-objects (the reference's fallback path,
ComputeQueryableExtensions.cs:628-633), which the oracle restates by hand. Random programs are
checked against the oracle's interpreter. Sums: rel 1e-5*log2(N) vs the float64 host sum.
"""
import math

import numpy as np
import pytest

import oracle
from dotcompute_amd import hip
from dotcompute_amd.hip import (ABS, ADD, CMP_AND, CMP_EQ, CMP_GE, CMP_GT, CMP_LE, CMP_LT, CMP_NE, CMP_OR, DIV,
                                FILTER, LOAD, MAP, MAX, MIN, MUL, NEG, PAND_Q, PNOT, POR_Q, PSTORE, RDIV, RSUB,
                                SQRT, SRC_ELEM, SRC_IMM, SRC_S0, SRC_S1, STORE_S0, STORE_S1, SUB, LinqChain)

pytestmark = pytest.mark.gpu

CHAIN = hip.where_gt0_select_2x_plus_1()


def ordered(chain):
    """A copy of `chain` that runs ToArray on the ticket-ordered lookback grid."""
    ch = type(chain).from_buffer_copy(chain)
    ch.flags |= hip.LINQ_FLAG_ORDERED_GRID
    return ch


def run_to_array(ctx, chain, x, offset=0):
    """ToArray on the kernel the library picks and on the lookback grid; both must agree bit for
    bit (the round-robin grid takes every 4-byte aligned input, so this keeps the lookback kernel
    under the same checks)."""
    n = x.size
    dx = ctx.empty(n + offset + 1, np.float32)
    if n:
        hip.check(hip.load().dc_hip_memcpy_h2d_async(ctx.handle, dx.ptr + 4 * offset, x.ctypes.data, x.nbytes), "h2d")
    src = hip.DeviceArray(ctx, dx.ptr + 4 * offset, 4 * n, np.dtype(np.float32), (n,))
    out = ctx.empty(n + 1, np.float32)
    cnt = ctx.empty(1, np.int64)
    res = []
    for ch in (chain, ordered(chain)):
        ctx.where_select_f32(ch, src, out, cnt, n)
        ctx.synchronize()
        k = int(cnt.to_host()[0])
        assert k >= 0, "resident grid reported a wait that gave up"
        res.append(out.to_host(k) if k else np.empty(0, np.float32))
    for a in (dx, out, cnt):
        ctx.free(a)
    assert res[0].size == res[1].size and np.array_equal(bits(res[0]), bits(res[1]))
    return res[0]


def run_sum(ctx, chain, x):
    n = x.size
    dx = ctx.to_device(x) if n else ctx.empty(1, np.float32)
    s = ctx.empty(1, np.float64)
    c = ctx.empty(1, np.int64)
    ctx.where_select_sum_f32(chain, dx, s, c, n)
    ctx.synchronize()
    res = (s.to_host()[0], int(c.to_host()[0]))
    for a in (dx, s, c):
        ctx.free(a)
    return res


def run_minmax(ctx, chain, x, op, offset=0):
    """Device Min/Max (op: hip.LINQ_MIN / LINQ_MAX) of the kept, mapped elements, with the input
    placed `offset` floats into its allocation. Returns (value as float32, count)."""
    n = x.size
    dx = ctx.empty(n + offset + 1, np.float32)
    if n:
        hip.check(hip.load().dc_hip_memcpy_h2d_async(ctx.handle, dx.ptr + 4 * offset, x.ctypes.data, x.nbytes), "h2d")
    src = hip.DeviceArray(ctx, dx.ptr + 4 * offset, 4 * n, np.dtype(np.float32), (n,))
    v = ctx.empty(1, np.float32)
    c = ctx.empty(1, np.int64)
    ctx.where_select_minmax_f32(chain, src, op, v, c, n)
    ctx.synchronize()
    res = (v.to_host()[0], int(c.to_host()[0]))
    for a in (dx, v, c):
        ctx.free(a)
    return res


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def same_floats(a, b) -> bool:
    """Bit-for-bit equality, except that any two NaNs match (x86 and CDNA produce different
    default NaN payloads; .NET exposes no payload semantics)."""
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    if a.shape != b.shape:
        return False
    nan = np.isnan(a)
    return bool(np.array_equal(nan, np.isnan(b)) and np.array_equal(bits(a[~nan]), bits(b[~nan])))


@pytest.mark.parametrize("n", [0, 1, 2, 63, 64, 4095, 4096, 4097, 12_289, 1_000_000, 16_000_000])
def test_where_select_to_array_bit_exact(ctx, n):
    x = oracle.gen_uniform_f32(n, 42 + 2, 0)
    got = run_to_array(ctx, CHAIN, x)
    ref = oracle.where_gt0_select_2x_plus_1(x)
    assert got.size == ref.size
    assert np.array_equal(bits(got), bits(ref))


def test_where_select_misaligned_input(ctx):
    x = oracle.gen_uniform_f32(10_000, 5, 0)
    got = run_to_array(ctx, CHAIN, x, offset=1)
    assert np.array_equal(bits(got), bits(oracle.where_gt0_select_2x_plus_1(x)))


def test_where_select_signed_zero_and_extremes(ctx):
    x = np.array([0.0, -0.0, 1e-45, -1e-45, 3.4e38, -3.4e38, np.inf, -np.inf, np.nan, 1.0, -1.0] * 500, np.float32)
    got = run_to_array(ctx, CHAIN, x)
    ref = oracle.where_gt0_select_2x_plus_1(x)
    assert np.array_equal(bits(got), bits(ref))  # +inf*2+1 = inf; 3.4e38*2 = inf


def test_reference_linq_golden_vectors(ctx):
    """Known answers of the reference LINQ tests, on the GPU."""
    def chain_gt_mul(t, m):
        return LinqChain.assemble([(LOAD, SRC_ELEM, 0), (CMP_GT, SRC_IMM, t), (FILTER, SRC_IMM, 0),
                                   (LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, m), (MAP, SRC_IMM, 0)])
    # ComputeQueryProviderTests.cs:341-365: {1..5}.Where(x > 3) -> {4, 5}
    w = LinqChain.assemble([(LOAD, SRC_ELEM, 0), (CMP_GT, SRC_IMM, 3), (FILTER, SRC_IMM, 0)])
    assert run_to_array(ctx, w, np.arange(1, 6, dtype=np.float32)).tolist() == [4, 5]
    # {1,2,3}.Select(x * 2) -> {2,4,6}
    s = LinqChain.assemble([(LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 2), (MAP, SRC_IMM, 0)])
    assert run_to_array(ctx, s, np.array([1, 2, 3], np.float32)).tolist() == [2, 4, 6]
    # LinqBackendIntegrationTests.cs:51-66: {1..5}.Where(x > 2).Select(x * 2) -> {6, 8, 10}
    assert run_to_array(ctx, chain_gt_mul(2, 2), np.arange(1, 6, dtype=np.float32)).tolist() == [6, 8, 10]
    # :139-161: {1..10}.Where(x > 3).Select(x * 3) -> {12, ..., 30}
    assert run_to_array(ctx, chain_gt_mul(3, 3), np.arange(1, 11, dtype=np.float32)).tolist() == list(range(12, 31, 3))
    # :309-325: 1..100 .Where(x % 2 == 0).Select(x * x): count 50, first 4, last 10000.
    # The op set has no remainder; for integer-valued x < 2^22, x is even exactly when rounding
    # x * 0.5 to an integer (adding and subtracting 2^23) and doubling gives x back.
    xs = np.arange(1, 101, dtype=np.float32)
    even = LinqChain.assemble([(LOAD, SRC_ELEM, 0), (STORE_S0, SRC_IMM, 0), (MUL, SRC_IMM, 0.5),
                               (ADD, SRC_IMM, 8388608.0), (SUB, SRC_IMM, 8388608.0), (MUL, SRC_IMM, 2.0),
                               (CMP_EQ, SRC_S0, 0), (FILTER, SRC_IMM, 0),
                               (LOAD, SRC_ELEM, 0), (MUL, SRC_ELEM, 0), (MAP, SRC_IMM, 0)])
    got = run_to_array(ctx, even, xs)
    assert got.size == 50 and got[0] == 4 and got[-1] == 10000
    assert np.array_equal(got, oracle.linq_where_select(even, xs))
    # Sum(1..1000) = 500500 through the fused Sum kernel with an empty chain
    empty = LinqChain.assemble([])
    ssum, cnt = run_sum(ctx, empty, np.arange(1, 1001, dtype=np.float32))
    assert ssum == 500500.0 and cnt == 1000


@pytest.mark.parametrize("n", [0, 1, 1000, 1_000_000, 16_000_000])
def test_where_select_sum(ctx, n):
    x = oracle.gen_uniform_f32(n, 44, 0)
    got, cnt = run_sum(ctx, CHAIN, x)
    f32_ref, seq_double, ref_cnt = oracle.where_gt0_select_2x_plus_1_sum(x)
    assert cnt == ref_cnt
    tol = 1e-5 * max(1.0, math.log2(max(n, 2)))
    assert abs(got - seq_double) <= tol * max(abs(seq_double), 1e-30) + 1e-12


def _random_program(rng):
    """A random but well-formed program: 1-3 stages, each a filter or a map."""
    code = []
    uses_saves = bool(rng.integers(0, 2))
    for _ in range(int(rng.integers(1, 4))):
        if rng.integers(0, 2):  # filter
            code.append((LOAD, SRC_ELEM, 0))
            code.append((int(rng.choice([CMP_GT, CMP_GE, CMP_LT, CMP_LE, CMP_NE])), SRC_IMM,
                         float(rng.uniform(-1, 1)), 0))
            if rng.integers(0, 2):
                code.append((PSTORE, SRC_IMM, 0))
                code.append((LOAD, SRC_ELEM, 0))
                code.append((ABS, SRC_IMM, 0))
                code.append((CMP_LT, SRC_IMM, float(rng.uniform(0.2, 1.0)), int(rng.choice([CMP_AND, CMP_OR]))))
                code.append((int(rng.choice([PAND_Q, POR_Q])), SRC_IMM, 0))
            if rng.integers(0, 4) == 0:
                code.append((PNOT, SRC_IMM, 0))
            code.append((FILTER, SRC_IMM, 0))
        else:  # map
            code.append((LOAD, SRC_ELEM, 0))
            for _ in range(int(rng.integers(1, 5))):
                op = int(rng.choice([ADD, SUB, RSUB, MUL, DIV, RDIV, MIN, MAX, NEG, ABS, SQRT]))
                src = SRC_IMM
                if uses_saves and rng.integers(0, 3) == 0:
                    code.append((STORE_S0, SRC_IMM, 0))
                    src = SRC_S0
                elif rng.integers(0, 4) == 0:
                    src = SRC_ELEM
                code.append((op, src, float(rng.uniform(-2, 2))))
            if uses_saves:
                code.append((STORE_S1, SRC_IMM, 0))
                code.append((ADD, SRC_S1, 0))
            code.append((MAP, SRC_IMM, 0))
    return LinqChain.assemble(code)


@pytest.mark.parametrize("seed", range(12))
def test_random_programs_match_interpreter(ctx, seed):
    rng = np.random.default_rng(seed)
    prog = _random_program(rng)
    assert hip.load().dc_linq_chain_validate(prog) == 0
    x = oracle.gen_uniform_f32(50_000 + seed * 977, 100 + seed, 0)
    got = run_to_array(ctx, prog, x)
    ref = oracle.linq_where_select(prog, x)
    assert got.size == ref.size
    assert same_floats(got, ref)
    s, c = run_sum(ctx, prog, x)
    _, sd, rc = oracle.linq_where_select_sum(prog, x)
    assert c == rc
    if np.isfinite(sd):
        assert abs(s - sd) <= 1e-5 * math.log2(x.size) * max(abs(sd), 1.0)


def test_invalid_program_rejected(ctx):
    bad = LinqChain.assemble([(99, SRC_IMM, 0)])
    x = ctx.empty(16, np.float32)
    out = ctx.empty(16, np.float32)
    cnt = ctx.empty(1, np.int64)
    with pytest.raises(hip.HipError) as e:
        ctx.where_select_f32(bad, x, out, cnt, 16)
    assert e.value.status == hip.DC_ERR_UNSUPPORTED
    for a in (x, out, cnt):
        ctx.free(a)


@pytest.mark.slow
def test_where_select_256m(ctx):
    n = 256 * 1024 * 1024
    dx = ctx.empty(n, np.float32)
    ctx.fill_uniform_f32(dx, seed=44, stream=0)
    out = ctx.empty(n, np.float32)
    cnt = ctx.empty(1, np.int64)
    ctx.where_select_f32(CHAIN, dx, out, cnt)
    ctx.synchronize()
    k = int(cnt.to_host()[0])
    x = oracle.gen_uniform_f32(n, 44, 0)
    ref = oracle.where_gt0_select_2x_plus_1(x)
    del x
    assert k == ref.size
    assert np.array_equal(bits(out.to_host(k)), bits(ref))
    s = ctx.empty(1, np.float64)
    c = ctx.empty(1, np.int64)
    ctx.where_select_sum_f32(CHAIN, dx, s, c)
    ctx.synchronize()
    assert int(c.to_host()[0]) == k
    ref_sum = float(np.sum(ref, dtype=np.float64))
    assert abs(s.to_host()[0] - ref_sum) <= 1e-5 * 28 * abs(ref_sum)
    # Min / Max of the same chain over the full input: the first smallest / largest kept element
    v = ctx.empty(1, np.float32)
    for op, ref_v in ((hip.LINQ_MIN, ref.min()), (hip.LINQ_MAX, ref.max())):
        ctx.where_select_minmax_f32(CHAIN, dx, op, v, c)
        ctx.synchronize()
        assert int(c.to_host()[0]) == k
        assert bits(v.to_host()) == bits(np.array([ref_v], np.float32))
    for a in (dx, out, cnt, s, c, v):
        ctx.free(a)


AFFINE_CHAINS = [
    # (description, program) — all lowered to the affine fast path
    ("Where(x >= 0.25)", [(LOAD, SRC_ELEM, 0), (CMP_GE, SRC_IMM, 0.25), (FILTER, SRC_IMM, 0)]),
    ("Select(x * 3)", [(LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 3.0), (MAP, SRC_IMM, 0)]),
    ("Select(x - 0.1)", [(LOAD, SRC_ELEM, 0), (SUB, SRC_IMM, 0.1), (MAP, SRC_IMM, 0)]),
    ("Where(x < 0).Select(x * -0.5 + 2).Where(x != 2.25)",
     [(LOAD, SRC_ELEM, 0), (CMP_LT, SRC_IMM, 0.0), (FILTER, SRC_IMM, 0),
      (LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, -0.5), (ADD, SRC_IMM, 2.0), (MAP, SRC_IMM, 0),
      (LOAD, SRC_ELEM, 0), (CMP_NE, SRC_IMM, 2.25), (FILTER, SRC_IMM, 0)]),
    ("Select(x * 1.1).Where(x <= 0.3).Select(x + 7)",
     [(LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 1.1), (MAP, SRC_IMM, 0),
      (LOAD, SRC_ELEM, 0), (CMP_LE, SRC_IMM, 0.3), (FILTER, SRC_IMM, 0),
      (LOAD, SRC_ELEM, 0), (ADD, SRC_IMM, 7.0), (MAP, SRC_IMM, 0)]),
    ("Where(x == 0)", [(LOAD, SRC_ELEM, 0), (CMP_EQ, SRC_IMM, 0.0), (FILTER, SRC_IMM, 0)]),
]


@pytest.mark.parametrize("idx", range(len(AFFINE_CHAINS)))
def test_affine_fast_path_matches_interpreter(ctx, idx):
    _, code = AFFINE_CHAINS[idx]
    prog = LinqChain.assemble(code)
    x = oracle.gen_uniform_f32(300_001, 77 + idx, 0)
    got = run_to_array(ctx, prog, x)
    assert same_floats(got, oracle.linq_where_select(prog, x))
    s, c = run_sum(ctx, prog, x)
    _, sd, rc = oracle.linq_where_select_sum(prog, x)
    assert c == rc
    assert abs(s - sd) <= 1e-5 * math.log2(x.size) * max(abs(sd), 1.0)


# ---- the round-robin kernel (every 4-byte aligned input) ----------------------------------------
# Tiles of 8 worker waves x 64 lanes x 16 elements; rr_min_n() = 4 full rounds of min(CUs, 256)
# tiles, the shape the software pipeline is built for.
RR_TILE = 8 * 64 * 16


def rr_min_n():
    return 4 * min(hip.device_info(0).compute_units, 256) * RR_TILE


def run_to_array_checked(ctx, chain, x, strategy, offset=0):
    """run_to_array, asserting which kernel the library picks for this input."""
    n = x.size
    dx = ctx.empty(n + offset + 1, np.float32)
    hip.check(hip.load().dc_hip_memcpy_h2d_async(ctx.handle, dx.ptr + 4 * offset, x.ctypes.data, x.nbytes), "h2d")
    src = hip.DeviceArray(ctx, dx.ptr + 4 * offset, 4 * n, np.dtype(np.float32), (n,))
    assert ctx.to_array_strategy(src, n) == strategy
    out = ctx.empty(n + 1, np.float32)
    cnt = ctx.empty(1, np.int64)
    ctx.where_select_f32(chain, src, out, cnt, n)
    ctx.synchronize()
    k = int(cnt.to_host()[0])
    assert k >= 0, "resident grid reported a wait that gave up"
    got = out.to_host(k) if k else np.empty(0, np.float32)
    for a in (dx, out, cnt):
        ctx.free(a)
    return got


@pytest.mark.parametrize("extra", [0, 1, 4097, RR_TILE * 3 + 5, 256 * RR_TILE - 1, 256 * RR_TILE * 2 + 12345])
def test_round_robin_sizes_bit_exact(ctx, extra):
    n = rr_min_n() + extra
    x = oracle.gen_uniform_f32(n, 500 + extra % 97, 0)
    got = run_to_array_checked(ctx, CHAIN, x, hip.STRATEGY_ROUNDS)
    ref = oracle.where_gt0_select_2x_plus_1(x)
    assert got.size == ref.size
    assert np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize("n", [1, 3, 100, RR_TILE - 1, RR_TILE, 2 * RR_TILE, 2 * RR_TILE + 1, 1 << 20, 1_000_000,
                               3_000_000])
def test_round_robin_small_inputs(ctx, n):
    """Every 4-byte aligned input runs the round-robin grid: below one workgroup per CU each
    workgroup owns one tile (the only round runs as the tail round), one full round plus a tail
    round (3M), and starts 1-3 floats past a 16-byte boundary; bit-exact, and equal to the lookback
    kernel's result."""
    x = oracle.gen_uniform_f32(n + 3, 70 + n % 13, 0)
    for offset in (0, 1, 3):
        got = run_to_array_checked(ctx, CHAIN, x[:n], hip.STRATEGY_ROUNDS, offset=offset)
        assert np.array_equal(bits(got), bits(oracle.where_gt0_select_2x_plus_1(x[:n])))
        assert np.array_equal(bits(got), bits(run_to_array(ctx, CHAIN, x[:n], offset=offset)))


def test_round_robin_threshold_and_alignment(ctx):
    n = rr_min_n()
    x = oracle.gen_uniform_f32(n + 3, 61, 0)
    # one element short of four rounds: three full rounds and a tail round, same result
    got = run_to_array_checked(ctx, CHAIN, x[: n - 1], hip.STRATEGY_ROUNDS)
    assert np.array_equal(bits(got), bits(oracle.where_gt0_select_2x_plus_1(x[: n - 1])))
    # a start 1-3 floats past a 16-byte boundary: the round-robin grid peels the 3-1 head elements
    for offset in (1, 2, 3):
        got = run_to_array_checked(ctx, CHAIN, x, hip.STRATEGY_ROUNDS, offset=offset)
        assert np.array_equal(bits(got), bits(oracle.where_gt0_select_2x_plus_1(x)))
    # a start that is not 4-byte aligned: the lookback kernel
    raw = ctx.empty(n + 2, np.float32)
    odd = hip.DeviceArray(ctx, raw.ptr + 2, 4 * n, np.dtype(np.float32), (n,))
    assert ctx.to_array_strategy(odd, n) == hip.STRATEGY_LOOKBACK
    ctx.free(raw)


@pytest.mark.parametrize("offset", [1, 2, 3])
@pytest.mark.parametrize("head", ["kept", "dropped", "mixed"])
def test_round_robin_peeled_head_every_program_kind(ctx, offset, head):
    # the head elements decide the offset of everything after them: kept, dropped or mixed heads,
    # on the canonical, affine and interpreter variants
    x = oracle.gen_uniform_f32(rr_min_n() + 5, 62 + offset, 0)
    x[:3] = {"kept": [0.5, 0.25, 0.75], "dropped": [-0.5, -0.25, -0.75], "mixed": [-0.5, 0.25, -0.75]}[head]
    progs = [CHAIN,
             LinqChain.assemble([(LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 3.0), (ADD, SRC_IMM, -0.5), (MAP, SRC_IMM, 0),
                                 (LOAD, SRC_ELEM, 0), (CMP_GT, SRC_IMM, 0.0), (FILTER, SRC_IMM, 0),
                                 (LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 0.5), (MAP, SRC_IMM, 0)]),
             LinqChain.assemble([(LOAD, SRC_ELEM, 0), (ABS, SRC_IMM, 0), (CMP_LT, SRC_IMM, 0.6), (FILTER, SRC_IMM, 0),
                                 (LOAD, SRC_ELEM, 0), (SQRT, SRC_IMM, 0), (MAP, SRC_IMM, 0)])]
    for prog in progs:
        got = run_to_array_checked(ctx, prog, x, hip.STRATEGY_ROUNDS, offset=offset)
        assert same_floats(got, oracle.linq_where_select(prog, x))


@pytest.mark.parametrize("cmp,imm", [(CMP_GT, -2.0), (CMP_GT, 2.0), (CMP_LT, -0.999)])
def test_round_robin_all_none_and_sparse(ctx, cmp, imm):
    # every element kept (the staging ring at 100% selectivity), none kept, and ~0.05% kept
    prog = LinqChain.assemble([(LOAD, SRC_ELEM, 0), (cmp, SRC_IMM, imm), (FILTER, SRC_IMM, 0),
                               (LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 3.0), (MAP, SRC_IMM, 0)])
    x = oracle.gen_uniform_f32(rr_min_n() + 999, 71, 0)
    got = run_to_array_checked(ctx, prog, x, hip.STRATEGY_ROUNDS)
    assert same_floats(got, oracle.linq_where_select(prog, x))


@pytest.mark.parametrize("seed", range(4))
def test_round_robin_random_programs(ctx, seed):
    # interpreter variants (with and without save registers) on the resident grid
    rng = np.random.default_rng(1000 + seed)
    prog = _random_program(rng)
    x = oracle.gen_uniform_f32(rr_min_n() + 777 * seed, 300 + seed, 0)
    got = run_to_array_checked(ctx, prog, x, hip.STRATEGY_ROUNDS)
    assert same_floats(got, oracle.linq_where_select(prog, x))


def _salted_input(n, seed):
    """Uniform input with signed zeros, infinities, NaN, denormals and exact thresholds mixed in."""
    x = oracle.gen_uniform_f32(n, seed, 0).copy()
    rng = np.random.default_rng(seed)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 1.17e-38, 0.25, -0.25, 0.5],
                        dtype=np.float32)
    idx = rng.choice(n, size=n // 50, replace=False)
    x[idx] = specials[rng.integers(0, specials.size, size=idx.size)]
    return x


SHAPE_PROGRAMS = {
    "F": lambda cmp, t: [(LOAD, SRC_ELEM, 0), (cmp, SRC_IMM, t), (FILTER, SRC_IMM, 0)],
    "M": lambda cmp, t: [(LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, -3.0), (ADD, SRC_IMM, 0.5), (MAP, SRC_IMM, 0)],
    "FM": lambda cmp, t: [(LOAD, SRC_ELEM, 0), (cmp, SRC_IMM, t), (FILTER, SRC_IMM, 0),
                          (LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 2.0), (ADD, SRC_IMM, 1.0), (MAP, SRC_IMM, 0)],
    "MF": lambda cmp, t: [(LOAD, SRC_ELEM, 0), (ADD, SRC_IMM, -0.25), (MAP, SRC_IMM, 0),
                          (LOAD, SRC_ELEM, 0), (cmp, SRC_IMM, t), (FILTER, SRC_IMM, 0)],
    "Fmul": lambda cmp, t: [(LOAD, SRC_ELEM, 0), (cmp, SRC_IMM, t), (FILTER, SRC_IMM, 0),
                            (LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 0.1), (MAP, SRC_IMM, 0)],
}


@pytest.mark.parametrize("shape", sorted(SHAPE_PROGRAMS))
@pytest.mark.parametrize("cmp", [CMP_GT, CMP_GE, CMP_LT, CMP_LE, CMP_EQ, CMP_NE])
def test_round_robin_canonical_shapes_special_values(ctx, shape, cmp):
    # one- and two-stage affine chains take a branch-free form of the comparison on the resident
    # grid; it must equal the direct comparison for every input, including -0, +-inf, NaN and
    # denormals, and for thresholds 0 (signed zeros) and values present in the input
    for t in (0.0, 0.25):
        if shape == "M" and t != 0.0:
            continue
        prog = LinqChain.assemble(SHAPE_PROGRAMS[shape](cmp, t))
        x = _salted_input(rr_min_n() + 1234, 900 + cmp)
        got = run_to_array_checked(ctx, prog, x, hip.STRATEGY_ROUNDS)
        assert same_floats(got, oracle.linq_where_select(prog, x)), (shape, cmp, t)


def test_round_robin_two_contexts_interleaved(ctx):
    # two contexts on one device each queue resident grids without host synchronisation between
    # them; the library orders resident grids device-wide, so both finish with exact results
    n = rr_min_n() + 333
    xs = [oracle.gen_uniform_f32(n, 610 + i, 0) for i in range(2)]
    ctxs = [ctx, hip.Context(0)]
    bufs = []
    for c, x in zip(ctxs, xs):
        dx = c.to_device(x)
        assert c.to_array_strategy(dx, n) == hip.STRATEGY_ROUNDS
        bufs.append((dx, c.empty(n, np.float32), c.empty(1, np.int64)))
    for _ in range(3):
        for c, (dx, out, cnt) in zip(ctxs, bufs):
            c.where_select_f32(CHAIN, dx, out, cnt, n)
    for c in ctxs:
        c.synchronize()
    for c, x, (dx, out, cnt) in zip(ctxs, xs, bufs):
        k = int(cnt.to_host()[0])
        ref = oracle.where_gt0_select_2x_plus_1(x)
        assert k == ref.size
        assert np.array_equal(bits(out.to_host(k)), bits(ref))
        for a in (dx, out, cnt):
            c.free(a)
    ctxs[1].close()


# ---- Where/Select -> Min / Max: bit-identical to Enumerable.Min/Max (oracle restatement) ----------
MINMAX = [("min", hip.LINQ_MIN), ("max", hip.LINQ_MAX)]
EMPTY = LinqChain.assemble([])


@pytest.mark.parametrize("n", [1, 2, 63, 64, 1000, 4095, 4097, 100_000, 1_000_000, 16_000_000])
@pytest.mark.parametrize("which", MINMAX)
def test_min_max_benchmark_chain(ctx, n, which):
    name, op = which
    x = oracle.gen_uniform_f32(n, 44, 0)
    got, cnt = run_minmax(ctx, CHAIN, x, op)
    ref, rcnt = oracle.linq_where_select_minmax(CHAIN, x, name)
    assert cnt == rcnt
    if rcnt:
        assert bits(got) == bits(ref)


@pytest.mark.parametrize("offset", [1, 2, 3])
@pytest.mark.parametrize("which", MINMAX)
def test_min_max_misaligned_and_golden(ctx, offset, which):
    name, op = which
    x = oracle.gen_uniform_f32(300_007, 5, 0)
    got, cnt = run_minmax(ctx, CHAIN, x, op, offset)
    ref, rcnt = oracle.linq_where_select_minmax(CHAIN, x, name)
    assert cnt == rcnt and bits(got) == bits(ref)
    r100 = np.arange(1, 101, dtype=np.float32)
    assert run_minmax(ctx, EMPTY, r100, op, offset) == ((1.0 if name == "min" else 100.0), 100)
    assert run_minmax(ctx, EMPTY, np.array([5, 2, 8, 1], np.float32), op)[0] == (1.0 if name == "min" else 8.0)


@pytest.mark.parametrize("which", MINMAX)
def test_min_max_empty_sequences(ctx, which):
    _, op = which
    assert run_minmax(ctx, EMPTY, np.empty(0, np.float32), op)[1] == 0
    none = LinqChain.assemble([(LOAD, SRC_ELEM, 0), (CMP_GT, SRC_IMM, 5.0), (FILTER, SRC_IMM, 0)])
    assert run_minmax(ctx, none, oracle.gen_uniform_f32(200_000, 3, 0), op)[1] == 0


@pytest.mark.parametrize("n", [1000, 70_001, 2_000_000])
@pytest.mark.parametrize("which", MINMAX)
def test_min_max_ties_and_nans_pick_the_enumerator_element(ctx, n, which):
    """Many equal minima/maxima of both zero signs, and NaNs with distinct payloads at random
    places: the element chosen (its bits) must be the one the sequential enumerator returns."""
    name, op = which
    rng = np.random.default_rng(n)
    signed_zeros = rng.choice(np.array([0x00000000, 0x80000000, 0x3F800000, 0xBF800000], np.uint32), n)
    x = signed_zeros.view(np.float32)
    for chain in (EMPTY, LinqChain.assemble([(LOAD, SRC_ELEM, 0), (CMP_NE, SRC_IMM, 1.0), (FILTER, SRC_IMM, 0)])):
        got, cnt = run_minmax(ctx, chain, x, op)
        ref, rcnt = oracle.linq_where_select_minmax(chain, x, name)
        assert cnt == rcnt and bits(got) == bits(ref)
    y = oracle.gen_uniform_f32(n, 9, 0).copy()
    pos = rng.choice(n, 5, replace=False)
    y.view(np.uint32)[pos] = 0x7FC00000 + np.arange(1, 6, dtype=np.uint32)  # quiet NaNs, distinct payloads
    all_nan = (0x7FC00000 + np.arange(1, n + 1, dtype=np.uint32) % 1000).view(np.float32)
    # the identity chain runs the general affine kernel, Select(x * 2) a canonical map kernel
    # (x * 2 + -0 keeps both zero signs and every NaN payload)
    for chain in (EMPTY, LinqChain.assemble([(LOAD, SRC_ELEM, 0), (MUL, SRC_IMM, 2.0), (MAP, SRC_IMM, 0)])):
        for data in (x, y, all_nan):
            got, cnt = run_minmax(ctx, chain, data, op)
            ref, rcnt = oracle.linq_where_select_minmax(chain, data, name)
            assert cnt == rcnt and bits(got) == bits(ref)


@pytest.mark.parametrize("seed", range(8))
def test_min_max_random_programs(ctx, seed):
    rng = np.random.default_rng(500 + seed)
    prog = _random_program(rng)
    x = oracle.gen_uniform_f32(80_000 + 313 * seed, 200 + seed, 0)
    for name, op in MINMAX:
        got, cnt = run_minmax(ctx, prog, x, op)
        ref, rcnt = oracle.linq_where_select_minmax(prog, x, name)
        assert cnt == rcnt
        if rcnt:
            assert same_floats(np.array([got]), np.array([ref]))


REDUCE_CANON = [(shape, cmp) for shape in sorted(SHAPE_PROGRAMS)
                for cmp in ([CMP_GT] if shape == "M" else [CMP_GT, CMP_GE, CMP_LT, CMP_LE, CMP_EQ, CMP_NE])]


@pytest.mark.parametrize("shape,cmp", REDUCE_CANON)
def test_reductions_canonical_chains_special_values(ctx, shape, cmp):
    """Sum / Count / Min / Max of the one- and two-stage affine chains, which run a kernel per
    shape and comparison, on inputs salted with -0, +-inf, NaN, denormals and exact thresholds,
    aligned and misaligned: counts and Min/Max bits equal the enumerator's."""
    for t in (0.0, 0.25):
        prog = LinqChain.assemble(SHAPE_PROGRAMS[shape](cmp, t))
        x = _salted_input(200_003, 40 + cmp)
        for offset in (0, 3):
            for name, op in MINMAX:
                got, cnt = run_minmax(ctx, prog, x, op, offset)
                ref, rcnt = oracle.linq_where_select_minmax(prog, x, name)
                assert cnt == rcnt, (shape, cmp, t, offset, name)
                if rcnt:
                    assert bits(got) == bits(ref), (shape, cmp, t, offset, name)
        s, c = run_sum(ctx, prog, x)
        _, sd, rc = oracle.linq_where_select_sum(prog, x)
        assert c == rc
        if np.isfinite(sd):
            assert abs(s - sd) <= 1e-5 * math.log2(x.size) * max(abs(sd), 1.0)
        else:
            assert (math.isnan(s) and math.isnan(sd)) or s == sd


FOLDS = [("min", hip.LINQ_FOLD_MIN), ("max", hip.LINQ_FOLD_MAX)]


@pytest.mark.parametrize("n", [0, 1, 1000, 70_001, 1_000_000, 16_000_000])
@pytest.mark.parametrize("which", FOLDS)
def test_fold_min_max_match_sequential_fold(ctx, n, which):
    """Aggregate((acc, x) => MathF.Min(acc, x)) / MathF.Max against the oracle's in-order fold: the
    value bit for bit (any NaN for NaN), the kept count exactly; with and without NaNs, with both
    zero signs as the extreme, on aligned and misaligned inputs."""
    name, op = which
    rng = np.random.default_rng(n + op)
    zeros = rng.choice(np.array([0x00000000, 0x80000000, 0x3F800000, 0x40000000], np.uint32), n).view(np.float32)
    salted = _salted_input(max(n, 1), 300 + op)[:n]
    plain = oracle.gen_uniform_f32(n, 301, 0)
    chains = (EMPTY, CHAIN, LinqChain.assemble([(LOAD, SRC_ELEM, 0), (CMP_NE, SRC_IMM, 2.0), (FILTER, SRC_IMM, 0)]))
    for data in (zeros, salted, plain):
        for chain in chains:
            for offset in ((0, 3) if n and n <= 1_000_000 else (0,)):
                got, cnt = run_minmax(ctx, chain, data, op, offset=offset)
                ref, rcnt = oracle.linq_where_select_fold(chain, data, name)
                assert cnt == rcnt
                if rcnt:
                    assert same_floats(np.array([got]), np.array([ref])), (name, chain.n_instr, offset, got, ref)


@pytest.mark.parametrize("seed", range(6))
def test_fold_random_programs(ctx, seed):
    """Random programs (the interpreter with and without save registers) and one with MathF.Pow
    (the library variant, Where(x < 0.5f).Select(x => -MathF.Pow(x, 3f))): the folds match the
    oracle's in-order fold, bit for bit; with Pow within 2 ulp (the two libraries' powf)."""
    rng = np.random.default_rng(900 + seed)
    prog = _random_program(rng)
    x = _salted_input(90_000 + 419 * seed, 400 + seed)
    if seed == 5:
        prog = LinqChain.assemble([(LOAD, SRC_ELEM, 0), (CMP_LT, SRC_IMM, 0.5), (FILTER, SRC_IMM, 0),
                                   (LOAD, SRC_ELEM, 0), (hip.POW, SRC_IMM, 3.0), (NEG, SRC_IMM, 0), (MAP, SRC_IMM, 0)])
    for name, op in FOLDS:
        got, cnt = run_minmax(ctx, prog, x, op)
        ref, rcnt = oracle.linq_where_select_fold(prog, x, name)
        assert cnt == rcnt
        if rcnt and seed == 5 and np.isfinite(ref) and ref != 0:
            g, r = np.array([got], np.float32).view(np.int32)[0], np.array([ref], np.float32).view(np.int32)[0]
            assert np.sign(got) == np.sign(ref) and abs(int(g) - int(r)) <= 2, (got, ref)
        elif rcnt:
            assert same_floats(np.array([got]), np.array([ref]))
