"""Writes tests/golden/*.json: small golden vectors for the hot path, computed WITHOUT the C oracle.

Inputs come from a pure-Python SplitMix64 (the published algorithm), expected outputs from NumPy
(float32 elementwise arithmetic, float64 matmul / dense SpMV, math.fsum for exact sums), plus the
known answers the reference's own tests assert. tests/test_oracle.py checks the C oracle against
these files, so an error in the oracle shows up as a mismatch with an independent computation.

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
M64 = (1 << 64) - 1


def splitmix64(z: int) -> int:
    z = (z + 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def gen_f32(n: int, seed: int, stream: int, unit: bool = False) -> np.ndarray:
    out = np.empty(n, np.float32)
    for i in range(n):
        r = splitmix64(seed ^ (stream << 40) ^ i)
        u = np.float32(r >> 40)
        out[i] = u * np.float32(2.0 ** -24) if unit else u * np.float32(2.0 ** -23) - np.float32(1.0)
    return out


def gen_i32(n: int, seed: int, stream: int, lo: int, hi: int) -> np.ndarray:
    span = hi - lo + 1
    return np.array([lo + (((splitmix64(seed ^ (stream << 40) ^ i) >> 32) * span) >> 32) for i in range(n)], np.int32)


def f32_bits(a) -> list[int]:
    return np.ascontiguousarray(a, np.float32).view(np.uint32).tolist()


def main() -> None:
    # SplitMix64 stream from state 0 (the generator's published first outputs).
    state, seq = 0, []
    for _ in range(3):
        seq.append(splitmix64(state))
        state = (state + 0x9E3779B97F4A7C15) & M64
    g = {"splitmix64_from_zero": [hex(v) for v in seq]}

    n = 4096
    a = gen_f32(n, 42, 0)
    b = gen_f32(n, 42, 1)
    g["inputs"] = {"f32_seed42_stream0_bits": f32_bits(a), "f32_seed42_stream1_bits": f32_bits(b),
                   "i32_seed43_stream1": gen_i32(n, 43, 1, -1000, 1000).tolist(),
                   "f32_unit_seed42_stream5_bits": f32_bits(gen_f32(64, 42, 5, True))}
    g["vector_add_bits"] = f32_bits(a + b)
    mask = a > np.float32(0.0)
    g["where_gt0_select_2x_plus_1_bits"] = f32_bits((a[mask] * np.float32(2.0)) + np.float32(1.0))
    g["where_gt0_select_2x_plus_1_sum_exact"] = math.fsum(float(v) for v in (a[mask] * np.float32(2.0)) + np.float32(1.0))
    g["sum_f32_exact"] = math.fsum(float(v) for v in a)
    g["sum_i32_exact"] = int(sum(int(v) for v in g["inputs"]["i32_seed43_stream1"]))

    m, k, nn = 16, 24, 8
    A = a[: m * k].reshape(m, k)
    B = b[: k * nn].reshape(k, nn)
    g["gemm_16x24x8_f64"] = (A.astype(np.float64) @ B.astype(np.float64)).ravel().tolist()

    # A 6-row CSR matrix and its dense product.
    rp = [0, 2, 2, 5, 6, 9, 10]
    col = [1, 4, 0, 3, 5, 2, 0, 1, 5, 3]
    val = [0.5, 0.5, 1 / 3, 1 / 3, 1 / 3, 1.0, 1 / 3, 1 / 3, 1 / 3, 1.0]
    x = [0.25, 0.5, 0.125, 1.0, 0.75, 0.0625]
    dense = np.zeros((6, 6))
    for r in range(6):
        for i in range(rp[r], rp[r + 1]):
            dense[r, col[i]] += np.float32(val[i])
    g["csr_6x6"] = {"row_pointers": rp, "col_indices": col, "values_f32_bits": f32_bits(np.array(val, np.float32)),
                    "x": x, "y_f64": (dense @ np.array(x, np.float32).astype(np.float64)).tolist()}

    # Known answers asserted by the reference's tests.
    g["reference_known_answers"] = {
        "ComputeQueryProviderTests.cs:341-365 Where(x>3) over 1..5": [4, 5],
        "ComputeQueryProviderTests.cs:341-365 Select(x*2) over 1,2,3": [2, 4, 6],
        "ComputeQueryProviderTests.cs:602-612 Sum 1..5": 15,
        "LinqBackendIntegrationTests.cs:51-66 Where(x>2).Select(x*2) over 1..5": [6, 8, 10],
        "LinqBackendIntegrationTests.cs:139-161 Where(x>3).Select(x*3) over 1..10": [12, 15, 18, 21, 24, 27, 30],
        "LinqBackendIntegrationTests.cs:164-176 Sum 1..1000": 500500,
        "LinqBackendIntegrationTests.cs:309-325 Where(x%2==0).Select(x*x) over 1..100": {"count": 50, "first": 4,
                                                                                         "last": 10000},
        "README.md:46-57 VectorAdd": {"a": [1, 2, 3, 4, 5], "b": [10, 20, 30, 40, 50], "result": [11, 22, 33, 44, 55]},
        "FutureExpansionTests.cs:553-570 Sum/Count/Max over Range(1,100)": {"sum": 5050, "count": 100, "max": 100},
        # ExpressionTreeVisitorTests.cs:113-147 asserts that Min()/Max() over {5,2,8,1} become Reduce
        # operations; the values are those of Enumerable.Min/Max over the same input.
        "ExpressionTreeVisitorTests.cs:113-147 Min/Max over 5,2,8,1": {"input": [5, 2, 8, 1], "min": 1, "max": 8},
    }
    with open(os.path.join(HERE, "hot_path_golden.json"), "w") as f:
        json.dump(g, f, indent=None, separators=(",", ":"))
    print("wrote", os.path.join(HERE, "hot_path_golden.json"))


if __name__ == "__main__":
    main()
