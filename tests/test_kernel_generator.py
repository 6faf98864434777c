"""CPU tests of the [Kernel] -> HIP generator (dotcompute_amd/generator): what it registers for
each sample kernel, the C# semantics it writes into the HIP source (promotions, literal types,
masked shifts, saturating casts, bounds-checked spans, per-buffer lengths) and what it refuses.
Mirrors the reference's generator tests (tests/Unit/DotCompute.Generators.Tests/Generator/
KernelExecutionMetadataTests.cs: a 2-D transpose kernel, an elementwise add bounded by .Length)
on this build's own kernels."""
import os
import subprocess

import pytest

from dotcompute_amd.generator import csharp as cs
from dotcompute_amd.generator import find_kernels, generate, translate

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KERNELS = os.path.join(ROOT, "dotcompute_amd", "kernels")


def one(src: str):
    ks = find_kernels(src)
    assert len(ks) == 1
    return translate(ks[0], ks[0].name)


def kernel(body: str, params: str = "ReadOnlySpan<float> a, Span<float> b", attr: str = "[Kernel]") -> dict:
    return one(f"namespace T {{ public static class K {{ {attr} public static void F({params}) {{ {body} }} }} }}")


def test_corpus_registers_every_kernel(tmp_path):
    recs = generate(sorted(os.path.join(KERNELS, f) for f in os.listdir(KERNELS) if f.endswith(".cs")),
                    str(tmp_path), root=ROOT)
    by = {r["km"].name: r for r in recs}
    assert set(by) == {"VectorAdd", "Saxpy", "ScaleClamp", "HashMix", "LongMix", "CopyPositive", "Gather", "IntDivide",
                       "Softplus", "Transpose", "MatMulNaive", "Stencil3D"}
    assert by["VectorAdd"]["km"].full_name == "Kernels.VectorAdd" and by["VectorAdd"]["km"].backends == ["CPU"]
    assert by["Saxpy"]["km"].full_name == "DotCompute.Samples.Elementwise.Saxpy"
    assert by["Saxpy"]["km"].backends == ["CPU", "HIP"]
    assert [by[k]["dims"] for k in ("Transpose", "MatMulNaive", "Stencil3D", "Saxpy")] == [2, 2, 3, 1]
    assert by["Softplus"]["entry"] is None and "MathF.Log" in by["Softplus"]["error"]
    hip = (tmp_path / "dc_generated_kernels.hip").read_text()
    reg = (tmp_path / "KernelRegistry.g.cpp").read_text()
    assert hip.count('extern "C" __global__') == 11
    assert 'k.Name = "Transpose";' in reg and "k.Dimensions = 2;" in reg and "HipKernelAbi::Generated" in reg
    assert 'k.HipDiagnostic = "call to MathF.Log";' in reg
    # the generated files of the build are exactly what the generator writes for this corpus
    built = os.path.join(ROOT, "dotcompute_amd", "_build", "generated", "KernelRegistry.g.cpp")
    if os.path.exists(built):
        assert open(built).read() == reg


def test_full_write_analysis_is_conservative():
    """Only a buffer written in full (the work-size buffer, assigned at the work index, at most under
    the bounds guard, before any return) may skip the copy to the device: anything else is copied in."""
    cov = lambda body, params="ReadOnlySpan<float> a, Span<float> b": kernel(body, params)["covered"]
    assert cov("int i = KernelContext.ThreadId.X; if (i < b.Length) b[i] = a[i];") == {"b"}
    assert cov("int i = KernelContext.ThreadId.X; b[i] = a[i] * 2f;") == {"b"}
    assert cov("int i = KernelContext.ThreadId.X; if (i < b.Length) { float t = a[i]; b[i] = t; }") == {"b"}
    assert cov("int i = KernelContext.ThreadId.X; if (i < b.Length && a[i] > 0f) b[i] = a[i];") == set()
    assert cov("int i = KernelContext.ThreadId.X; if (a[i] > 0f) b[i] = 1f; else b[i] = 2f;") == set()
    assert cov("int i = KernelContext.ThreadId.X; if (a[i] > 0f) return; b[i] = 1f;") == set()
    assert cov("int i = KernelContext.ThreadId.X; i = i / 2; b[i] = 1f;") == set()
    assert cov("int i = KernelContext.ThreadId.X; b[i / 2] = 1f;") == set()
    # the work size is the FIRST writable span: a second output is not covered by its index
    assert cov("int i = KernelContext.ThreadId.X; if (i < b.Length) { b[i] = a[i]; c[i] = a[i]; }",
               "ReadOnlySpan<float> a, Span<float> b, Span<float> c") == {"b"}


def test_transpose_2d_coordinates_and_intrinsics():
    """TransposeNaive of KernelExecutionMetadataTests: the coordinates come from the trailing int
    extents (cols -> x, rows -> y) and BlockId/BlockDim map as in the CPU invoker (0 and extent)."""
    r = one("""
    namespace TestApp { public static class Transpose {
      [Kernel(Backends = KernelBackends.CPU | KernelBackends.CUDA, VectorSize = 8, IsParallel = true)]
      public static void TransposeNaive(ReadOnlySpan<float> input, Span<float> output, int rows, int cols) {
        int row = KernelContext.ThreadId.Y + KernelContext.BlockId.Y * KernelContext.BlockDim.Y;
        int col = KernelContext.ThreadId.X + KernelContext.BlockId.X * KernelContext.BlockDim.X;
        if (row < rows && col < cols) output[col * rows + row] = input[row * cols + col];
      } } }""")
    src = r["source"]
    assert r["dims"] == 2 and r["km"].full_name == "TestApp.Transpose.TransposeNaive"
    assert r["km"].backends == ["CPU", "CUDA"] and r["km"].vector_size == 8
    assert "const int32_t __xext = (int32_t)cols, __yext = (int32_t)rows, __zext = 1;" in src
    assert "__x = __ii % __xext, __y = __ii / __xext" in src
    assert "int32_t row = (__y + (0 * __yext));" in src
    assert "void TransposeNaive(const float* input, float* output, int32_t rows, int32_t cols, const dc_gen_launch __l)" in src


def test_length_is_each_buffers_own_length():
    """The elementwise add bounded by c.Length (KernelExecutionMetadataTests' second case): each
    .Length reads that buffer's length, every access is bounds-checked."""
    r = kernel("int i = KernelContext.ThreadId.X; if (i < c.Length) c[i] = a[i] + b[i];",
               "ReadOnlySpan<float> a, ReadOnlySpan<float> b, Span<float> c")
    src = r["source"]
    assert r["needs_length"] and "(i < ((int32_t)__len2))" in src
    assert "dcg::ld(a, (int64_t)(i), __len0, __l) + dcg::ld(b, (int64_t)(i), __len1, __l)" in src
    assert "if ((uint64_t)__k1 < (uint64_t)__len2) c[__k1] = __v1;" in src
    assert r["reads"] == {"a", "b"} and r["writes"] == {"c"}


@pytest.mark.parametrize("expr,ctype,fragment", [
    ("u + i", "long", "((int64_t)(u)) + ((int64_t)(i))"),        # uint + int is long in C#
    ("u + 1", "uint", "(u + ((uint32_t)(1)))"),
    ("i * 2147483648", "long", "((int64_t)(i)) * ((int64_t)(2147483648u))"),  # the literal is a uint; uint * int is long
    ("3000000000", "uint", "3000000000u"),
    ("0xFFFFFFFFFF", "long", "1099511627775ll"),
    ("1.5f * i", "float", "(1.5f * ((float)(i)))"),
    ("2f", "float", "2.0f"),
    ("i << 33", "int", "dcg::shl<int32_t>(i, (int32_t)(33))"),
    ("u >> i", "uint", "dcg::shr<uint32_t>(u, (int32_t)(i))"),
    ("(int)f", "int", "dcg::f2i<int32_t>(f)"),
    ("i / 3", "int", "dcg::idiv<int32_t>(i, 3, __l)"),
    ("f % 2f", "float", "fmodf(f, 2.0f)"),
    ("-u", "long", "(-((int64_t)(u)))"),
    ("Math.Max(f, 2.0)", "double", "dcg::fmax_net<double>(((double)(f)), 2.0)"),
    ("Math.Abs(i)", "int", "dcg::abs_checked<int32_t>(i, __l)"),
    ("MathF.Sqrt(i)", "float", "sqrtf(((float)(i)))"),
    ("Math.Sqrt(f)", "double", "sqrt(((double)(f)))"),
])
def test_csharp_promotions_and_literals(expr, ctype, fragment):
    params = "Span<float> o, int i, uint u, float f"
    r = kernel(f"var v = {expr}; o[0] = (float)v;", params)
    assert r["error"] is None, r["error"]
    assert f"{ {'long': 'int64_t', 'uint': 'uint32_t', 'int': 'int32_t', 'float': 'float', 'double': 'double'}[ctype]} v = " in r["source"]
    assert fragment in r["source"], r["source"]


def test_compound_assignment_narrows_like_csharp():
    r = kernel("byte c = 250; c += 10; short s = 1; s <<= 3; o[0] = c + s;", "Span<int> o")
    src = r["source"]
    assert "(c = ((uint8_t)((((int32_t)(c)) + 10))));" in src
    assert "dcg::shl<int32_t>(((int32_t)(s)), (int32_t)(3))" in src
    r = kernel("float x = 1f; x += 2.5;", "Span<float> o")  # double not implicitly convertible to float
    assert r["entry"] is None and "double to float" in r["error"]


@pytest.mark.parametrize("body,params,why", [
    ('string s = "x";', "Span<float> o", "string"),
    ("o[0] = MathF.Exp(1f);", "Span<float> o", "MathF.Exp"),
    ("switch (1) { }", "Span<float> o", "switch"),
    ("int x = o[0];", "Span<float> o", "float to int"),
    ("o[0] = a[0];", "Span<float> o, ReadOnlySpan<decimal> a", "decimal"),
    ("a[0] = 1f;", "ReadOnlySpan<float> a", "ReadOnlySpan"),
    ("var q = o;", "Span<float> o", "used as a value"),
    ("int x = 1; { int x = 2; }", "Span<float> o", "shadows"),
    ("o[0] = 1f", "Span<float> o", "expected `;`"),
    ("ulong big = 1; int i = 2; var z = big + i;", "Span<float> o", "ulong with a signed operand"),
    ("o[(long)1] = 1f;", "Span<float> o", "span index of type long"),
    ("float f = 1f; int k = (byte)f;", "Span<float> o", "cast from float to byte"),
])
def test_unsupported_constructs_leave_no_hip_slot(body, params, why):
    r = kernel(body, params)
    assert r["entry"] is None and r["source"] is None
    assert why in r["error"], r["error"]


def test_ref_parameters_and_nonvoid_methods_are_rejected(tmp_path):
    (k,) = find_kernels("class K { [Kernel] public static void F(ref int x) { } }")
    assert "parameter modifier `ref`" in k.error and translate(k, "F")["entry"] is None
    with pytest.raises(cs.Unsupported):
        find_kernels("class K { [Kernel] public static int F(Span<int> x) { return 1; } }")
    f = tmp_path / "K.cs"
    f.write_text("class K { [Kernel] public static void F(ref int x) { } }")
    generate([str(f)], str(tmp_path / "g"))
    assert "K.F is not registered: parameter modifier `ref`" in (tmp_path / "g" / "KernelRegistry.g.cpp").read_text()


def test_generated_kernels_compile_for_gfx950(tmp_path):
    """The translation of the corpus plus a kernel using every supported construct compiles with
    hipcc for gfx950 (the build compiles the corpus too; this also covers the extra constructs)."""
    extra = """
    namespace X { public static class All {
      [Kernel] public static void Everything(ReadOnlySpan<double> d, Span<long> o, ReadOnlySpan<byte> bytes,
                                             Span<short> s, ulong seed, int n, int m) {
        int i = KernelContext.ThreadId.X, j = KernelContext.ThreadId.Y;
        if (i >= n || j >= m) return;
        long acc = 0;
        for (int k = 0, q = 1; k < bytes.Length; k += 2, q++) { if (k > 100) break; acc += bytes[k] * q; }
        while (acc > 1000) { acc >>= 1; if (acc == 7) continue; }
        double x = d[i] > 0.5 ? Math.Sqrt(d[i]) : -Math.Abs(d[i]);
        o[i] = acc + (long)x + (long)(seed >> 3) - (i % 3);
        s[j] += (short)1; s[j]++; --acc;
        bool flag = !(i == j) & (acc != 0) | false;
        if (flag) o[i] ^= ~acc;
        o[i] = unchecked_ok(o[i]);
      } } }""".replace("o[i] = unchecked_ok(o[i]);", "")
    d = tmp_path / "gen"
    cs_file = tmp_path / "Extra.cs"
    cs_file.write_text(extra)
    files = sorted(os.path.join(KERNELS, f) for f in os.listdir(KERNELS) if f.endswith(".cs")) + [str(cs_file)]
    recs = generate(files, str(d))
    assert all(r["entry"] for r in recs if r["km"].name != "Softplus"), [r["error"] for r in recs]
    (d / "probe.hip").write_text('#include "dc_generated_kernels.hip"\n')
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    r = subprocess.run([hipcc, "--genco", "--offload-arch=gfx950", "-O1", "-std=c++17", "-fwrapv", "-ffp-contract=off",
                        "-Werror", "-Wno-unused-command-line-argument", "-I", str(d), "-I",
                        os.path.join(ROOT, "dotcompute_amd", "csrc"), str(d / "probe.hip"), "-o", str(d / "probe.hsaco")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
