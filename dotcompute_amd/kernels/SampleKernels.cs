// [Kernel] methods of the HIP backend's sample project. The build translates each one to a gfx950
// kernel (dotcompute_amd/generator) and registers it; the GPU tests run them through
// IComputeOrchestrator.ExecuteAsync(name, "HIP", ...) against the CPU oracle.
using System;
using DotCompute.Generators;

namespace DotCompute.Samples
{
    public static class Elementwise
    {
        // y = a*x + y: reads and writes y (the orchestrator copies it in and back).
        [Kernel(Backends = KernelBackends.CPU | KernelBackends.HIP)]
        public static void Saxpy(ReadOnlySpan<float> x, Span<float> y, float a)
        {
            int i = KernelContext.ThreadId.X;
            if (i < y.Length)
            {
                y[i] = a * x[i] + y[i];
            }
        }

        // Branches, the conditional operator and MathF.Min/Max (NaN and signed-zero rules of .NET).
        [Kernel(Backends = KernelBackends.CPU | KernelBackends.HIP)]
        public static void ScaleClamp(ReadOnlySpan<float> input, Span<float> output, float scale, float lo, float hi)
        {
            int i = KernelContext.ThreadId.X;
            if (i >= output.Length)
                return;
            float v = input[i] * scale;
            if (v > 0f)
                output[i] = MathF.Min(v, hi);
            else
                output[i] = v < lo ? lo : MathF.Max(v, lo * 0.5f);
        }

        // Unsigned 32-bit arithmetic: wrapping multiplies, shifts and xor (the lowbias32 integer
        // hash of C. Wellons' hash-prospector).
        [Kernel(Backends = KernelBackends.CPU | KernelBackends.HIP)]
        public static void HashMix(ReadOnlySpan<uint> keys, Span<uint> hashes, uint seed)
        {
            int i = KernelContext.ThreadId.X;
            if (i < hashes.Length)
            {
                uint h = keys[i] ^ seed;
                h ^= h >> 16;
                h *= 0x7feb352du;
                h ^= h >> 15;
                h *= 0x846ca68bu;
                h ^= h >> 16;
                hashes[i] = h;
            }
        }

        // 64-bit integers: shift counts masked to 6 bits, int/long promotion, and a float -> long
        // cast that saturates.
        [Kernel(Backends = KernelBackends.CPU | KernelBackends.HIP)]
        public static void LongMix(ReadOnlySpan<long> a, ReadOnlySpan<float> f, Span<long> b, int shift)
        {
            int i = KernelContext.ThreadId.X;
            if (i < b.Length)
            {
                long s = a[i] << shift;
                b[i] = s + (long)(f[i] * 3.0e18f) + i;
            }
        }

        // A conditional write: elements whose input is not positive keep what the caller's output
        // array held, so the orchestrator must copy that array in before the launch.
        [Kernel(Backends = KernelBackends.CPU | KernelBackends.HIP)]
        public static void CopyPositive(ReadOnlySpan<float> input, Span<float> output)
        {
            int i = KernelContext.ThreadId.X;
            if (i < output.Length && input[i] > 0f)
                output[i] = input[i];
        }

        // Indices read from memory: an index outside the source throws IndexOutOfRangeException.
        [Kernel(Backends = KernelBackends.CPU | KernelBackends.HIP)]
        public static void Gather(ReadOnlySpan<float> source, ReadOnlySpan<int> index, Span<float> destination)
        {
            int i = KernelContext.ThreadId.X;
            if (i < destination.Length)
                destination[i] = source[index[i]];
        }

        // Integer division: a zero divisor throws DivideByZeroException.
        [Kernel(Backends = KernelBackends.CPU | KernelBackends.HIP)]
        public static void IntDivide(ReadOnlySpan<int> a, ReadOnlySpan<int> b, Span<int> quotient)
        {
            int i = KernelContext.ThreadId.X;
            if (i < quotient.Length)
                quotient[i] = a[i] / b[i];
        }

        // MathF.Exp is outside the translatable subset: this kernel registers for the CPU only.
        [Kernel]
        public static void Softplus(ReadOnlySpan<float> x, Span<float> y)
        {
            int i = KernelContext.ThreadId.X;
            if (i < y.Length)
                y[i] = MathF.Log(1f + MathF.Exp(x[i]));
        }
    }

    public static class Grids
    {
        // 2-D: the coordinates come from the trailing (rows, cols) extents.
        [Kernel(Backends = KernelBackends.CPU | KernelBackends.HIP)]
        public static void Transpose(ReadOnlySpan<float> input, Span<float> output, int rows, int cols)
        {
            int r = KernelContext.BlockId.Y * KernelContext.BlockDim.Y + KernelContext.ThreadId.Y;
            int c = KernelContext.BlockId.X * KernelContext.BlockDim.X + KernelContext.ThreadId.X;
            if (r < rows && c < cols)
                output[c * rows + r] = input[r * cols + c];
        }

        // 2-D with a loop: C[m x n] = A[m x k] * B[k x n], one output element per work item, the
        // inner product accumulated in order with one rounding per multiply and per add.
        [Kernel(Backends = KernelBackends.CPU | KernelBackends.HIP)]
        public static void MatMulNaive(ReadOnlySpan<float> a, ReadOnlySpan<float> b, Span<float> c, int k, int m, int n)
        {
            int row = KernelContext.ThreadId.Y;
            int col = KernelContext.ThreadId.X;
            if (row < m && col < n)
            {
                float sum = 0f;
                for (int p = 0; p < k; p++)
                {
                    sum += a[row * k + p] * b[p * n + col];
                }
                c[row * n + col] = sum;
            }
        }

        // 3-D: a stencil over (depth, height, width) with a boundary branch.
        [Kernel(Backends = KernelBackends.CPU | KernelBackends.HIP)]
        public static void Stencil3D(ReadOnlySpan<float> src, Span<float> dst, int depth, int height, int width)
        {
            int x = KernelContext.ThreadId.X;
            int y = KernelContext.ThreadId.Y;
            int z = KernelContext.ThreadId.Z;
            if (x < width && y < height && z < depth)
            {
                int idx = (z * height + y) * width + x;
                float left = x > 0 ? src[idx - 1] : 0f;
                float below = z > 0 ? src[idx - width * height] : 0f;
                dst[idx] = src[idx] * 2f - left - 0.5f * below;
            }
        }
    }
}
