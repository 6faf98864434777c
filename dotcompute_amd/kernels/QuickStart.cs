// The README quick-start kernel (Kernels.VectorAdd), the [Kernel] the orchestrator benchmark runs:
// `await orchestrator.ExecuteAsync<float[]>("VectorAdd", "HIP", a, b, result)`.
using System;
using DotCompute.Generators;

public static class Kernels
{
    [Kernel]
    public static void VectorAdd(ReadOnlySpan<float> a, ReadOnlySpan<float> b, Span<float> result)
    {
        int idx = KernelContext.ThreadId.X;
        if (idx < result.Length) result[idx] = a[idx] + b[idx];
    }
}
