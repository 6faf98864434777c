// dc_module_kernels.hip — the code object (dc_kernels_gfx950.hsaco) behind the generic
// module-load + launch path (dc_hip_module_load / dc_hip_launch_kernel), i.e. what the managed
// HipCompiledKernel resolves by registry name: the kernels the generator translated from the
// [Kernel] methods of dotcompute_amd/kernels/*.cs (dc_generated_kernels.hip, written into the build
// directory), and a hand-written kernel with the parameter list of the reference's CUDA SpMV string.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "dc_generated_kernels.hip"

// Sparse y = A·x with one wavefront per row (64 lanes stride the row's nonzeros, then a wave
// reduction); parameter list of SparseMatrixKernels.CUDASparseMatrixKernel
// (src/Extensions/DotCompute.Algorithms/Kernels/LinearAlgebra/SparseMatrixKernels.cs:47-75).
// Launch: blocks of 256 threads, 4 rows per block.
extern "C" __global__ __launch_bounds__(256) void csr_spmv(const float* __restrict__ values,
                                                           const int* __restrict__ col_indices,
                                                           const int* __restrict__ row_pointers,
                                                           const float* __restrict__ x, float* __restrict__ y,
                                                           int num_rows) {
  const int row = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= num_rows) return;  // whole waves exit together: row is wave-uniform
  float sum = 0.0f;
  for (int i = row_pointers[row] + lane; i < row_pointers[row + 1]; i += 64) sum += values[i] * x[col_indices[i]];
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  if (lane == 0) y[row] = sum;
}
