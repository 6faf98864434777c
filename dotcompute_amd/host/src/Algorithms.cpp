// Algorithms.cpp — MatrixOperations and SparseOps on the HIP accelerator.
#include "DotCompute/Algorithms.hpp"

namespace DotCompute::Algorithms {

using Backends::Hip::Check;
using Backends::Hip::HipAccelerator;

namespace {
HipAccelerator& RequireHip(IAccelerator& accelerator) {
  auto* hip = dynamic_cast<HipAccelerator*>(&accelerator);
  if (!hip)
    throw NotSupportedException("this build runs MatMul/SpMV on HIP accelerators only (got '" +
                                accelerator.Info().DeviceType + "')");
  return *hip;
}
}  // namespace

Matrix::Matrix(int32_t rows, int32_t columns) : rows_(rows), cols_(columns) {
  if (rows < 0 || columns < 0) throw ArgumentException("matrix dimensions must be non-negative");
  data_.assign((size_t)rows * columns, 0.0f);
}

Matrix::Matrix(int32_t rows, int32_t columns, std::vector<float> data)
    : rows_(rows), cols_(columns), data_(std::move(data)) {
  if (rows < 0 || columns < 0) throw ArgumentException("matrix dimensions must be non-negative");
  if ((int64_t)data_.size() != (int64_t)rows * columns)
    throw ArgumentException("data length " + std::to_string(data_.size()) + " does not match " +
                            std::to_string(rows) + "x" + std::to_string(columns));
}

std::future<Matrix> MatrixOperations::MultiplyAsync(const Matrix& a, const Matrix& b, IAccelerator& accelerator,
                                                    MatMulPrecision precision) {
  if (a.Columns() != b.Rows())
    throw ArgumentException("Matrix multiplication requires A.Columns == B.Rows (got A=" + std::to_string(a.Rows()) +
                            "x" + std::to_string(a.Columns()) + ", B=" + std::to_string(b.Rows()) + "x" +
                            std::to_string(b.Columns()) + ").");
  HipAccelerator& hip = RequireHip(accelerator);
  const int64_t m = a.Rows(), k = a.Columns(), n = b.Columns();
  Matrix c(a.Rows(), b.Columns());
  auto& mem = hip.Memory();
  auto da = mem.AllocateAsync<float>(std::max<int64_t>(m * k, 1));
  auto db = mem.AllocateAsync<float>(std::max<int64_t>(k * n, 1));
  auto dc = mem.AllocateAsync<float>(std::max<int64_t>(m * n, 1));
  if (m > 0 && k > 0) da->CopyFromHost(a.Data().data(), (size_t)(m * k) * sizeof(float));
  if (k > 0 && n > 0) db->CopyFromHost(b.Data().data(), (size_t)(k * n) * sizeof(float));
  if (precision == MatMulPrecision::Float32) {
    Check(dc_hip_gemm_f32(hip.Context(), da->Data(), db->Data(), dc->Data(), m, n, k), "dc_hip_gemm_f32");
  } else {
    auto ha = mem.AllocateAsync<uint16_t>(std::max<int64_t>(m * k, 1));
    auto hb = mem.AllocateAsync<uint16_t>(std::max<int64_t>(k * n, 1));
    Check(dc_hip_convert_f32_to_bf16(hip.Context(), da->Data(), ha->Data(), m * k), "convert A");
    Check(dc_hip_convert_f32_to_bf16(hip.Context(), db->Data(), hb->Data(), k * n), "convert B");
    Check(dc_hip_gemm_bf16(hip.Context(), ha->Data(), hb->Data(), dc->Data(), m, n, k), "dc_hip_gemm_bf16");
    hip.Synchronize();
  }
  hip.Synchronize();
  if (m > 0 && n > 0) dc->CopyToHost(c.Data().data(), (size_t)(m * n) * sizeof(float));
  std::promise<Matrix> p;
  p.set_value(std::move(c));
  return p.get_future();
}

namespace {
// The kernels index values/columns/x through the row pointers: reject a malformed CSR on the host
// (the reference would fail with IndexOutOfRangeException inside SpMV).
template <typename T>
void ValidateCsr(const CsrMatrix<T>& a) {
  if (a.Rows < 0 || a.Columns < 0) throw ArgumentException("CSR dimensions must be non-negative");
  if (a.RowPointers.empty() || a.RowPointers[0] != 0 || (int64_t)a.RowPointers.back() != a.NonZeroCount())
    throw ArgumentException("CSR rowPointers must start at 0 and end at NNZ");
  for (size_t r = 0; r + 1 < a.RowPointers.size(); ++r)
    if (a.RowPointers[r + 1] < a.RowPointers[r]) throw ArgumentException("CSR rowPointers must be non-decreasing");
  for (int32_t c : a.ColumnIndices)
    if (c < 0 || c >= a.Columns) throw ArgumentException("CSR column index out of range");
}

template <typename T>
struct DeviceCsr {
  std::shared_ptr<IUnifiedMemoryBufferT<int32_t>> rp, col;
  std::shared_ptr<IUnifiedMemoryBufferT<T>> val;
};

template <typename T>
DeviceCsr<T> Upload(HipAccelerator& hip, const CsrMatrix<T>& a) {
  DeviceCsr<T> d;
  auto& mem = hip.Memory();
  const size_t nnz = a.Values.size();
  d.rp = mem.AllocateAsync<int32_t>(a.RowPointers.size());
  d.col = mem.AllocateAsync<int32_t>(std::max<size_t>(nnz, 1));
  d.val = mem.AllocateAsync<T>(std::max<size_t>(nnz, 1));
  d.rp->CopyFromHost(a.RowPointers.data(), a.RowPointers.size() * sizeof(int32_t));
  if (nnz) {
    d.col->CopyFromHost(a.ColumnIndices.data(), nnz * sizeof(int32_t));
    d.val->CopyFromHost(a.Values.data(), nnz * sizeof(T));
  }
  return d;
}

int32_t SpmvCsr(dc_hip_ctx* ctx, const int32_t* rp, const int32_t* col, const float* val, const float* x, float* y,
                int64_t rows, int64_t cols, int64_t nnz) {
  return dc_hip_spmv_csr_f32(ctx, rp, col, val, x, y, rows, cols, nnz);
}
int32_t SpmvCsr(dc_hip_ctx* ctx, const int32_t* rp, const int32_t* col, const double* val, const double* x, double* y,
                int64_t rows, int64_t cols, int64_t nnz) {
  return dc_hip_spmv_csr_f64(ctx, rp, col, val, x, y, rows, cols, nnz);
}
int32_t SpmvCsr(dc_hip_ctx* ctx, const int32_t* rp, const int32_t* col, const int32_t* val, const int32_t* x,
                int32_t* y, int64_t rows, int64_t cols, int64_t nnz) {
  return dc_hip_spmv_csr_i32(ctx, rp, col, val, x, y, rows, cols, nnz);
}

template <typename T>
std::vector<T> SpMVOn(const CsrMatrix<T>& a, const std::vector<T>& x, IAccelerator& accelerator) {
  if ((int64_t)a.Columns != (int64_t)x.size())
    throw ArgumentException("SpMV dimension mismatch: matrix A is " + std::to_string(a.Rows) + "x" +
                            std::to_string(a.Columns) + " but vector x has " + std::to_string(x.size()) +
                            " element(s). For y = A·x the number of columns in A must equal the length of x.");
  HipAccelerator& hip = RequireHip(accelerator);
  ValidateCsr(a);
  DeviceCsr<T> d = Upload(hip, a);
  auto dx = hip.Memory().AllocateAsync<T>(std::max<size_t>(x.size(), 1));
  auto dy = hip.Memory().AllocateAsync<T>(std::max<int32_t>(a.Rows, 1));
  if (!x.empty()) dx->CopyFromHost(x.data(), x.size() * sizeof(T));
  Check(SpmvCsr(hip.Context(), d.rp->Data(), d.col->Data(), d.val->Data(), dx->Data(), dy->Data(), a.Rows, a.Columns,
                a.NonZeroCount()),
        "dc_hip_spmv_csr");
  hip.Synchronize();
  std::vector<T> y((size_t)a.Rows);
  if (!y.empty()) dy->CopyToHost(y.data(), y.size() * sizeof(T));
  return y;
}
}  // namespace

std::vector<float> SparseOps::SpMV(const CsrMatrix<float>& a, const std::vector<float>& x, IAccelerator& accelerator) {
  return SpMVOn(a, x, accelerator);
}
std::vector<double> SparseOps::SpMV(const CsrMatrix<double>& a, const std::vector<double>& x,
                                    IAccelerator& accelerator) {
  return SpMVOn(a, x, accelerator);
}
std::vector<int32_t> SparseOps::SpMV(const CsrMatrix<int32_t>& a, const std::vector<int32_t>& x,
                                     IAccelerator& accelerator) {
  return SpMVOn(a, x, accelerator);
}

std::vector<float> SparseOps::PowerIterate(const CsrMatrix<float>& a, const std::vector<float>& x0, int32_t iterations,
                                           IAccelerator& accelerator, double* lastSum) {
  if (a.Rows != a.Columns) throw ArgumentException("power iteration needs a square matrix");
  if ((int64_t)x0.size() != (int64_t)a.Columns) throw ArgumentException("x0 length must equal the column count");
  if (iterations < 0) throw ArgumentException("iterations must be non-negative");
  HipAccelerator& hip = RequireHip(accelerator);
  ValidateCsr(a);
  DeviceCsr<float> d = Upload(hip, a);
  auto dx = hip.Memory().AllocateAsync<float>(std::max<size_t>(x0.size(), 1));
  auto dy = hip.Memory().AllocateAsync<float>(std::max<size_t>(x0.size(), 1));
  auto ds = hip.Memory().AllocateAsync<double>(1);
  if (!x0.empty()) dx->CopyFromHost(x0.data(), x0.size() * sizeof(float));
  Check(dc_hip_spmv_power_iterate_f32(hip.Context(), d.rp->Data(), d.col->Data(), d.val->Data(), dx->Data(), dy->Data(),
                                      a.Rows, a.NonZeroCount(), iterations, ds->Data()),
        "dc_hip_spmv_power_iterate_f32");
  hip.Synchronize();
  std::vector<float> x(x0.size());
  if (!x.empty()) dx->CopyToHost(x.data(), x.size() * sizeof(float));
  if (lastSum) {
    *lastSum = 0.0;
    if (iterations > 0 && a.Rows > 0) ds->CopyToHost(lastSum, sizeof(double));
  }
  return x;
}

}  // namespace DotCompute::Algorithms
