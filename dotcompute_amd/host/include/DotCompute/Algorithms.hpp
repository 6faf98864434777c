// Algorithms.hpp — dense MatMul and CSR SpMV on the HIP accelerator.
//
// Reference: Matrix (src/Extensions/DotCompute.Algorithms/LinearAlgebra/Matrix.cs:17,110, row-major
// float storage), MatrixOperations.MultiplyAsync (LinearAlgebra/Operations/MatrixOperations.cs:28-64),
// CsrMatrix<T> (Sparse/SparseMatrix.cs:68-272) and SparseOps.SpMV (Sparse/SparseMatrix.cs:669-692).
// Differences by design: there is no size threshold below which the multiply moves to the host,
// and no silent host fallback when the device call fails — errors surface as exceptions.
#pragma once

#include "Abstractions.hpp"
#include "Backends/Hip.hpp"

namespace DotCompute::Algorithms {

class Matrix {
 public:
  Matrix(int32_t rows, int32_t columns);
  Matrix(int32_t rows, int32_t columns, std::vector<float> data);
  int32_t Rows() const { return rows_; }
  int32_t Columns() const { return cols_; }
  int64_t Size() const { return (int64_t)rows_ * cols_; }
  float& operator()(int32_t r, int32_t c) { return data_[(size_t)r * cols_ + c]; }
  float operator()(int32_t r, int32_t c) const { return data_[(size_t)r * cols_ + c]; }
  std::vector<float>& Data() { return data_; }
  const std::vector<float>& Data() const { return data_; }

 private:
  int32_t rows_, cols_;
  std::vector<float> data_;
};

enum class MatMulPrecision { Float32, BFloat16 };

class MatrixOperations {
 public:
  // C = A·B. Throws ArgumentException when A.Columns != B.Rows (MatrixOperations.cs:33-38).
  // Float32 runs the fp32 MFMA kernel; BFloat16 rounds A and B to bf16 (RNE) on the device and
  // accumulates in fp32.
  static std::future<Matrix> MultiplyAsync(const Matrix& a, const Matrix& b, IAccelerator& accelerator,
                                           MatMulPrecision precision = MatMulPrecision::Float32);
};

template <typename T>
class CsrMatrix {
 public:
  // Validation and messages of SparseMatrix.cs:80-91.
  CsrMatrix(int32_t rows, int32_t columns, std::vector<T> values, std::vector<int32_t> columnIndices,
            std::vector<int32_t> rowPointers)
      : Rows(rows), Columns(columns), Values(std::move(values)), ColumnIndices(std::move(columnIndices)),
        RowPointers(std::move(rowPointers)) {
    if ((int64_t)RowPointers.size() != (int64_t)rows + 1)
      throw ArgumentException("CSR rowPointers must have exactly rows+1=" + std::to_string((int64_t)rows + 1) +
                              " entries (got " + std::to_string(RowPointers.size()) +
                              "). The last entry equals NNZ (number of non-zeros).");
    if (Values.size() != ColumnIndices.size())
      throw ArgumentException("CSR values.Length (" + std::to_string(Values.size()) +
                              ") must equal columnIndices.Length (" + std::to_string(ColumnIndices.size()) + ").");
  }
  int32_t Rows;
  int32_t Columns;
  std::vector<T> Values;
  std::vector<int32_t> ColumnIndices;
  std::vector<int32_t> RowPointers;
  int64_t NonZeroCount() const { return (int64_t)Values.size(); }
};

class SparseOps {
 public:
  // y = A·x (SparseMatrix.cs:669-692): ArgumentException when A.Columns != x.Length. The reference
  // is generic over INumber<T>; float, double and int run on the HIP kernels (int arithmetic wraps,
  // as C#'s unchecked default).
  static std::vector<float> SpMV(const CsrMatrix<float>& a, const std::vector<float>& x, IAccelerator& accelerator);
  static std::vector<double> SpMV(const CsrMatrix<double>& a, const std::vector<double>& x, IAccelerator& accelerator);
  static std::vector<int32_t> SpMV(const CsrMatrix<int32_t>& a, const std::vector<int32_t>& x,
                                   IAccelerator& accelerator);
  // The SpMV benchmark: `iterations` times y = A·x; x = y / sum(y). Returns x (rows == columns).
  static std::vector<float> PowerIterate(const CsrMatrix<float>& a, const std::vector<float>& x0, int32_t iterations,
                                         IAccelerator& accelerator, double* lastSum = nullptr);
};

}  // namespace DotCompute::Algorithms
