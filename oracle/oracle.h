/*
 * oracle.h — CPU restatement of the DotCompute reference semantics for the HIP hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load liboracle.so, and only as the checker (or as the timed CPU baseline). The HIP product
 * path never calls it.
 *
 * The reference (mivertowski/DotCompute) is C#/.NET 10; there is no .NET SDK in this image, so
 * the reference cannot be compiled or run here (oracle/_ref stays empty). Each function below
 * cites the reference file:line whose behaviour it restates; the inputs come from this build's
 * own counter-based generators (the reference's System.Random streams are BCL-internal).
 *
 * Pinning (what each function is checked against in tests/test_oracle.py):
 *   generators ........ golden fixtures (tests/golden), splitmix64 published test vectors,
 *                       distribution moments, Zipf CDF closed form
 *   vector_add ........ reference known-answer tests, closed form
 *   sum_f32 ............ reference known answers (Sum 1..5 = 15, Sum 1..1000 = 500500), exact
 *                       integer-valued floats, math.fsum / Neumaier, permutation invariance
 *   sum_i32 ............ exact Python int sum, overflow boundaries
 *   linq ............... reference LINQ golden vectors ({1..5}.Where(x>3) -> {4,5}, ...), numpy
 *                       boolean-mask evaluation, hand-written lambdas vs the program interpreter
 *   gemm ............... numpy float64 matmul, identity/permutation matrices, rank-1 closed form
 *   spmv ............... dense brute force (numpy) on small graphs, stochastic-matrix invariants
 */
#ifndef DC_ORACLE_H
#define DC_ORACLE_H

#include <stdint.h>

#include "../include/dotcompute_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- generators (this build's input spec) ---- */
uint64_t oracle_splitmix64(uint64_t z);
void oracle_gen_uniform_f32(float* dst, int64_t n, uint64_t seed, uint32_t stream, int32_t unit_interval);
void oracle_gen_uniform_i32(int32_t* dst, int64_t n, uint64_t seed, uint32_t stream, int32_t lo, int32_t hi);
int64_t oracle_gen_zipf_rowptr(int64_t rows, double alpha, int32_t max_degree, uint64_t seed,
                               int32_t* row_pointers);
void oracle_gen_zipf_fill(int64_t rows, int64_t cols, uint64_t seed, const int32_t* row_pointers,
                          int32_t* col_indices, float* values);

/* ---- VectorAdd ---- */
void oracle_vector_add_f32(const float* a, const float* b, float* result, int64_t n);

/* ---- Sum ---- */
float oracle_sum_f32_enumerable(const float* x, int64_t n, double* as_double);
float oracle_sum_f32_partitioned(const float* x, int64_t n, int32_t partitions, double* as_double);
double oracle_sum_f32_compensated(const float* x, int64_t n);
int32_t oracle_sum_i32_checked(const int32_t* x, int64_t n, int32_t* sum_out);
int32_t oracle_sum_i32_bcl(const int32_t* x, int64_t n, int32_t lanes, int32_t* sum_out);
int64_t oracle_sum_i32_exact(const int32_t* x, int64_t n);

/* ---- LINQ Where/Select ---- */
int64_t oracle_where_gt0_select_2x_plus_1(const float* in, int64_t n, float* out);
float oracle_where_gt0_select_2x_plus_1_sum(const float* in, int64_t n, int64_t* count, double* as_double);
int32_t oracle_linq_eval(const dc_linq_chain* chain, float x, float* y_out);
int64_t oracle_linq_where_select(const dc_linq_chain* chain, const float* in, int64_t n, float* out);
float oracle_linq_where_select_sum(const dc_linq_chain* chain, const float* in, int64_t n,
                                   int64_t* count, double* as_double);
/* Where/Select -> Min / Max of the kept, mapped elements. The reference runs these terminal
 * operators as LINQ-to-objects (ComputeQueryableExtensions.cs:265-267 scalar branch; Min/Max become
 * Reduce operations, ExpressionTreeVisitor.cs:244-245), i.e. the .NET 10 BCL
 * System.Linq.Enumerable.Min/Max(IEnumerable<float>) (global.json:3-4; not vendored in the
 * reference), restated here as its published enumerator loop:
 *   Min: the first element; if it is NaN return it; then for each x: if (x < value) value = x;
 *        else if (IsNaN(x)) return x.       (the first NaN wins; else the first smallest)
 *   Max: the first element; while it is NaN take the next (return it if none is left); then for
 *        each x: if (x > value) value = x.  (NaNs skipped; the first largest; all NaN: the last)
 * Writes the result to *out and returns the number of kept elements (0: the sequence is empty and
 * the caller throws InvalidOperationException), or a negative value for an invalid program. */
int64_t oracle_linq_where_select_min(const dc_linq_chain* chain, const float* in, int64_t n, float* out);
int64_t oracle_linq_where_select_max(const dc_linq_chain* chain, const float* in, int64_t n, float* out);
/* Aggregate((acc, x) => MathF.Min(acc, x)) (op 0) / MathF.Max (op 1) over the kept, mapped
 * elements, folded in sequence order from the first one: result to *out, returns the kept count
 * (0: the caller throws InvalidOperationException) or a negative value for an invalid program. */
int64_t oracle_linq_where_select_fold(const dc_linq_chain* chain, const float* in, int64_t n, int32_t op, float* out);
/* The same two operators after .Where(x > 0f).Select(x * 2f + 1f) with the lambdas written out
 * (op 0 = Min, 1 = Max): the CPU baseline of the fused Min/Max leg. */
int64_t oracle_where_gt0_select_2x_plus_1_minmax(const float* in, int64_t n, int32_t op, float* out);

/* ---- LINQ Where/Select over int32 (C# int semantics, exceptions reported as 4 * index + kind,
 * kind DC_LINQ_FAULT_*; -1 = none) ---- */
int32_t oracle_linq_eval_i32(const dc_linq_chain* chain, int32_t x, int32_t* y_out, int32_t* fault_out);
int64_t oracle_linq_where_select_i32(const dc_linq_chain* chain, const int32_t* in, int64_t n, int32_t* out,
                                     int64_t* fault_out);
int64_t oracle_linq_where_select_sum_i32(const dc_linq_chain* chain, const int32_t* in, int64_t n,
                                         int64_t* total_out, int32_t* overflow_out, int64_t* fault_out);
int64_t oracle_linq_where_select_minmax_i32(const dc_linq_chain* chain, const int32_t* in, int64_t n, int32_t op,
                                            int32_t* value_out, int64_t* fault_out);

/* ---- GEMM ---- */
void oracle_gemm_f32_naive(const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k,
                           int32_t threads);
void oracle_gemm_f32_naive_rows(const float* a, const float* b, float* c, int64_t m, int64_t n,
                                int64_t k, int64_t row_begin, int64_t row_end, int32_t threads);
void oracle_gemm_f32_blocked(const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k);
void oracle_gemm_f64_rows(const float* a, const float* b, double* c, double* abs_c, int64_t m,
                          int64_t n, int64_t k, const int64_t* rows, int64_t n_rows, int32_t threads);
uint16_t oracle_f32_to_bf16(float x);
float oracle_bf16_to_f32(uint16_t h);
void oracle_f32_to_bf16_array(const float* x, uint16_t* out, int64_t n);

/* ---- SpMV ---- */
int32_t oracle_spmv_csr_f32(const int32_t* row_pointers, const int32_t* col_indices, const float* values,
                            const float* x, float* y, int64_t rows, int64_t cols, int64_t x_len);
void oracle_spmv_csr_f64(const int32_t* row_pointers, const int32_t* col_indices, const float* values,
                         const double* x, double* y, int64_t rows);
int32_t oracle_spmv_csr_f64d(const int32_t* row_pointers, const int32_t* col_indices, const double* values,
                             const double* x, double* y, int64_t rows, int64_t cols, int64_t x_len);
int32_t oracle_spmv_csr_i32(const int32_t* row_pointers, const int32_t* col_indices, const int32_t* values,
                            const int32_t* x, int32_t* y, int64_t rows, int64_t cols, int64_t x_len);
int32_t oracle_spmv_power_f32(const int32_t* row_pointers, const int32_t* col_indices, const float* values,
                              float* x, float* y, int64_t rows, int32_t iterations, double* last_sum);


/* [Kernel] samples of dotcompute_amd/kernels/ (*.cs files) under the CPU invoker's semantics.
 * Return 0, or 1 (IndexOutOfRange), 2 (DivideByZero), 3 (Overflow) for the first exception. */
float oracle_net_minf(float a, float b);
float oracle_net_maxf(float a, float b);
int64_t oracle_net_f2l(float x);
int32_t oracle_kernel_saxpy(const float* x, int64_t nx, float* y, int64_t ny, float a);
int32_t oracle_kernel_scale_clamp(const float* in, int64_t nin, float* out, int64_t nout, float scale, float lo,
                                  float hi);
int32_t oracle_kernel_hash_mix(const uint32_t* keys, int64_t nk, uint32_t* hashes, int64_t nh, uint32_t seed);
int32_t oracle_kernel_long_mix(const int64_t* a, int64_t na, const float* f, int64_t nf, int64_t* b, int64_t nb,
                               int32_t shift);
int32_t oracle_kernel_gather(const float* src, int64_t nsrc, const int32_t* index, int64_t nidx, float* dst,
                             int64_t ndst);
int32_t oracle_kernel_int_divide(const int32_t* a, int64_t na, const int32_t* b, int64_t nb, int32_t* q, int64_t nq);
int32_t oracle_kernel_transpose(const float* in, int64_t nin, float* out, int64_t nout, int32_t rows, int32_t cols);
int32_t oracle_kernel_matmul_naive(const float* a, int64_t na, const float* b, int64_t nb, float* c, int64_t nc,
                                   int32_t k, int32_t m, int32_t n);
int32_t oracle_kernel_stencil3d(const float* src, int64_t ns, float* dst, int64_t nd, int32_t depth, int32_t height,
                                int32_t width);

#ifdef __cplusplus
}
#endif

#endif
