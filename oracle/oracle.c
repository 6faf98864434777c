/*
 * oracle.c — CPU restatement of the DotCompute reference semantics for the HIP hot path.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg as the checker / timed CPU baseline; never by the HIP product path.
 *
 * Built with -ffp-contract=off so every float operation rounds once, as .NET's RyuJIT does for
 * scalar float arithmetic (it never contracts a*b+c into an FMA).
 * Citations are paths in the mivertowski/DotCompute repository.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------ */
/* Generators: this build's input specification (not reference code).                          */
/* ------------------------------------------------------------------------------------------ */

/* SplitMix64 finaliser (Steele, Lea, Flood, "Fast splittable pseudorandom number generators",
 * OOPSLA 2014; constants as published with Java 8's SplittableRandom). */
uint64_t oracle_splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static inline uint64_t key_of(uint64_t seed, uint32_t stream, uint64_t i) {
  return seed ^ ((uint64_t)stream << 40) ^ i;
}

void oracle_gen_uniform_f32(float* dst, int64_t n, uint64_t seed, uint32_t stream, int32_t unit_interval) {
  for (int64_t i = 0; i < n; ++i) {
    uint64_t r = oracle_splitmix64(key_of(seed, stream, (uint64_t)i));
    float u = (float)(uint32_t)(r >> 40);
    if (unit_interval)
      dst[i] = u * 0x1p-24f;          /* [0, 1) */
    else
      dst[i] = u * 0x1p-23f - 1.0f;   /* [-1, 1), exact */
  }
}

void oracle_gen_uniform_i32(int32_t* dst, int64_t n, uint64_t seed, uint32_t stream, int32_t lo, int32_t hi) {
  uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
  for (int64_t i = 0; i < n; ++i) {
    uint64_t r = oracle_splitmix64(key_of(seed, stream, (uint64_t)i));
    dst[i] = (int32_t)((int64_t)lo + (int64_t)(((r >> 32) * span) >> 32));
  }
}

/* Zipf(alpha) on [1, max_degree] by inverse CDF: degree = smallest d with cdf[d] > u, u in [0,1)
 * from 53 random bits. Stream 3 keyed by row index. */
int64_t oracle_gen_zipf_rowptr(int64_t rows, double alpha, int32_t max_degree, uint64_t seed,
                               int32_t* row_pointers) {
  if (rows < 0 || max_degree < 1) return -1;
  double* cdf = (double*)malloc(sizeof(double) * (size_t)(max_degree + 1));
  if (!cdf) return -1;
  double total = 0.0;
  for (int32_t d = 1; d <= max_degree; ++d) total += pow((double)d, -alpha);
  double acc = 0.0;
  cdf[0] = 0.0;
  for (int32_t d = 1; d <= max_degree; ++d) {
    acc += pow((double)d, -alpha);
    cdf[d] = acc / total;
  }
  cdf[max_degree] = 1.0;
  int64_t nnz = 0;
  row_pointers[0] = 0;
  for (int64_t r = 0; r < rows; ++r) {
    uint64_t z = oracle_splitmix64(key_of(seed, 3u, (uint64_t)r));
    double u = (double)(z >> 11) * 0x1p-53;
    int32_t lo = 1, hi = max_degree; /* smallest d in [1,max] with cdf[d] > u */
    while (lo < hi) {
      int32_t mid = lo + (hi - lo) / 2;
      if (cdf[mid] > u) hi = mid; else lo = mid + 1;
    }
    nnz += lo;
    if (nnz > 2147483647LL) { free(cdf); return -1; }
    row_pointers[r + 1] = (int32_t)nnz;
  }
  free(cdf);
  return nnz;
}

/* Columns: stream 4 keyed by the global nonzero index; uniform over the cols-1 non-diagonal
 * columns (self-loops skipped by shifting c >= row up by one). Values: 1/out-degree. */
void oracle_gen_zipf_fill(int64_t rows, int64_t cols, uint64_t seed, const int32_t* row_pointers,
                          int32_t* col_indices, float* values) {
  uint64_t span = (uint64_t)(cols - 1);
  for (int64_t r = 0; r < rows; ++r) {
    int32_t b = row_pointers[r], e = row_pointers[r + 1];
    float v = 1.0f / (float)(e - b);
    for (int32_t j = b; j < e; ++j) {
      uint64_t z = oracle_splitmix64(key_of(seed, 4u, (uint64_t)j));
      int64_t c = (int64_t)(((z >> 32) * span) >> 32);
      if (c >= r) c += 1;
      col_indices[j] = (int32_t)c;
      values[j] = v;
    }
  }
}

/* ------------------------------------------------------------------------------------------ */
/* VectorAdd                                                                                    */
/* ------------------------------------------------------------------------------------------ */

/* The generator-emitted CPU invoker runs the [Kernel] body `result[i] = a[i] + b[i]` over the
 * flat range [0, N) on one thread (src/Runtime/DotCompute.Generators/Kernel/Generation/
 * KernelExecutionMetadataEmitter.cs:117-170, invoked by src/Runtime/DotCompute.Runtime/Services/
 * KernelExecutionService.cs:275-288). OptimizedVectorAddKernel computes the same sums with
 * Vector<float> (src/Backends/DotCompute.Backends.CPU/Kernels/Optimized/
 * OptimizedVectorAddKernel.cs:91-108); one IEEE rounding per element either way. */
void oracle_vector_add_f32(const float* a, const float* b, float* result, int64_t n) {
  for (int64_t i = 0; i < n; ++i) result[i] = a[i] + b[i];
}

/* ------------------------------------------------------------------------------------------ */
/* Sum                                                                                          */
/* ------------------------------------------------------------------------------------------ */

/* Enumerable.Sum(IEnumerable<float>) as reached from ComputeQueryProvider.Execute's scalar branch
 * (src/Extensions/DotCompute.Linq/ComputeQueryableExtensions.cs:265-267): a sequential double
 * accumulator, cast to float at the end (.NET 10 BCL System.Linq, Sum.cs). */
float oracle_sum_f32_enumerable(const float* x, int64_t n, double* as_double) {
  double s = 0.0;
  for (int64_t i = 0; i < n; ++i) s += (double)x[i];
  if (as_double) *as_double = s;
  return (float)s;
}

typedef struct {
  const float* x;
  int64_t start, end;
  double sum;
} part_arg;

static void* part_worker(void* p) {
  part_arg* a = (part_arg*)p;
  double s = 0.0;
  for (int64_t i = a->start; i < a->end; ++i) s += (double)a->x[i];
  a->sum = s;
  return NULL;
}

/* OptimizedReductionKernel: ProcessorCount contiguous partitions (the last takes the remainder),
 * each a sequential double sum, run under Parallel.For, then partitionSums.Sum() in partition
 * order and a float cast (src/Backends/DotCompute.Backends.CPU/Kernels/Optimized/
 * OptimizedReductionKernel.cs:69-95). One thread per partition here. */
float oracle_sum_f32_partitioned(const float* x, int64_t n, int32_t partitions, double* as_double) {
  if (partitions < 1) partitions = 1;
  part_arg* args = (part_arg*)calloc((size_t)partitions, sizeof(part_arg));
  pthread_t* th = (pthread_t*)calloc((size_t)partitions, sizeof(pthread_t));
  int64_t per = n / partitions;
  for (int32_t p = 0; p < partitions; ++p) {
    args[p].x = x;
    args[p].start = (int64_t)p * per;
    args[p].end = (p == partitions - 1) ? n : args[p].start + per;
    pthread_create(&th[p], NULL, part_worker, &args[p]);
  }
  double total = 0.0;
  for (int32_t p = 0; p < partitions; ++p) {
    pthread_join(th[p], NULL);
    total += args[p].sum;
  }
  free(args);
  free(th);
  if (as_double) *as_double = total;
  return (float)total;
}

/* Neumaier-compensated double sum: the near-exact float64 host reference the fp32 tolerance
 * rel 1e-5*log2(N) is measured against. */
double oracle_sum_f32_compensated(const float* x, int64_t n) {
  double s = 0.0, c = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    double v = (double)x[i];
    double t = s + v;
    if (fabs(s) >= fabs(v)) c += (s - t) + v; else c += (v - t) + s;
    s = t;
  }
  return s + c;
}

/* Enumerable.Sum(IEnumerable<int>) is `checked` int32 arithmetic and throws OverflowException
 * (.NET BCL, reached from ComputeQueryableExtensions.cs:265-267). Returns DC_ERR_OVERFLOW where it
 * would throw: sequentially, as soon as a running total leaves int32. */
int32_t oracle_sum_i32_checked(const int32_t* x, int64_t n, int32_t* sum_out) {
  int64_t s = 0;
  for (int64_t i = 0; i < n; ++i) {
    s += x[i];
    if (s > 2147483647LL || s < -2147483648LL) return DC_ERR_OVERFLOW;
  }
  if (sum_out) *sum_out = (int32_t)s;
  return DC_OK;
}

/* Enumerable.Sum(IEnumerable<int>) as the .NET 10 BCL runs it for array / List<int> sources
 * (dotnet/runtime, src/libraries/System.Linq/src/System/Linq/Sum.cs: Sum<T,TResult>(ReadOnlySpan<T>)
 * and SumSignedIntegersVectorized; not vendored in the reference, reached from
 * ComputeQueryableExtensions.cs:265-267). When Vector<int>.Count = W > 2 and n >= 4W it sums W
 * wrapping int32 lanes (lane l takes elements l, l+W, l+2W, ...), tracking signed overflow of every
 * lane add as (r ^ a) & (r ^ d) and throwing after each unrolled group of 4 vectors (then after the
 * single-vector loop); the lane totals are then added in lane order with checked adds, then the
 * remaining elements. Otherwise it is one checked running total. `lanes` = W (8 on x64, 4 on
 * Arm64). Returns DC_ERR_OVERFLOW where the BCL throws OverflowException. */
int32_t oracle_sum_i32_bcl(const int32_t* x, int64_t n, int32_t lanes, int32_t* sum_out) {
  if (lanes > 2 && lanes <= 16 && n >= 4 * (int64_t)lanes) {
    uint32_t acc[16] = {0};
    const int64_t W = lanes;
    int64_t index = 0;
    int64_t limit = n - 4 * W;
    do {
      uint32_t tracking = 0;
      for (int u = 0; u < 4; ++u)
        for (int64_t l = 0; l < W; ++l) {
          const uint32_t a = acc[l], d = (uint32_t)x[index + u * W + l], r = a + d;
          tracking |= (r ^ a) & (r ^ d);
          acc[l] = r;
        }
      if (tracking >> 31) return DC_ERR_OVERFLOW;
      index += 4 * W;
    } while (index < limit);
    limit = n - W;
    if (index < limit) {
      uint32_t tracking = 0;
      do {
        for (int64_t l = 0; l < W; ++l) {
          const uint32_t a = acc[l], d = (uint32_t)x[index + l], r = a + d;
          tracking |= (r ^ a) & (r ^ d);
          acc[l] = r;
        }
        index += W;
      } while (index < limit);
      if (tracking >> 31) return DC_ERR_OVERFLOW;
    }
    int64_t result = 0;
    for (int64_t l = 0; l < W; ++l) {
      result += (int32_t)acc[l];
      if (result > 2147483647LL || result < -2147483648LL) return DC_ERR_OVERFLOW;
    }
    for (; index < n; ++index) {
      result += x[index];
      if (result > 2147483647LL || result < -2147483648LL) return DC_ERR_OVERFLOW;
    }
    if (sum_out) *sum_out = (int32_t)result;
    return DC_OK;
  }
  return oracle_sum_i32_checked(x, n, sum_out);
}

int64_t oracle_sum_i32_exact(const int32_t* x, int64_t n) {
  int64_t s = 0;
  for (int64_t i = 0; i < n; ++i) s += x[i];
  return s;
}

/* ------------------------------------------------------------------------------------------ */
/* LINQ Where -> Select                                                                         */
/* ------------------------------------------------------------------------------------------ */

/* The configuration's chain written out by hand, as LINQ-to-objects evaluates it after
 * ComputeQueryProvider.ExecuteTyped falls back (ComputeQueryableExtensions.cs:346-352 ->
 * ExecuteFallback :628-633 -> Enumerable.Where(...).Select(...).ToArray()): elements visited in
 * order, `x > 0f` keeps (so -0 and +0 are dropped), `x * 2f + 1f` rounds after each operation. */
int64_t oracle_where_gt0_select_2x_plus_1(const float* in, int64_t n, float* out) {
  int64_t k = 0;
  for (int64_t i = 0; i < n; ++i) {
    float x = in[i];
    if (x > 0.0f) {
      float t = x * 2.0f;
      out[k++] = t + 1.0f;
    }
  }
  return k;
}

/* .Where(x > 0f).Select(x * 2f + 1f).Sum(): Enumerable.Sum over the iterator chain (double
 * accumulator, float result), ComputeQueryableExtensions.cs:265-267. */
float oracle_where_gt0_select_2x_plus_1_sum(const float* in, int64_t n, int64_t* count, double* as_double) {
  double s = 0.0;
  int64_t k = 0;
  for (int64_t i = 0; i < n; ++i) {
    float x = in[i];
    if (x > 0.0f) {
      float t = x * 2.0f;
      float y = t + 1.0f;
      s += (double)y;
      ++k;
    }
  }
  if (count) *count = k;
  if (as_double) *as_double = s;
  return (float)s;
}

/* MathF.Min/MathF.Max (.NET Core 3.0+): IEEE 754-2019 minimum/maximum, NaN-propagating and
 * ordering -0 below +0. */
static float net_min(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  if (a == b) return signbit(a) ? a : b;
  return a < b ? a : b;
}
static float net_max(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  if (a == b) return signbit(a) ? b : a;
  return a > b ? a : b;
}

/* Reference interpreter of the dc_linq_chain register program for ONE element (the program model
 * is documented in include/dotcompute_hip.h). Returns 1 if the element is kept, 0 if filtered,
 * negative on a malformed program. */
int32_t oracle_linq_eval(const dc_linq_chain* chain, float x, float* y_out) {
  float e = x, v = 0.0f, s0 = 0.0f, s1 = 0.0f;
  int p = 0, q = 0, keep = 1;
  if (!chain || chain->n_instr < 0 || chain->n_instr > DC_LINQ_MAX_INSTR) return DC_ERR_INVALID_ARGUMENT;
  for (int32_t pc = 0; pc < chain->n_instr; ++pc) {
    const dc_linq_instr* in = &chain->code[pc];
    float o;
    switch (in->src) {
      case DC_LQ_SRC_IMM: o = in->imm; break;
      case DC_LQ_SRC_ELEM: o = e; break;
      case DC_LQ_SRC_S0: o = s0; break;
      case DC_LQ_SRC_S1: o = s1; break;
      default: return DC_ERR_INVALID_ARGUMENT;
    }
    int c = 0, is_cmp = 0;
    switch (in->op) {
      case DC_LQ_NOP: break;
      case DC_LQ_LOAD: v = o; break;
      case DC_LQ_ADD: v = v + o; break;
      case DC_LQ_SUB: v = v - o; break;
      case DC_LQ_RSUB: v = o - v; break;
      case DC_LQ_MUL: v = v * o; break;
      case DC_LQ_DIV: v = v / o; break;
      case DC_LQ_RDIV: v = o / v; break;
      case DC_LQ_MIN: v = net_min(v, o); break;
      case DC_LQ_MAX: v = net_max(v, o); break;
      case DC_LQ_NEG: v = -v; break;
      case DC_LQ_ABS: v = fabsf(v); break;
      case DC_LQ_SQRT: v = sqrtf(v); break;
      case DC_LQ_REM: v = fmodf(v, o); break;   /* C# float %: truncated remainder, exact */
      case DC_LQ_RREM: v = fmodf(o, v); break;
      case DC_LQ_FLOOR: v = floorf(v); break;   /* MathF.Floor */
      case DC_LQ_CEIL: v = ceilf(v); break;     /* MathF.Ceiling */
      case DC_LQ_ROUND: v = rintf(v); break;    /* MathF.Round: to nearest, ties to even */
      case DC_LQ_POW: v = powf(v, o); break;    /* MathF.Pow calls the C runtime's powf */
      case DC_LQ_RPOW: v = powf(o, v); break;
      case DC_LQ_STORE_S0: s0 = v; break;
      case DC_LQ_STORE_S1: s1 = v; break;
      case DC_LQ_CMP_GT: c = v > o; is_cmp = 1; break;
      case DC_LQ_CMP_GE: c = v >= o; is_cmp = 1; break;
      case DC_LQ_CMP_LT: c = v < o; is_cmp = 1; break;
      case DC_LQ_CMP_LE: c = v <= o; is_cmp = 1; break;
      case DC_LQ_CMP_EQ: c = v == o; is_cmp = 1; break;
      case DC_LQ_CMP_NE: c = v != o; is_cmp = 1; break;
      case DC_LQ_PNOT: p = !p; break;
      case DC_LQ_PSTORE: q = p; break;
      case DC_LQ_PAND_Q: p = p && q; break;
      case DC_LQ_POR_Q: p = p || q; break;
      case DC_LQ_FILTER: keep = keep && p; break;
      case DC_LQ_MAP: e = v; break;
      default: return DC_ERR_INVALID_ARGUMENT;
    }
    if (is_cmp) {
      if (in->mode == DC_LQ_CMP_SET) p = c;
      else if (in->mode == DC_LQ_CMP_AND) p = p && c;
      else if (in->mode == DC_LQ_CMP_OR) p = p || c;
      else return DC_ERR_INVALID_ARGUMENT;
    }
  }
  if (y_out) *y_out = e;
  return keep;
}

/* LINQ-to-objects Where/Select chain (ComputeQueryableExtensions.cs:628-633): order-preserving
 * compaction of the kept, mapped elements. Returns the count, or a negative status. */
int64_t oracle_linq_where_select(const dc_linq_chain* chain, const float* in, int64_t n, float* out) {
  int64_t k = 0;
  for (int64_t i = 0; i < n; ++i) {
    float y;
    int32_t r = oracle_linq_eval(chain, in[i], &y);
    if (r < 0) return r;
    if (r) out[k++] = y;
  }
  return k;
}

float oracle_linq_where_select_sum(const dc_linq_chain* chain, const float* in, int64_t n,
                                   int64_t* count, double* as_double) {
  double s = 0.0;
  int64_t k = 0;
  for (int64_t i = 0; i < n; ++i) {
    float y;
    int32_t r = oracle_linq_eval(chain, in[i], &y);
    if (r < 0) { if (count) *count = r; return 0.0f; }
    if (r) { s += (double)y; ++k; }
  }
  if (count) *count = k;
  if (as_double) *as_double = s;
  return (float)s;
}

/* ---- int32 chains: C# `int` arithmetic (ECMA-334 12.10 / 12.12, unchecked context) ---------
 * + - * and unary - wrap modulo 2^32; / and % truncate toward zero (ECMA-335 III.3.31 div,
 * III.3.55 rem) and throw DivideByZeroException for a zero divisor and an ArithmeticException
 * (OverflowException on x64 .NET) for int.MinValue / -1 and int.MinValue % -1; Math.Abs(int)
 * throws OverflowException for int.MinValue; Math.Min/Max(int, int). Elements are evaluated one at
 * a time, stage by stage, and an element dropped by a Where stage is not evaluated further (the
 * iterator never passes it to the next stage), as LINQ-to-objects runs the chain
 * (ComputeQueryableExtensions.cs:628-633). The reference's generator types `int` lambdas this way
 * (CodeGeneration/CudaKernelGenerator.cs:1351 `%`, :1399-1416 `int`). */
static int32_t wrap32(int64_t v) { return (int32_t)(uint32_t)(uint64_t)v; }

int32_t oracle_linq_eval_i32(const dc_linq_chain* chain, int32_t x, int32_t* y_out, int32_t* fault_out) {
  int32_t e = x, v = 0, s0 = 0, s1 = 0;
  int p = 0, q = 0, keep = 1;
  if (fault_out) *fault_out = 0;
  if (!chain || chain->n_instr < 0 || chain->n_instr > DC_LINQ_MAX_INSTR) return DC_ERR_INVALID_ARGUMENT;
  for (int32_t pc = 0; pc < chain->n_instr && keep; ++pc) {
    const dc_linq_instr* in = &chain->code[pc];
    int32_t o;
    switch (in->src) {
      case DC_LQ_SRC_IMM: o = in->imm_i32; break;
      case DC_LQ_SRC_ELEM: o = e; break;
      case DC_LQ_SRC_S0: o = s0; break;
      case DC_LQ_SRC_S1: o = s1; break;
      default: return DC_ERR_INVALID_ARGUMENT;
    }
    int c = 0, is_cmp = 0;
    int32_t num = 0, den = 1;
    switch (in->op) {
      case DC_LQ_NOP: break;
      case DC_LQ_LOAD: v = o; break;
      case DC_LQ_ADD: v = wrap32((int64_t)v + o); break;
      case DC_LQ_SUB: v = wrap32((int64_t)v - o); break;
      case DC_LQ_RSUB: v = wrap32((int64_t)o - v); break;
      case DC_LQ_MUL: v = wrap32((int64_t)v * o); break;
      case DC_LQ_DIV: case DC_LQ_REM: num = v; den = o; break;
      case DC_LQ_RDIV: case DC_LQ_RREM: num = o; den = v; break;
      case DC_LQ_MIN: v = v < o ? v : o; break;
      case DC_LQ_MAX: v = v > o ? v : o; break;
      case DC_LQ_NEG: v = wrap32(-(int64_t)v); break;
      case DC_LQ_ABS:
        if (v == INT32_MIN) { if (fault_out) *fault_out = DC_LINQ_FAULT_OVERFLOW; return 0; }
        v = v < 0 ? -v : v;
        break;
      case DC_LQ_STORE_S0: s0 = v; break;
      case DC_LQ_STORE_S1: s1 = v; break;
      case DC_LQ_CMP_GT: c = v > o; is_cmp = 1; break;
      case DC_LQ_CMP_GE: c = v >= o; is_cmp = 1; break;
      case DC_LQ_CMP_LT: c = v < o; is_cmp = 1; break;
      case DC_LQ_CMP_LE: c = v <= o; is_cmp = 1; break;
      case DC_LQ_CMP_EQ: c = v == o; is_cmp = 1; break;
      case DC_LQ_CMP_NE: c = v != o; is_cmp = 1; break;
      case DC_LQ_PNOT: p = !p; break;
      case DC_LQ_PSTORE: q = p; break;
      case DC_LQ_PAND_Q: p = p && q; break;
      case DC_LQ_POR_Q: p = p || q; break;
      case DC_LQ_FILTER: keep = keep && p; break;
      case DC_LQ_MAP: e = v; break;
      default: return DC_ERR_UNSUPPORTED; /* SQRT, FLOOR, CEIL, ROUND, POW: no int form */
    }
    if (in->op == DC_LQ_DIV || in->op == DC_LQ_RDIV || in->op == DC_LQ_REM || in->op == DC_LQ_RREM) {
      if (den == 0) { if (fault_out) *fault_out = DC_LINQ_FAULT_DIVIDE_BY_ZERO; return 0; }
      if (den == -1 && num == INT32_MIN) { if (fault_out) *fault_out = DC_LINQ_FAULT_OVERFLOW; return 0; }
      v = (in->op == DC_LQ_DIV || in->op == DC_LQ_RDIV) ? num / den : num % den; /* C99: truncation */
    }
    if (is_cmp) {
      if (in->mode == DC_LQ_CMP_SET) p = c;
      else if (in->mode == DC_LQ_CMP_AND) p = p && c;
      else if (in->mode == DC_LQ_CMP_OR) p = p || c;
      else return DC_ERR_INVALID_ARGUMENT;
    }
  }
  if (y_out) *y_out = e;
  return keep;
}

/* Runs element i; returns 1 kept, 0 dropped, or -1 when it throws (then *fault = 4 i + kind). */
static int eval_i32_at(const dc_linq_chain* chain, const int32_t* in, int64_t i, int32_t* y, int64_t* fault) {
  int32_t kind = 0;
  const int32_t r = oracle_linq_eval_i32(chain, in[i], y, &kind);
  if (r < 0) { *fault = r; return -2; }
  if (kind) { *fault = 4 * i + kind; return -1; }
  return r;
}

int64_t oracle_linq_where_select_i32(const dc_linq_chain* chain, const int32_t* in, int64_t n, int32_t* out,
                                     int64_t* fault_out) {
  int64_t k = 0, fault = DC_LINQ_FAULT_NONE;
  for (int64_t i = 0; i < n; ++i) {
    int32_t y;
    const int r = eval_i32_at(chain, in, i, &y, &fault);
    if (r == -2) return fault;
    if (r < 0) break;
    if (r) out[k++] = y;
  }
  if (fault_out) *fault_out = fault;
  return k;
}

/* Enumerable.Sum(IEnumerable<int>) over the Where/Select iterator (no span): `checked(sum += x)`
 * element by element. Up to the first element that throws (*fault_out = its code, else -1):
 * *total_out = the exact int64 sum of the kept, mapped elements, *overflow_out = 1 if the checked
 * int32 running total left int32 at some element. Returns the kept count. The exception C# raises
 * is the earlier of the two events; a caller that needs it checks the overflow on the elements
 * before the fault (oracle_linq_where_select_sum_i32 over n = fault index). */
int64_t oracle_linq_where_select_sum_i32(const dc_linq_chain* chain, const int32_t* in, int64_t n,
                                         int64_t* total_out, int32_t* overflow_out, int64_t* fault_out) {
  int64_t k = 0, s = 0, fault = DC_LINQ_FAULT_NONE;
  int32_t ovf = 0;
  for (int64_t i = 0; i < n; ++i) {
    int32_t y;
    const int r = eval_i32_at(chain, in, i, &y, &fault);
    if (r == -2) return fault;
    if (r < 0) break;
    if (r) {
      s += y;
      if (s < INT32_MIN || s > INT32_MAX) ovf = 1;
      ++k;
    }
  }
  if (total_out) *total_out = s;
  if (overflow_out) *overflow_out = ovf;
  if (fault_out) *fault_out = fault;
  return k;
}

/* Enumerable.Min / Max(IEnumerable<int>) (op 0 = Min, 1 = Max): the smallest / largest kept,
 * mapped element up to the first throwing element. Returns the kept count (0 = empty sequence). */
int64_t oracle_linq_where_select_minmax_i32(const dc_linq_chain* chain, const int32_t* in, int64_t n, int32_t op,
                                            int32_t* value_out, int64_t* fault_out) {
  int64_t k = 0, fault = DC_LINQ_FAULT_NONE;
  int32_t best = 0;
  for (int64_t i = 0; i < n; ++i) {
    int32_t y;
    const int r = eval_i32_at(chain, in, i, &y, &fault);
    if (r == -2) return fault;
    if (r < 0) break;
    if (r) {
      if (k == 0 || (op == 0 ? y < best : y > best)) best = y;
      ++k;
    }
  }
  if (value_out) *value_out = best;
  if (fault_out) *fault_out = fault;
  return k;
}

/* BCL Enumerable.Min / Max(IEnumerable<float>), .NET 10 (global.json:3-4), as one step per kept,
 * mapped element. `k` counts the elements seen, so an empty sequence is visible to the caller.
 * Min: the enumerator loop stops at the first NaN (`stopped`), else the first smallest wins.
 * Max: leading NaNs are replaced by the next element; after the first non-NaN value only a
 * strictly larger element replaces it. */
typedef struct {
  int64_t k;
  float value;
  int stopped;
} bcl_extreme;

static inline void bcl_min_step(bcl_extreme* s, float x) {
  if (s->k++ == 0) {
    s->value = x;
    if (isnan(x)) s->stopped = 1;
    return;
  }
  if (s->stopped) return;
  if (x < s->value) s->value = x;
  else if (isnan(x)) { s->value = x; s->stopped = 1; }
}

static inline void bcl_max_step(bcl_extreme* s, float x) {
  if (s->k++ == 0 || isnan(s->value)) { s->value = x; return; }
  if (x > s->value) s->value = x;
}

int64_t oracle_linq_where_select_min(const dc_linq_chain* chain, const float* in, int64_t n, float* out) {
  bcl_extreme s = {0, 0.0f, 0};
  for (int64_t i = 0; i < n; ++i) {
    float x;
    int32_t r = oracle_linq_eval(chain, in[i], &x);
    if (r < 0) return r;
    if (r) bcl_min_step(&s, x);
  }
  if (out) *out = s.value;
  return s.k;
}

int64_t oracle_linq_where_select_max(const dc_linq_chain* chain, const float* in, int64_t n, float* out) {
  bcl_extreme s = {0, 0.0f, 0};
  for (int64_t i = 0; i < n; ++i) {
    float x;
    int32_t r = oracle_linq_eval(chain, in[i], &x);
    if (r < 0) return r;
    if (r) bcl_max_step(&s, x);
  }
  if (out) *out = s.value;
  return s.k;
}

/* Enumerable.Aggregate(func) with func = (acc, x) => MathF.Min(acc, x) (op 0) or MathF.Max (op 1)
 * over the kept, mapped elements (Aggregate maps to Reduce, ExpressionTreeVisitor.cs:263): the
 * accumulator starts as the first element and takes func(acc, x) for each later one, in sequence
 * order. net_min / net_max are MathF.Min / MathF.Max (NaN if either is NaN, -0 below +0). */
int64_t oracle_linq_where_select_fold(const dc_linq_chain* chain, const float* in, int64_t n, int32_t op, float* out) {
  int64_t k = 0;
  float acc = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    float x;
    int32_t r = oracle_linq_eval(chain, in[i], &x);
    if (r < 0) return r;
    if (!r) continue;
    acc = k++ == 0 ? x : (op == 0 ? net_min(acc, x) : net_max(acc, x));
  }
  if (out) *out = acc;
  return k;
}

/* .Where(x > 0f).Select(x * 2f + 1f).Min() / .Max() with the lambdas written out, as the
 * LINQ-to-objects fallback runs them (ComputeQueryableExtensions.cs:265-267): the same steps as
 * above without the chain interpreter. op 0 = Min, 1 = Max. */
int64_t oracle_where_gt0_select_2x_plus_1_minmax(const float* in, int64_t n, int32_t op, float* out) {
  bcl_extreme s = {0, 0.0f, 0};
  for (int64_t i = 0; i < n; ++i) {
    float x = in[i];
    if (x > 0.0f) {
      float t = x * 2.0f;
      float y = t + 1.0f;
      if (op == 0) bcl_min_step(&s, y);
      else bcl_max_step(&s, y);
    }
  }
  if (out) *out = s.value;
  return s.k;
}

/* ------------------------------------------------------------------------------------------ */
/* GEMM                                                                                          */
/* ------------------------------------------------------------------------------------------ */

typedef struct {
  const float* a; const float* b; float* c;
  int64_t n, k, r0, r1;
} gemm_arg;

static void* gemm_worker(void* p) {
  gemm_arg* g = (gemm_arg*)p;
  for (int64_t i = g->r0; i < g->r1; ++i) {
    for (int64_t j = 0; j < g->n; ++j) {
      float sum = 0.0f;
      for (int64_t l = 0; l < g->k; ++l) sum += g->a[i * g->k + l] * g->b[l * g->n + j];
      g->c[i * g->n + j] = sum;
    }
  }
  return NULL;
}

/* OptimizedMatrixMultiplyKernel: Parallel.For over rows i, then j, then a sequential fp32
 * `sum += A[i*n+k] * B[k*n+j]` (src/Backends/DotCompute.Backends.CPU/Kernels/Optimized/
 * OptimizedMatrixMultiplyKernel.cs:72-96; square there, general m×k·k×n here). Rows
 * [row_begin, row_end) only, split over `threads` threads. */
void oracle_gemm_f32_naive_rows(const float* a, const float* b, float* c, int64_t m, int64_t n,
                                int64_t k, int64_t row_begin, int64_t row_end, int32_t threads) {
  (void)m;
  if (threads < 1) threads = 1;
  int64_t rows = row_end - row_begin;
  if (rows <= 0) return;
  if (threads > rows) threads = (int32_t)rows;
  gemm_arg* args = (gemm_arg*)calloc((size_t)threads, sizeof(gemm_arg));
  pthread_t* th = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
  for (int32_t t = 0; t < threads; ++t) {
    args[t] = (gemm_arg){a, b, c, n, k, row_begin + rows * t / threads, row_begin + rows * (t + 1) / threads};
    pthread_create(&th[t], NULL, gemm_worker, &args[t]);
  }
  for (int32_t t = 0; t < threads; ++t) pthread_join(th[t], NULL);
  free(args);
  free(th);
}

void oracle_gemm_f32_naive(const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k,
                           int32_t threads) {
  oracle_gemm_f32_naive_rows(a, b, c, m, n, k, 0, m, threads);
}

/* MatrixOperations.MultiplyBlocked: 64-blocked i0/j0/k0 loops; the running result[i,j] carries
 * across k-blocks, so each entry is still a sequential-k fp32 sum
 * (src/Extensions/DotCompute.Algorithms/LinearAlgebra/Operations/MatrixOperations.cs:570-612). */
void oracle_gemm_f32_blocked(const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k) {
  const int64_t B = 64;
  for (int64_t i = 0; i < m * n; ++i) c[i] = 0.0f;
  for (int64_t i0 = 0; i0 < m; i0 += B)
    for (int64_t j0 = 0; j0 < n; j0 += B)
      for (int64_t k0 = 0; k0 < k; k0 += B) {
        int64_t im = i0 + B < m ? i0 + B : m;
        int64_t jm = j0 + B < n ? j0 + B : n;
        int64_t km = k0 + B < k ? k0 + B : k;
        for (int64_t i = i0; i < im; ++i)
          for (int64_t j = j0; j < jm; ++j) {
            float sum = c[i * n + j];
            for (int64_t l = k0; l < km; ++l) sum += a[i * k + l] * b[l * n + j];
            c[i * n + j] = sum;
          }
      }
}

typedef struct {
  const float* a; const float* b; double* c; double* abs_c;
  int64_t n, k; const int64_t* rows; int64_t r0, r1;
} gemm64_arg;

static void* gemm64_worker(void* p) {
  gemm64_arg* g = (gemm64_arg*)p;
  double* acc = (double*)calloc((size_t)g->n, sizeof(double));
  double* aacc = (double*)calloc((size_t)g->n, sizeof(double));
  for (int64_t t = g->r0; t < g->r1; ++t) {
    int64_t i = g->rows[t];
    memset(acc, 0, sizeof(double) * (size_t)g->n);
    memset(aacc, 0, sizeof(double) * (size_t)g->n);
    for (int64_t l = 0; l < g->k; ++l) {
      double av = (double)g->a[i * g->k + l];
      const float* brow = g->b + l * g->n;
      for (int64_t j = 0; j < g->n; ++j) {
        double bv = (double)brow[j];
        acc[j] += av * bv;
        aacc[j] += fabs(av * bv);
      }
    }
    memcpy(g->c + t * g->n, acc, sizeof(double) * (size_t)g->n);
    if (g->abs_c) memcpy(g->abs_c + t * g->n, aacc, sizeof(double) * (size_t)g->n);
  }
  free(acc);
  free(aacc);
  return NULL;
}

/* float64 GEMM rows (the tolerance reference): row t of the output holds row rows[t] of A·B, and
 * abs_c the matching row of |A|·|B| for the per-entry bound. */
void oracle_gemm_f64_rows(const float* a, const float* b, double* c, double* abs_c, int64_t m,
                          int64_t n, int64_t k, const int64_t* rows, int64_t n_rows, int32_t threads) {
  (void)m;
  if (threads < 1) threads = 1;
  if (threads > n_rows) threads = (int32_t)(n_rows > 0 ? n_rows : 1);
  gemm64_arg* args = (gemm64_arg*)calloc((size_t)threads, sizeof(gemm64_arg));
  pthread_t* th = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
  for (int32_t t = 0; t < threads; ++t) {
    args[t] = (gemm64_arg){a, b, c, abs_c, n, k, rows, n_rows * t / threads, n_rows * (t + 1) / threads};
    pthread_create(&th[t], NULL, gemm64_worker, &args[t]);
  }
  for (int32_t t = 0; t < threads; ++t) pthread_join(th[t], NULL);
  free(args);
  free(th);
}

/* IEEE binary32 -> bfloat16, round to nearest even on the dropped 16 bits; NaN stays a quiet NaN. */
uint16_t oracle_f32_to_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void oracle_f32_to_bf16_array(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_bf16(x[i]);
}

/* ------------------------------------------------------------------------------------------ */
/* SpMV                                                                                          */
/* ------------------------------------------------------------------------------------------ */

/* SparseOps.SpMV<T>: throws when A.Columns != x.Length, then per row a sequential
 * `sum += Values[i] * x[ColumnIndices[i]]` in T = float, y[row] = sum
 * (src/Extensions/DotCompute.Algorithms/Sparse/SparseMatrix.cs:669-692). */
int32_t oracle_spmv_csr_f32(const int32_t* row_pointers, const int32_t* col_indices, const float* values,
                            const float* x, float* y, int64_t rows, int64_t cols, int64_t x_len) {
  if (cols != x_len) return DC_ERR_DIMENSION;
  for (int64_t r = 0; r < rows; ++r) {
    float sum = 0.0f;
    for (int32_t i = row_pointers[r]; i < row_pointers[r + 1]; ++i) sum += values[i] * x[col_indices[i]];
    y[r] = sum;
  }
  return DC_OK;
}

void oracle_spmv_csr_f64(const int32_t* row_pointers, const int32_t* col_indices, const float* values,
                         const double* x, double* y, int64_t rows) {
  for (int64_t r = 0; r < rows; ++r) {
    double sum = 0.0;
    for (int32_t i = row_pointers[r]; i < row_pointers[r + 1]; ++i) sum += (double)values[i] * x[col_indices[i]];
    y[r] = sum;
  }
}

/* SparseOps.SpMV<double> (SparseMatrix.cs:669-692 with T = double): per row 0.0 plus each
 * product in index order. */
int32_t oracle_spmv_csr_f64d(const int32_t* row_pointers, const int32_t* col_indices, const double* values,
                             const double* x, double* y, int64_t rows, int64_t cols, int64_t x_len) {
  if (cols != x_len) return DC_ERR_DIMENSION;
  for (int64_t r = 0; r < rows; ++r) {
    double sum = 0.0;
    for (int32_t i = row_pointers[r]; i < row_pointers[r + 1]; ++i) sum += values[i] * x[col_indices[i]];
    y[r] = sum;
  }
  return DC_OK;
}

/* SparseOps.SpMV<int>: C#'s unchecked int multiply and add wrap modulo 2^32. */
int32_t oracle_spmv_csr_i32(const int32_t* row_pointers, const int32_t* col_indices, const int32_t* values,
                            const int32_t* x, int32_t* y, int64_t rows, int64_t cols, int64_t x_len) {
  if (cols != x_len) return DC_ERR_DIMENSION;
  for (int64_t r = 0; r < rows; ++r) {
    uint32_t sum = 0;
    for (int32_t i = row_pointers[r]; i < row_pointers[r + 1]; ++i)
      sum += (uint32_t)values[i] * (uint32_t)x[col_indices[i]];
    y[r] = (int32_t)sum;
  }
  return DC_OK;
}

/* The SpMV benchmark's power iteration: `iterations` times y = SpMV(A, x) (as above), then the
 * L1 normalisation x = y / sum(y) with the sum in float64 and each quotient rounded to float. */
int32_t oracle_spmv_power_f32(const int32_t* row_pointers, const int32_t* col_indices, const float* values,
                              float* x, float* y, int64_t rows, int32_t iterations, double* last_sum) {
  double s = 0.0;
  for (int32_t it = 0; it < iterations; ++it) {
    oracle_spmv_csr_f32(row_pointers, col_indices, values, x, y, rows, rows, rows);
    s = 0.0;
    for (int64_t r = 0; r < rows; ++r) s += (double)y[r];
    for (int64_t r = 0; r < rows; ++r) x[r] = (float)((double)y[r] / s);
  }
  if (last_sum) *last_sum = s;
  return DC_OK;
}

/* ------------------------------------------------------------------------------------------ */
/* [Kernel] sample bodies (dotcompute_amd/kernels/ (*.cs files)) as the reference's CPU backend runs them: */
/* the generated CPU invoker loops __i over [0, work) (work = first writable buffer's length),    */
/* rebuilds the coordinates from the trailing int parameters and runs the body once per work    */
/* item, span accesses bounds-checked (KernelExecutionMetadataEmitter.cs:117-170, 203-245;       */
/* KernelExecutionService.cs:275-288, 382-406). Returns 0, or the DC_GEN_ERR_* + 1 of the first  */
/* exception in loop order.                                                                       */
/* ------------------------------------------------------------------------------------------ */
#define ORC_IDX(len, i) ((uint64_t)(int64_t)(i) < (uint64_t)(len))

/* Math.Min / Math.Max(float) of .NET: IEEE 754-2019 minimum / maximum (NaN wins, -0 < +0). */
float oracle_net_minf(float a, float b) {
  if (a != b) return (a == a) ? (a < b ? a : b) : a;
  return signbit(a) ? a : b;
}
float oracle_net_maxf(float a, float b) {
  if (a != b) return (a == a) ? (b < a ? a : b) : a;
  return signbit(b) ? a : b;
}

/* (long)x for a float x, .NET 9+: truncation, saturating, NaN -> 0. */
int64_t oracle_net_f2l(float x) {
  if (x != x) return 0;
  if (x <= -9223372036854775808.0f) return INT64_MIN;
  if (x >= 9223372036854775808.0f) return INT64_MAX;
  return (int64_t)x;
}

int32_t oracle_kernel_saxpy(const float* x, int64_t nx, float* y, int64_t ny, float a) {
  for (int64_t i = 0; i < ny; ++i) {
    if (!ORC_IDX(nx, i)) return 1;
    y[i] = a * x[i] + y[i];
  }
  return 0;
}

int32_t oracle_kernel_scale_clamp(const float* in, int64_t nin, float* out, int64_t nout, float scale, float lo,
                                  float hi) {
  for (int64_t i = 0; i < nout; ++i) {
    if (!ORC_IDX(nin, i)) return 1;
    const float v = in[i] * scale;
    out[i] = v > 0.0f ? oracle_net_minf(v, hi) : (v < lo ? lo : oracle_net_maxf(v, lo * 0.5f));
  }
  return 0;
}

int32_t oracle_kernel_hash_mix(const uint32_t* keys, int64_t nk, uint32_t* hashes, int64_t nh, uint32_t seed) {
  for (int64_t i = 0; i < nh; ++i) {
    if (!ORC_IDX(nk, i)) return 1;
    uint32_t h = keys[i] ^ seed;
    h ^= h >> 16;
    h *= 0x7feb352du;
    h ^= h >> 15;
    h *= 0x846ca68bu;
    h ^= h >> 16;
    hashes[i] = h;
  }
  return 0;
}

int32_t oracle_kernel_long_mix(const int64_t* a, int64_t na, const float* f, int64_t nf, int64_t* b, int64_t nb,
                               int32_t shift) {
  for (int64_t i = 0; i < nb; ++i) {
    if (!ORC_IDX(na, i)) return 1;
    const uint64_t s = (uint64_t)a[i] << (shift & 63);
    if (!ORC_IDX(nf, i)) return 1;
    const float prod = f[i] * 3.0e18f;
    b[i] = (int64_t)(s + (uint64_t)oracle_net_f2l(prod) + (uint64_t)i);  /* unchecked: wraps */
  }
  return 0;
}

int32_t oracle_kernel_gather(const float* src, int64_t nsrc, const int32_t* index, int64_t nidx, float* dst,
                             int64_t ndst) {
  for (int64_t i = 0; i < ndst; ++i) {
    if (!ORC_IDX(nidx, i)) return 1;
    if (!ORC_IDX(nsrc, index[i])) return 1;
    dst[i] = src[index[i]];
  }
  return 0;
}

int32_t oracle_kernel_int_divide(const int32_t* a, int64_t na, const int32_t* b, int64_t nb, int32_t* q, int64_t nq) {
  for (int64_t i = 0; i < nq; ++i) {
    if (!ORC_IDX(na, i) || !ORC_IDX(nb, i)) return 1;
    if (b[i] == 0) return 2;
    if (b[i] == -1 && a[i] == INT32_MIN) return 3;
    q[i] = a[i] / b[i];
  }
  return 0;
}

int32_t oracle_kernel_transpose(const float* in, int64_t nin, float* out, int64_t nout, int32_t rows, int32_t cols) {
  for (int64_t i = 0; i < nout; ++i) {
    if (cols == 0) return 2;
    const int32_t x = (int32_t)i % cols, y = (int32_t)i / cols;
    if (y < rows && x < cols) {
      const int64_t src = (int64_t)(int32_t)((uint32_t)y * (uint32_t)cols + (uint32_t)x);
      const int64_t dst = (int64_t)(int32_t)((uint32_t)x * (uint32_t)rows + (uint32_t)y);
      if (!ORC_IDX(nin, src) || !ORC_IDX(nout, dst)) return 1;
      out[dst] = in[src];
    }
  }
  return 0;
}

int32_t oracle_kernel_matmul_naive(const float* a, int64_t na, const float* b, int64_t nb, float* c, int64_t nc,
                                   int32_t k, int32_t m, int32_t n) {
  for (int64_t i = 0; i < nc; ++i) {
    if (n == 0) return 2;
    const int32_t col = (int32_t)i % n, row = (int32_t)i / n;
    if (row < m && col < n) {
      float sum = 0.0f;
      for (int32_t p = 0; p < k; ++p) {
        const int64_t ia = (int64_t)row * k + p, ib = (int64_t)p * n + col;
        if (!ORC_IDX(na, ia) || !ORC_IDX(nb, ib)) return 1;
        sum += a[ia] * b[ib];
      }
      const int64_t ic = (int64_t)row * n + col;
      if (!ORC_IDX(nc, ic)) return 1;
      c[ic] = sum;
    }
  }
  return 0;
}

int32_t oracle_kernel_stencil3d(const float* src, int64_t ns, float* dst, int64_t nd, int32_t depth, int32_t height,
                                int32_t width) {
  for (int64_t i = 0; i < nd; ++i) {
    if (width == 0 || height == 0) return 2;
    const int32_t x = (int32_t)i % width, y = ((int32_t)i / width) % height, z = (int32_t)i / (width * height);
    if (x < width && y < height && z < depth) {
      const int64_t idx = ((int64_t)z * height + y) * width + x;
      float left = 0.0f, below = 0.0f;
      if (x > 0) {
        if (!ORC_IDX(ns, idx - 1)) return 1;
        left = src[idx - 1];
      }
      if (z > 0) {
        if (!ORC_IDX(ns, idx - (int64_t)width * height)) return 1;
        below = src[idx - (int64_t)width * height];
      }
      if (!ORC_IDX(ns, idx) || !ORC_IDX(nd, idx)) return 1;
      dst[idx] = src[idx] * 2.0f - left - 0.5f * below;
    }
  }
  return 0;
}
