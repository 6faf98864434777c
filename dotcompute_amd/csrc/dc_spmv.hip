// dc_spmv.hip — CSR SpMV y = A·x (float32) for gfx950, and the normalised power iteration the
// SpMV benchmark runs (y = A·x; x = y / Σy, 20 times).
//
// Work assignment is row-binned, because out-degrees follow a Zipf law (most rows hold 1-8
// nonzeros, a thin tail holds up to 4096):
//   short rows (nnz <= 16·G): a group of G lanes per row (G = smallest power of two >= the mean
//     row length, 4..32). The group's lanes stride the row's nonzeros (coalesced value/column
//     reads across the wave, since a wave covers 64/G consecutive rows) and combine with a
//     butterfly inside the group; lane 0 of the group writes y[row].
//   long rows: found by a classification pass (appended to a list), then one 256-thread
//     workgroup per row with a fixed-order block reduction.
// Each row's sum has a fixed order for a given (G, row length), so results are deterministic.
// The x gathers are served mostly by L2 / MALL (x is 4·cols bytes: 64 MB at 16M rows).
#include <algorithm>

#include "dc_device.hpp"
#include "dc_internal.hpp"

namespace {

constexpr int kBlock = 256;
constexpr int kLongBlock = 256;

template <int G>
__global__ __launch_bounds__(kBlock) void spmv_short_rows(const int32_t* __restrict__ rp, const int32_t* __restrict__ col,
                                                          const float* __restrict__ val, const float* __restrict__ x,
                                                          float* __restrict__ y, int64_t rows, int32_t long_threshold) {
  const int64_t gid = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  const int64_t row = gid / G;
  const int sub = threadIdx.x & (G - 1);
  // Whole groups leave together (row is uniform inside a group), so the butterfly below only
  // ever reads lanes of active groups.
  if (row >= rows) return;
  const int32_t b = rp[row], e = rp[row + 1];
  if (e - b > long_threshold) return;  // written by the long-row pass
  float sum = 0.0f;
  for (int32_t i = b + sub; i < e; i += G) sum += val[i] * x[col[i]];
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off, G);
  if (sub == 0) y[row] = sum;
}

// Appends every row longer than long_threshold to `list`. One atomic per wave (ballot + mbcnt
// give each long row its slot), so the counter is not hammered once per long row.
__global__ __launch_bounds__(kBlock) void spmv_classify(const int32_t* __restrict__ rp, int64_t rows,
                                                        int32_t long_threshold, int32_t* __restrict__ list,
                                                        uint32_t* __restrict__ count) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  const int lane = threadIdx.x & 63;
  // Every lane of a wave runs the same number of iterations (the bound is rounded up to whole
  // strides), so the ballot and the broadcast below always see the full wave.
  const int64_t iters = (rows + stride - 1) / stride;
  for (int64_t it = 0; it < iters; ++it) {
    const int64_t r = it * stride + blockIdx.x * (int64_t)kBlock + threadIdx.x;
    const bool is_long = r < rows && (rp[r + 1] - rp[r] > long_threshold);
    const uint64_t m = __ballot(is_long);
    if (m == 0) continue;
    uint32_t base = 0;
    if (lane == 0)
      base = __hip_atomic_fetch_add(count, (uint32_t)__builtin_popcountll(m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
    if (is_long)
      list[base + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u))] = (int32_t)r;
  }
}

__global__ __launch_bounds__(kLongBlock) void spmv_long_rows(const int32_t* __restrict__ rp, const int32_t* __restrict__ col,
                                                             const float* __restrict__ val, const float* __restrict__ x,
                                                             float* __restrict__ y, const int32_t* __restrict__ list,
                                                             const uint32_t* __restrict__ count) {
  __shared__ float lds[kLongBlock / dc::kWave];
  const uint32_t n_long = *count;
  for (uint32_t t = blockIdx.x; t < n_long; t += gridDim.x) {
    const int32_t row = list[t];
    const int32_t b = rp[row], e = rp[row + 1];
    float sum = 0.0f;
    for (int32_t i = b + (int32_t)threadIdx.x; i < e; i += kLongBlock) sum += val[i] * x[col[i]];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = sum;
    __syncthreads();
    if (threadIdx.x == 0) {
      float total = lds[0];
#pragma unroll
      for (int w = 1; w < kLongBlock / dc::kWave; ++w) total += lds[w];
      y[row] = total;
    }
    __syncthreads();
  }
}

// x[i] = (float)(y[i] / s), s = *sum (float64 division, one rounding to float).
__global__ __launch_bounds__(kBlock) void normalise_kernel(const float* __restrict__ y, float* __restrict__ x, int64_t n,
                                                           const double* __restrict__ sum) {
  const double s = *sum;
  int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (; i < n; i += stride) x[i] = (float)((double)y[i] / s);
}

struct SpmvPlan {
  int group;
  int32_t long_threshold;
  size_t list_cap;
};

SpmvPlan make_plan(int64_t rows, int64_t nnz) {
  const double mean = rows > 0 ? (double)nnz / (double)rows : 1.0;
  int g = 4;
  while (g < 32 && g < mean) g <<= 1;
  SpmvPlan p;
  p.group = g;
  p.long_threshold = 16 * g;
  p.list_cap = (size_t)(nnz / (p.long_threshold + 1) + 1);
  return p;
}

int32_t launch_classify(dc_hip_ctx* ctx, const SpmvPlan& plan, const int32_t* rp, int64_t rows) {
  DC_RETURN_IF(dc::ensure_spmv_rows(ctx, plan.list_cap));
  uint32_t* count = ctx->counters + DC_SLOT_SPMV_LONG;
  DC_RETURN_IF(dc::zero_async(ctx, count, sizeof(uint32_t)));
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((rows + kBlock - 1) / kBlock, 16384));
  spmv_classify<<<grid, kBlock, 0, ctx->stream>>>(rp, rows, plan.long_threshold, ctx->spmv_rows, count);
  return dc::last_launch_status();
}

int32_t launch_spmv(dc_hip_ctx* ctx, const SpmvPlan& plan, const int32_t* rp, const int32_t* col, const float* val,
                    const float* x, float* y, int64_t rows) {
  const int64_t threads = rows * plan.group;
  const unsigned grid = (unsigned)std::max<int64_t>(1, (threads + kBlock - 1) / kBlock);
  switch (plan.group) {
    case 4: spmv_short_rows<4><<<grid, kBlock, 0, ctx->stream>>>(rp, col, val, x, y, rows, plan.long_threshold); break;
    case 8: spmv_short_rows<8><<<grid, kBlock, 0, ctx->stream>>>(rp, col, val, x, y, rows, plan.long_threshold); break;
    case 16: spmv_short_rows<16><<<grid, kBlock, 0, ctx->stream>>>(rp, col, val, x, y, rows, plan.long_threshold); break;
    default: spmv_short_rows<32><<<grid, kBlock, 0, ctx->stream>>>(rp, col, val, x, y, rows, plan.long_threshold); break;
  }
  DC_RETURN_IF(dc::last_launch_status());
  const unsigned lgrid = (unsigned)std::max<size_t>(1, std::min<size_t>(plan.list_cap, 2048));
  spmv_long_rows<<<lgrid, kLongBlock, 0, ctx->stream>>>(rp, col, val, x, y, ctx->spmv_rows,
                                                        ctx->counters + DC_SLOT_SPMV_LONG);
  return dc::last_launch_status();
}

int32_t check_csr(const int32_t* rp, const int32_t* col, const float* val, int64_t rows, int64_t nnz) {
  if (rows < 0 || nnz < 0 || nnz > INT32_MAX || rows >= INT32_MAX) return DC_ERR_INVALID_ARGUMENT;
  if (!rp || (nnz > 0 && (!col || !val))) return DC_ERR_INVALID_ARGUMENT;
  return DC_OK;
}

}  // namespace

extern "C" {

DC_HIP_API int32_t dc_hip_spmv_csr_f32(dc_hip_ctx* ctx, const int32_t* row_pointers, const int32_t* col_indices,
                                       const float* values, const float* x, float* y, int64_t rows, int64_t cols,
                                       int64_t nnz) {
  DC_RETURN_IF(check_csr(row_pointers, col_indices, values, rows, nnz));
  if (cols < 0 || (rows > 0 && !y) || (cols > 0 && !x)) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  if (rows == 0) return DC_OK;
  const SpmvPlan plan = make_plan(rows, nnz);
  DC_RETURN_IF(launch_classify(ctx, plan, row_pointers, rows));
  return launch_spmv(ctx, plan, row_pointers, col_indices, values, x, y, rows);
}

DC_HIP_API int32_t dc_hip_spmv_power_iterate_f32(dc_hip_ctx* ctx, const int32_t* row_pointers,
                                                 const int32_t* col_indices, const float* values, float* x, float* y,
                                                 int64_t rows, int64_t nnz, int32_t iterations, double* last_sum_out) {
  DC_RETURN_IF(check_csr(row_pointers, col_indices, values, rows, nnz));
  if (iterations < 0 || (rows > 0 && (!x || !y))) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  if (rows == 0 || iterations == 0) return DC_OK;
  const SpmvPlan plan = make_plan(rows, nnz);
  DC_RETURN_IF(launch_classify(ctx, plan, row_pointers, rows));
  double* s = ctx->scalars;
  const unsigned ngrid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((rows + kBlock - 1) / kBlock, 16384));
  for (int32_t it = 0; it < iterations; ++it) {
    DC_RETURN_IF(launch_spmv(ctx, plan, row_pointers, col_indices, values, x, y, rows));
    DC_RETURN_IF(dc::launch_reduce_sum_f32(ctx, y, rows, s));
    normalise_kernel<<<ngrid, kBlock, 0, ctx->stream>>>(y, x, rows, s);
    DC_RETURN_IF(dc::last_launch_status());
  }
  if (last_sum_out) DC_RETURN_IF_HIP(hipMemcpyAsync(last_sum_out, s, sizeof(double), hipMemcpyDeviceToDevice, ctx->stream));
  return DC_OK;
}

}  // extern "C"
