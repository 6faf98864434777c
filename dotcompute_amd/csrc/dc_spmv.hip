// dc_spmv.hip — CSR SpMV y = A·x (float32) for gfx950, and the normalised power iteration the
// SpMV benchmark runs (y = A·x; x = y / Σy, 20 times).
//
// Out-degrees follow a Zipf law: most rows hold 1-8 nonzeros, a thin tail holds up to 4096. A
// thread or a small lane group per row would leave most lanes idle and turn every row into a
// chain of dependent, uncoalesced loads, so the work is split by NONZEROS instead:
//   windows: the nonzero array is cut into windows of kWindow entries. Workgroup k owns the rows
//     whose first nonzero lies in window k (row_start[k] = lower_bound(row_pointers, k·kWindow),
//     found once by an analysis pass). It streams the products values[i]·x[col[i]] of those rows
//     into LDS with fully coalesced value/column loads (x is a gather, served mostly by L2 / the
//     256 MB MALL), then one thread per row adds its products in index order — the same order as
//     SparseOps.SpMV (SparseMatrix.cs:669-692), so short rows are bit-identical to the reference.
//   long rows (more than kLongRow nonzeros): listed by a classification pass and handled one
//     workgroup per row with a fixed-order block reduction (deterministic, not sequential order).
// A window's product span is at most kWindow + kLongRow entries (only its last row can run past
// the window, and it is short or excluded), which sizes the LDS buffer.
#include <algorithm>

#include "dc_device.hpp"
#include "dc_internal.hpp"

namespace {

constexpr int kBlock = 256;
constexpr int kWindow = 1024;   // nonzeros per window
constexpr int kLongRow = 512;   // rows longer than this go to the long-row pass
constexpr int kLongBlock = 256;

// row_start[k] = first row whose first nonzero index is >= k·kWindow, for k in [0, windows);
// row_start[windows] = rows.
__global__ __launch_bounds__(kBlock) void spmv_window_starts(const int32_t* __restrict__ rp, int64_t rows,
                                                             int32_t windows, int32_t* __restrict__ row_start) {
  const int64_t k = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (k > windows) return;
  if (k == windows) {
    row_start[k] = (int32_t)rows;
    return;
  }
  const int64_t target = k * (int64_t)kWindow;
  int64_t lo = 0, hi = rows;  // search rp[0..rows]
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)rp[mid] < target) lo = mid + 1; else hi = mid;
  }
  row_start[k] = (int32_t)lo;
}

// Appends every row longer than kLongRow to `list`. One atomic per wave (ballot + mbcnt give each
// long row its slot), so the counter is not hammered once per long row.
__global__ __launch_bounds__(kBlock) void spmv_classify(const int32_t* __restrict__ rp, int64_t rows,
                                                        int32_t* __restrict__ list, uint32_t* __restrict__ count) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  const int lane = threadIdx.x & 63;
  // Every lane of a wave runs the same number of iterations (the bound is rounded up to whole
  // strides), so the ballot and the broadcast below always see the full wave.
  const int64_t iters = (rows + stride - 1) / stride;
  for (int64_t it = 0; it < iters; ++it) {
    const int64_t r = it * stride + blockIdx.x * (int64_t)kBlock + threadIdx.x;
    const bool is_long = r < rows && (rp[r + 1] - rp[r] > kLongRow);
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

__global__ __launch_bounds__(kBlock) void spmv_windows_kernel(const int32_t* __restrict__ rp, const int32_t* __restrict__ col,
                                                              const float* __restrict__ val, const float* __restrict__ x,
                                                              float* __restrict__ y,
                                                              const int32_t* __restrict__ row_start) {
  __shared__ float s_prod[kWindow + kLongRow];
  const int32_t r0 = row_start[blockIdx.x], r1 = row_start[blockIdx.x + 1];
  if (r0 >= r1) return;  // uniform across the workgroup: no row starts in this window
  const int32_t b = rp[r0];
  const int32_t last_begin = rp[r1 - 1], last_end = rp[r1];
  // The last row may run past the window; if it is long it belongs to the long-row pass.
  int32_t e = (last_end - last_begin > kLongRow) ? last_begin : last_end;
  e = min(e, b + kWindow + kLongRow);  // a well-formed CSR never needs this clamp; it keeps LDS in bounds
  // All column/value loads of this thread's slots go out first, then all x gathers, so a window
  // costs two memory round trips instead of two per slot. Values and columns are streamed once
  // (non-temporal); x is what the caches are for.
  constexpr int kSlots = (kWindow + kLongRow) / kBlock;
  int32_t c[kSlots];
  float v[kSlots];
#pragma unroll
  for (int k = 0; k < kSlots; ++k) {
    const int32_t i = b + (int32_t)threadIdx.x + k * kBlock;
    c[k] = 0;
    v[k] = 0.0f;
    if (i < e) {
      c[k] = __builtin_nontemporal_load(col + i);
      v[k] = __builtin_nontemporal_load(val + i);
    }
  }
#pragma unroll
  for (int k = 0; k < kSlots; ++k) {
    const int32_t i = b + (int32_t)threadIdx.x + k * kBlock;
    if (i < e) s_prod[i - b] = v[k] * x[c[k]];
  }
  __syncthreads();
  for (int32_t r = r0 + (int32_t)threadIdx.x; r < r1; r += kBlock) {
    const int32_t rb = rp[r], re = rp[r + 1];
    if (re - rb > kLongRow) continue;
    float sum = 0.0f;
    const int32_t i0 = max(rb - b, 0), i1 = min(re - b, e - b);
    for (int32_t i = i0; i < i1; ++i) sum += s_prod[i];
    __builtin_nontemporal_store(sum, y + r);
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
    // Four slots per pass: their loads and gathers are independent and overlap.
    for (int32_t i0 = b + (int32_t)threadIdx.x; i0 < e; i0 += 4 * kLongBlock) {
      int32_t c[4];
      float v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int32_t i = i0 + k * kLongBlock;
        c[k] = 0;
        v[k] = 0.0f;
        if (i < e) {
          c[k] = __builtin_nontemporal_load(col + i);
          v[k] = __builtin_nontemporal_load(val + i);
        }
      }
      float p[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) p[k] = (i0 + k * kLongBlock < e) ? v[k] * x[c[k]] : 0.0f;
      sum += (p[0] + p[1]) + (p[2] + p[3]);
    }
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
  int32_t windows;
  size_t list_cap;
};

SpmvPlan make_plan(int64_t nnz) {
  SpmvPlan p;
  p.windows = (int32_t)(nnz / kWindow + 1);  // every first-nonzero index in [0, nnz] has a window
  p.list_cap = (size_t)(nnz / (kLongRow + 1) + 1);
  return p;
}

// Analysis: window starts and the long-row list (once per matrix in the power iteration).
int32_t launch_analysis(dc_hip_ctx* ctx, const SpmvPlan& plan, const int32_t* rp, int64_t rows) {
  DC_RETURN_IF(dc::ensure_spmv_rows(ctx, plan.list_cap));
  DC_RETURN_IF(dc::ensure_spmv_windows(ctx, (size_t)plan.windows + 1));
  uint32_t* count = ctx->counters + DC_SLOT_SPMV_LONG;
  DC_RETURN_IF(dc::zero_async(ctx, count, sizeof(uint32_t)));
  const unsigned wgrid = (unsigned)((plan.windows + 1 + kBlock - 1) / kBlock);
  spmv_window_starts<<<wgrid, kBlock, 0, ctx->stream>>>(rp, rows, plan.windows, ctx->spmv_windows);
  DC_RETURN_IF(dc::last_launch_status());
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((rows + kBlock - 1) / kBlock, 16384));
  spmv_classify<<<grid, kBlock, 0, ctx->stream>>>(rp, rows, ctx->spmv_rows, count);
  return dc::last_launch_status();
}

int32_t launch_spmv(dc_hip_ctx* ctx, const SpmvPlan& plan, const int32_t* rp, const int32_t* col, const float* val,
                    const float* x, float* y) {
  spmv_windows_kernel<<<(unsigned)plan.windows, kBlock, 0, ctx->stream>>>(rp, col, val, x, y, ctx->spmv_windows);
  DC_RETURN_IF(dc::last_launch_status());
  const unsigned lgrid = (unsigned)std::max<size_t>(1, std::min<size_t>(plan.list_cap, 2048));
  spmv_long_rows<<<lgrid, kLongBlock, 0, ctx->stream>>>(rp, col, val, x, y, ctx->spmv_rows,
                                                        ctx->counters + DC_SLOT_SPMV_LONG);
  return dc::last_launch_status();
}

int32_t check_csr(const int32_t* rp, const int32_t* col, const float* val, int64_t rows, int64_t nnz) {
  if (rows < 0 || nnz < 0 || nnz > INT32_MAX - 2 * kWindow || rows >= INT32_MAX) return DC_ERR_INVALID_ARGUMENT;
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
  const SpmvPlan plan = make_plan(nnz);
  DC_RETURN_IF(launch_analysis(ctx, plan, row_pointers, rows));
  return launch_spmv(ctx, plan, row_pointers, col_indices, values, x, y);
}

DC_HIP_API int32_t dc_hip_spmv_power_iterate_f32(dc_hip_ctx* ctx, const int32_t* row_pointers,
                                                 const int32_t* col_indices, const float* values, float* x, float* y,
                                                 int64_t rows, int64_t nnz, int32_t iterations, double* last_sum_out) {
  DC_RETURN_IF(check_csr(row_pointers, col_indices, values, rows, nnz));
  if (iterations < 0 || (rows > 0 && (!x || !y))) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  if (rows == 0 || iterations == 0) return DC_OK;
  const SpmvPlan plan = make_plan(nnz);
  DC_RETURN_IF(launch_analysis(ctx, plan, row_pointers, rows));
  double* s = ctx->scalars;
  const unsigned ngrid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((rows + kBlock - 1) / kBlock, 16384));
  for (int32_t it = 0; it < iterations; ++it) {
    DC_RETURN_IF(launch_spmv(ctx, plan, row_pointers, col_indices, values, x, y));
    DC_RETURN_IF(dc::launch_reduce_sum_f32(ctx, y, rows, s));
    normalise_kernel<<<ngrid, kBlock, 0, ctx->stream>>>(y, x, rows, s);
    DC_RETURN_IF(dc::last_launch_status());
  }
  if (last_sum_out) DC_RETURN_IF_HIP(hipMemcpyAsync(last_sum_out, s, sizeof(double), hipMemcpyDeviceToDevice, ctx->stream));
  return DC_OK;
}

}  // extern "C"
