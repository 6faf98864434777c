// dc_streaming.hip — HBM-bound streaming kernels for gfx950: VectorAdd and the deterministic
// float64-accumulated / int64-exact sum reductions.
//
// Layout: inputs are contiguous 1-D arrays in HBM; every thread moves 16-byte vectors
// (global_load_dwordx4) with a grid-stride loop, several loads in flight per thread.
// Reductions: per-thread accumulators in a fixed order -> DPP wave tree -> LDS block tree ->
// per-block partial -> the last block to finish (agent-scope ticket) combines the partials in
// block order. Fixed grid size for a given n, so the result is bit-reproducible run to run.
#include <algorithm>

#include "dc_device.hpp"
#include "dc_internal.hpp"

namespace {

constexpr int kBlock = 256;
constexpr int kUnroll = 4;           // 16-byte loads in flight per thread per iteration
constexpr int kMaxReduceBlocks = 2048;

// ---------------------------------------------------------------------------------------------
// VectorAdd: result[i] = a[i] + b[i] (one rounding per element, bit-exact with any IEEE CPU).
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void vector_add_f32x4_kernel(const dc::f32x4* __restrict__ a,
                                                                  const dc::f32x4* __restrict__ b,
                                                                  dc::f32x4* __restrict__ r, int64_t n4,
                                                                  const float* __restrict__ a_tail,
                                                                  const float* __restrict__ b_tail,
                                                                  float* __restrict__ r_tail, int tail) {
  int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (; i < n4; i += stride) {
    dc::f32x4 x = dc::load_stream(a + i);
    dc::f32x4 y = dc::load_stream(b + i);
    __builtin_nontemporal_store(x + y, r + i);
  }
  if (blockIdx.x == 0 && threadIdx.x < tail) r_tail[threadIdx.x] = a_tail[threadIdx.x] + b_tail[threadIdx.x];
}

__global__ __launch_bounds__(kBlock) void vector_add_f32_kernel(const float* __restrict__ a,
                                                                const float* __restrict__ b,
                                                                float* __restrict__ r, int64_t n) {
  int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (; i < n; i += stride) r[i] = a[i] + b[i];
}

// ---------------------------------------------------------------------------------------------
// Sum reductions.
// ---------------------------------------------------------------------------------------------
__device__ inline double add4(double acc, dc::f32x4 v) {
  acc += (double)v.x;
  acc += (double)v.y;
  acc += (double)v.z;
  acc += (double)v.w;
  return acc;
}
__device__ inline int64_t add4(int64_t acc, dc::i32x4 v) {
  return acc + (int64_t)v.x + (int64_t)v.y + (int64_t)v.z + (int64_t)v.w;
}

template <typename In4, typename In, typename Acc>
__device__ inline Acc thread_partial(const In* __restrict__ x, int64_t n, bool vec_ok) {
  Acc acc0 = 0, acc1 = 0;
  const int64_t tid = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  int64_t done = 0;
  if (vec_ok) {
    const In4* x4 = reinterpret_cast<const In4*>(x);
    const int64_t n4 = n >> 2;
    int64_t i = tid;
    for (; i + (kUnroll - 1) * stride < n4; i += kUnroll * stride) {
      In4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) v[u] = dc::load_stream(x4 + i + u * stride);
#pragma unroll
      for (int u = 0; u < kUnroll; u += 2) {
        acc0 = add4(acc0, v[u]);
        acc1 = add4(acc1, v[u + 1]);
      }
    }
    for (; i < n4; i += stride) acc0 = add4(acc0, dc::load_stream(x4 + i));
    done = n4 << 2;
  }
  for (int64_t i = done + tid; i < n; i += stride) acc1 += (Acc)x[i];
  return acc0 + acc1;
}

// Combine: every block writes its partial; the block that takes the last ticket sums all partials
// in block order (fixed tree), writes the result and returns the ticket counter to zero.
template <typename Acc>
__device__ inline bool last_block_combine(Acc block_total, Acc* __restrict__ partials, uint32_t* __restrict__ done,
                                          Acc* lds, Acc* result) {
  __shared__ bool s_last;
  if (threadIdx.x == 0) {
    partials[blockIdx.x] = block_total;
    dc::fence_release_agent();
    uint32_t t = dc::fetch_add_agent_u32(done, 1u);
    s_last = (t == gridDim.x - 1);
  }
  __syncthreads();
  if (!s_last) return false;
  dc::fence_acquire_agent();
  Acc acc = 0;
  for (unsigned i = threadIdx.x; i < gridDim.x; i += kBlock)
    acc += __hip_atomic_load(partials + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  Acc total = dc::block_sum64<kBlock>(acc, lds);
  if (threadIdx.x == 0) {
    *result = total;
    dc::store_agent_u32(done, 0u);
  }
  return true;
}

__global__ __launch_bounds__(kBlock) void reduce_sum_f32_kernel(const float* __restrict__ x, int64_t n, int vec_ok,
                                                                double* __restrict__ partials,
                                                                uint32_t* __restrict__ done,
                                                                double* __restrict__ out) {
  __shared__ double lds[kBlock / dc::kWave];
  double acc = thread_partial<dc::f32x4, float, double>(x, n, vec_ok != 0);
  double block_total = dc::block_sum64<kBlock>(acc, lds);
  last_block_combine<double>(block_total, partials, done, lds, out);
}

__global__ __launch_bounds__(kBlock) void reduce_sum_i32_kernel(const int32_t* __restrict__ x, int64_t n, int vec_ok,
                                                                int64_t* __restrict__ partials,
                                                                uint32_t* __restrict__ done,
                                                                int64_t* __restrict__ out,
                                                                int32_t* __restrict__ overflow_out) {
  __shared__ int64_t lds[kBlock / dc::kWave];
  int64_t acc = thread_partial<dc::i32x4, int32_t, int64_t>(x, n, vec_ok != 0);
  int64_t block_total = dc::block_sum64<kBlock>(acc, lds);
  __shared__ int64_t s_total;
  if (last_block_combine<int64_t>(block_total, partials, done, lds, &s_total)) {
    if (threadIdx.x == 0) {
      *out = s_total;
      if (overflow_out) *overflow_out = (s_total > 2147483647LL || s_total < -2147483648LL) ? 1 : 0;
    }
  }
}

// Grid for a reduction over n elements: a fixed function of n (not of the device), so results
// are reproducible across runs and devices.
unsigned reduce_grid(int64_t n) {
  int64_t per_block = (int64_t)kBlock * 4 * kUnroll;  // elements one block consumes per iteration
  int64_t g = (n + per_block - 1) / per_block;
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(g, kMaxReduceBlocks));
}

}  // namespace

extern "C" {

DC_HIP_API int32_t dc_hip_vector_add_f32(dc_hip_ctx* ctx, const float* a, const float* b, float* result, int64_t n) {
  if (n < 0 || (n > 0 && (!a || !b || !result))) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  if (n == 0) return DC_OK;
  if (dc::aligned16(a) && dc::aligned16(b) && dc::aligned16(result)) {
    int64_t n4 = n >> 2;
    int tail = (int)(n & 3);
    int64_t blocks = std::max<int64_t>(1, std::min<int64_t>((n4 + kBlock - 1) / kBlock, 8192));
    vector_add_f32x4_kernel<<<(unsigned)blocks, kBlock, 0, ctx->stream>>>(
        reinterpret_cast<const dc::f32x4*>(a), reinterpret_cast<const dc::f32x4*>(b),
        reinterpret_cast<dc::f32x4*>(result), n4, a + (n4 << 2), b + (n4 << 2), result + (n4 << 2), tail);
  } else {
    int64_t blocks = std::max<int64_t>(1, std::min<int64_t>((n + kBlock - 1) / kBlock, 8192));
    vector_add_f32_kernel<<<(unsigned)blocks, kBlock, 0, ctx->stream>>>(a, b, result, n);
  }
  return dc::last_launch_status();
}

DC_HIP_API int32_t dc_hip_reduce_sum_f32(dc_hip_ctx* ctx, const float* input, int64_t n, double* sum_out) {
  if (n < 0 || !sum_out || (n > 0 && !input)) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  unsigned grid = reduce_grid(n);
  DC_RETURN_IF(dc::ensure_partials(ctx, grid * sizeof(double)));
  reduce_sum_f32_kernel<<<grid, kBlock, 0, ctx->stream>>>(input, n, dc::aligned16(input) ? 1 : 0,
                                                          static_cast<double*>(ctx->partials),
                                                          ctx->counters + DC_SLOT_REDUCE_DONE, sum_out);
  return dc::last_launch_status();
}

DC_HIP_API int32_t dc_hip_reduce_sum_i32(dc_hip_ctx* ctx, const int32_t* input, int64_t n, int64_t* sum_out,
                                         int32_t* overflow_out) {
  if (n < 0 || !sum_out || (n > 0 && !input)) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  unsigned grid = reduce_grid(n);
  DC_RETURN_IF(dc::ensure_partials(ctx, grid * sizeof(int64_t)));
  reduce_sum_i32_kernel<<<grid, kBlock, 0, ctx->stream>>>(input, n, dc::aligned16(input) ? 1 : 0,
                                                          static_cast<int64_t*>(ctx->partials),
                                                          ctx->counters + DC_SLOT_REDUCE_DONE, sum_out, overflow_out);
  return dc::last_launch_status();
}

}  // extern "C"
