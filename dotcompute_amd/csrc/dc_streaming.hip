// dc_streaming.hip — HBM-bound streaming kernels for gfx950: VectorAdd and the deterministic
// float64-accumulated / int64-exact sum reductions.
//
// Layout: inputs are contiguous 1-D arrays in HBM; every thread moves 16-byte vectors
// (global_load_dwordx4) with a grid-stride loop, several loads in flight per thread.
// Reductions: per-thread accumulators in a fixed order -> DPP wave tree -> LDS block tree ->
// per-block partial -> a one-block pass sums the partials in block order. Fixed grid size for a
// given n, so the result is bit-reproducible run to run.
#include <algorithm>
#include <type_traits>

#include "dc_device.hpp"
#include "dc_internal.hpp"

namespace {

constexpr int kBlock = 256;

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
// Sum reductions: pass 1 — each block sums one contiguous chunk of the input (threads stride
// 16-byte vectors through it, kUnroll loads in flight) into a per-block partial; pass 2 — one
// block sums the partials in block order. Two launches instead of a last-block combine: the
// combine would need agent-scope release/acquire fences in every block, which on gfx950 write
// back and invalidate the XCD's L2 and cost more than the second launch (measured at 256M
// elements: 195 us with a last-block combine against 155 us for the two launches).
// ---------------------------------------------------------------------------------------------
constexpr int kRedBlock = 512;
constexpr int kRedUnroll = 8;
constexpr int kFinalBlock = 1024;

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

// Vectors [v0, v1) of this block's chunk; the scalar tail (n % 4 elements) goes to the last block.
template <typename In4, typename In, typename Acc>
__device__ inline Acc chunk_partial(const In* __restrict__ x, int64_t n, bool vec_ok) {
  Acc acc0 = 0, acc1 = 0;
  const int64_t n4 = vec_ok ? (n >> 2) : 0;
  const int64_t per = (n4 + gridDim.x - 1) / gridDim.x;
  const int64_t v0 = min(n4, (int64_t)blockIdx.x * per), v1 = min(n4, v0 + per);
  const In4* x4 = reinterpret_cast<const In4*>(x);
  int64_t i = v0 + threadIdx.x;
  for (; i + (kRedUnroll - 1) * kRedBlock < v1; i += kRedUnroll * kRedBlock) {
    In4 v[kRedUnroll];
#pragma unroll
    for (int u = 0; u < kRedUnroll; ++u) v[u] = dc::load_stream(x4 + i + u * kRedBlock);
#pragma unroll
    for (int u = 0; u < kRedUnroll; u += 2) {
      acc0 = add4(acc0, v[u]);
      acc1 = add4(acc1, v[u + 1]);
    }
  }
  for (; i < v1; i += kRedBlock) acc0 = add4(acc0, dc::load_stream(x4 + i));
  if (blockIdx.x == gridDim.x - 1)
    for (int64_t s = (n4 << 2) + threadIdx.x; s < n; s += kRedBlock) acc1 += (Acc)x[s];
  return acc0 + acc1;
}

__global__ __launch_bounds__(kRedBlock) void reduce_sum_f32_pass1(const float* __restrict__ x, int64_t n, int vec_ok,
                                                                  double* __restrict__ partials) {
  __shared__ double lds[kRedBlock / dc::kWave];
  double acc = chunk_partial<dc::f32x4, float, double>(x, n, vec_ok != 0);
  double t = dc::block_sum64<kRedBlock>(acc, lds);
  if (threadIdx.x == 0) partials[blockIdx.x] = t;
}

__global__ __launch_bounds__(kRedBlock) void reduce_sum_i32_pass1(const int32_t* __restrict__ x, int64_t n, int vec_ok,
                                                                  int64_t* __restrict__ partials) {
  __shared__ int64_t lds[kRedBlock / dc::kWave];
  int64_t acc = chunk_partial<dc::i32x4, int32_t, int64_t>(x, n, vec_ok != 0);
  int64_t t = dc::block_sum64<kRedBlock>(acc, lds);
  if (threadIdx.x == 0) partials[blockIdx.x] = t;
}

// Sums partials[0..count) in a fixed order: thread t takes t, t+1024, ... then the block tree.
template <typename Acc>
__global__ __launch_bounds__(kFinalBlock) void reduce_partials(const Acc* __restrict__ partials, int count,
                                                               Acc* __restrict__ out, int32_t* __restrict__ overflow) {
  __shared__ Acc lds[kFinalBlock / dc::kWave];
  Acc acc = 0;
  // Thread t adds partials t, t + 1024, t + 2048, ... in that order; eight loads go out together.
  for (int i0 = threadIdx.x; i0 < count; i0 += 8 * kFinalBlock) {
    Acc v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = i0 + k * kFinalBlock < count ? partials[i0 + k * kFinalBlock] : Acc(0);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (i0 + k * kFinalBlock < count) acc += v[k];
  }
  Acc total = dc::block_sum64<kFinalBlock>(acc, lds);
  if (threadIdx.x == 0) {
    *out = total;
    if constexpr (std::is_integral<Acc>::value) {
      if (overflow) *overflow = (total > 2147483647LL || total < -2147483648LL) ? 1 : 0;
    }
  }
}

// Grid for a reduction over n elements: a fixed function of n (not of the device), so results
// are reproducible across runs and devices.
unsigned reduce_grid(int64_t n) {
  const int64_t per_block = (int64_t)kRedBlock * 4 * kRedUnroll;  // elements per block-iteration
  const int64_t g = (n + per_block - 1) / per_block;
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(g, 1024));  // 2 workgroups per CU: measured best
}

}  // namespace

namespace dc {

int32_t launch_reduce_sum_f32(dc_hip_ctx* ctx, const float* input, int64_t n, double* sum_out) {
  unsigned grid = reduce_grid(n);
  DC_RETURN_IF(dc::ensure_partials(ctx, grid * sizeof(double)));
  double* partials = static_cast<double*>(ctx->partials);
  reduce_sum_f32_pass1<<<grid, kRedBlock, 0, ctx->stream>>>(input, n, dc::aligned16(input) ? 1 : 0, partials);
  reduce_partials<double><<<1, kFinalBlock, 0, ctx->stream>>>(partials, (int)grid, sum_out, nullptr);
  return dc::last_launch_status();
}

int32_t launch_reduce_partials_f64(dc_hip_ctx* ctx, const double* partials, int count, double* sum_out) {
  reduce_partials<double><<<1, kFinalBlock, 0, ctx->stream>>>(partials, count, sum_out, nullptr);
  return dc::last_launch_status();
}

}  // namespace dc

extern "C" {

DC_HIP_API int32_t dc_hip_vector_add_f32(dc_hip_ctx* ctx, const float* a, const float* b, float* result, int64_t n) {
  if (n < 0 || (n > 0 && (!a || !b || !result))) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  if (n == 0) return DC_OK;
  if (dc::aligned16(a) && dc::aligned16(b) && dc::aligned16(result)) {
    int64_t n4 = n >> 2;
    int tail = (int)(n & 3);
    int64_t blocks = std::max<int64_t>(1, std::min<int64_t>((n4 + kBlock - 1) / kBlock, 32768));
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
  return dc::launch_reduce_sum_f32(ctx, input, n, sum_out);
}

DC_HIP_API int32_t dc_hip_reduce_sum_i32(dc_hip_ctx* ctx, const int32_t* input, int64_t n, int64_t* sum_out,
                                         int32_t* overflow_out) {
  if (n < 0 || !sum_out || (n > 0 && !input)) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  unsigned grid = reduce_grid(n);
  DC_RETURN_IF(dc::ensure_partials(ctx, grid * sizeof(int64_t)));
  int64_t* partials = static_cast<int64_t*>(ctx->partials);
  reduce_sum_i32_pass1<<<grid, kRedBlock, 0, ctx->stream>>>(input, n, dc::aligned16(input) ? 1 : 0, partials);
  reduce_partials<int64_t><<<1, kFinalBlock, 0, ctx->stream>>>(partials, (int)grid, sum_out, overflow_out);
  return dc::last_launch_status();
}

}  // extern "C"
