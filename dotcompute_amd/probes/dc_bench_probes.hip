// dc_bench_probes.hip — measurement-only streaming probes for bench.py, built into
// libdotcompute_bench.so (not part of the product library or its ABI): plain kernels with the
// read/write mixes of the fused LINQ kernels, whose times the benchmark reports as the measured
// streaming ceilings beside the fused kernels. They run on a dc_hip_ctx of libdotcompute_hip.so
// (its stream and lock), so their HIP events line up with the product kernels' on one stream.
#include "dc_bench_probes.h"

#include "../csrc/dc_device.hpp"
#include "../csrc/dc_internal.hpp"

namespace {

constexpr int kVaBlock = 1024;  // the VectorAdd kernel's layout: one 16-byte vector per thread
constexpr int64_t kVaMaxBlocks = 0xFFFFFFFFll / kVaBlock;

__global__ __launch_bounds__(kVaBlock) void probe_copy_kernel(const dc::f32x4* __restrict__ s,
                                                              dc::f32x4* __restrict__ d, int64_t n4) {
  const int64_t stride = (int64_t)gridDim.x * kVaBlock;
  for (int64_t i = (int64_t)blockIdx.x * kVaBlock + threadIdx.x; i < n4; i += stride)
    __builtin_nontemporal_store(dc::load_stream(s + i), d + i);
}
__global__ __launch_bounds__(kVaBlock) void probe_read2_write1_kernel(const dc::f32x4* __restrict__ s,
                                                                      dc::f32x4* __restrict__ d, int64_t h4) {
  const int64_t stride = (int64_t)gridDim.x * kVaBlock;
  for (int64_t i = (int64_t)blockIdx.x * kVaBlock + threadIdx.x; i < h4; i += stride)
    __builtin_nontemporal_store(dc::load_stream(s + i) + dc::load_stream(s + h4 + i), d + i);
}
__global__ __launch_bounds__(kVaBlock) void probe_read_kernel(const dc::f32x4* __restrict__ s,
                                                              dc::f32x4* __restrict__ d, int64_t n4, float never) {
  const int64_t stride = (int64_t)gridDim.x * kVaBlock;
  for (int64_t i = (int64_t)blockIdx.x * kVaBlock + threadIdx.x; i < n4; i += stride) {
    const dc::f32x4 v = dc::load_stream(s + i);
    if (v.x == never || v.y == never || v.z == never || v.w == never) d[0] = v;  // never is NaN
  }
}

}  // namespace

extern "C" {

DC_BENCH_API int32_t dc_bench_stream_probe(dc_hip_ctx* ctx, int32_t kind, const float* src, float* dst, int64_t n) {
  if (n < 0 || (n & 7) != 0 || kind < DC_PROBE_COPY || kind > DC_PROBE_READ) return DC_ERR_INVALID_ARGUMENT;
  if (n > 0 && (!src || !dst)) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  if (n == 0) return DC_OK;
  if (!dc::aligned16(src) || !dc::aligned16(dst)) return DC_ERR_MISALIGNED;
  const auto* s = reinterpret_cast<const dc::f32x4*>(src);
  auto* d = reinterpret_cast<dc::f32x4*>(dst);
  const int64_t v = kind == DC_PROBE_READ2_WRITE1 ? n >> 3 : n >> 2;  // vectors per thread pass
  const unsigned blocks = (unsigned)std::min<int64_t>((v + kVaBlock - 1) / kVaBlock, kVaMaxBlocks);
  if (kind == DC_PROBE_COPY)
    probe_copy_kernel<<<blocks, kVaBlock, 0, ctx->stream>>>(s, d, v);
  else if (kind == DC_PROBE_READ2_WRITE1)
    probe_read2_write1_kernel<<<blocks, kVaBlock, 0, ctx->stream>>>(s, d, v);
  else
    probe_read_kernel<<<blocks, kVaBlock, 0, ctx->stream>>>(s, d, v, __builtin_nanf(""));
  return dc::last_launch_status();
}

}  // extern "C"
