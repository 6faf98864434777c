// dc_runtime.hip — devices, contexts, memory, events, modules, generic launch, seeded generators.
//
// The context replaces what CudaAccelerator owns (device, stream; src/Backends/
// DotCompute.Backends.CUDA/CudaAccelerator.cs:140-146) plus the kernels' scratch. Every entry
// point returns an int32 status (0 = success, hipError_t > 0, DC_ERR_* < 0).
#include <dlfcn.h>
#include <sys/stat.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "dc_device.hpp"
#include "dc_internal.hpp"

namespace {

__global__ void fill_u32_kernel(uint32_t* __restrict__ dst, uint32_t value, int64_t words) {
  int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < words; i += stride) dst[i] = value;
}

__global__ void fill_u8_kernel(uint8_t* __restrict__ dst, uint8_t value, int64_t bytes) {
  int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < bytes; i += stride) dst[i] = value;
}

__global__ void fill_uniform_f32_kernel(float* __restrict__ dst, int64_t n, uint64_t seed, uint32_t stream,
                                        int unit_interval) {
  int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) dst[i] = dc::gen_f32(dc::splitmix64(dc::gen_key(seed, stream, (uint64_t)i)), unit_interval);
}

__global__ void fill_uniform_i32_kernel(int32_t* __restrict__ dst, int64_t n, uint64_t seed, uint32_t stream,
                                        int32_t lo, uint64_t span) {
  int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) dst[i] = dc::gen_i32(dc::splitmix64(dc::gen_key(seed, stream, (uint64_t)i)), lo, span);
}

unsigned grid_for(int64_t items, int block, int64_t max_blocks = 8192) {
  int64_t g = (items + block - 1) / block;
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(g, max_blocks));
}

int32_t fill_bytes(dc_hip_ctx* ctx, void* dst, uint8_t value, size_t bytes) {
  if (bytes == 0) return DC_OK;
  if (!dst) return DC_ERR_INVALID_ARGUMENT;
  uintptr_t p = reinterpret_cast<uintptr_t>(dst);
  if ((p & 3u) == 0 && (bytes & 3u) == 0) {
    uint32_t v = value * 0x01010101u;
    int64_t words = (int64_t)(bytes / 4);
    fill_u32_kernel<<<grid_for(words, 256), 256, 0, ctx->stream>>>(static_cast<uint32_t*>(dst), v, words);
  } else {
    fill_u8_kernel<<<grid_for((int64_t)bytes, 256), 256, 0, ctx->stream>>>(static_cast<uint8_t*>(dst), value,
                                                                           (int64_t)bytes);
  }
  return dc::last_launch_status();
}

}  // namespace

namespace dc {

int32_t zero_async(dc_hip_ctx* ctx, void* dst, size_t bytes) { return fill_bytes(ctx, dst, 0, bytes); }

int32_t ensure_partials(dc_hip_ctx* ctx, size_t bytes) {
  if (ctx->partials_bytes >= bytes) return DC_OK;
  size_t want = std::max<size_t>(bytes, 64 * 1024);
  void* p = nullptr;
  // The old buffer may still be read by queued kernels: wait before releasing it.
  DC_RETURN_IF_HIP(hipStreamSynchronize(ctx->stream));
  if (ctx->partials) DC_RETURN_IF_HIP(hipFree(ctx->partials));
  ctx->partials = nullptr;
  ctx->partials_bytes = 0;
  if (hipMalloc(&p, want) != hipSuccess) return DC_ERR_OUT_OF_MEMORY;
  ctx->partials = p;
  ctx->partials_bytes = want;
  return DC_OK;
}

int32_t ensure_spmv_windows(dc_hip_ctx* ctx, size_t count) {
  if (ctx->spmv_windows_cap >= count) return DC_OK;
  size_t want = std::max<size_t>(count, 4096);
  DC_RETURN_IF_HIP(hipStreamSynchronize(ctx->stream));
  if (ctx->spmv_windows) DC_RETURN_IF_HIP(hipFree(ctx->spmv_windows));
  ctx->spmv_windows = nullptr;
  ctx->spmv_windows_cap = 0;
  void* p = nullptr;
  if (hipMalloc(&p, want * sizeof(int32_t)) != hipSuccess) return DC_ERR_OUT_OF_MEMORY;
  ctx->spmv_windows = static_cast<int32_t*>(p);
  ctx->spmv_windows_cap = want;
  return DC_OK;
}

int32_t ensure_spmv_plan_mem(dc_hip_ctx* ctx, size_t bytes) {
  if (ctx->spmv_plan_bytes >= bytes) return DC_OK;
  DC_RETURN_IF_HIP(hipStreamSynchronize(ctx->stream));
  if (ctx->spmv_plan_mem) DC_RETURN_IF_HIP(hipFree(ctx->spmv_plan_mem));
  ctx->spmv_plan_mem = nullptr;
  ctx->spmv_plan_bytes = 0;
  void* p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess) return DC_ERR_OUT_OF_MEMORY;
  ctx->spmv_plan_mem = p;
  ctx->spmv_plan_bytes = bytes;
  return DC_OK;
}

int32_t ensure_status(dc_hip_ctx* ctx, size_t words, uint32_t* epoch_out) {
  constexpr uint32_t kEpochMask = (1u << 22) - 1;  // 22-bit epoch field in each status word
  if (ctx->status_words < words) {
    size_t want = std::max<size_t>(words, 4096);
    DC_RETURN_IF_HIP(hipStreamSynchronize(ctx->stream));
    if (ctx->status) DC_RETURN_IF_HIP(hipFree(ctx->status));
    ctx->status = nullptr;
    ctx->status_words = 0;
    void* p = nullptr;
    if (hipMalloc(&p, want * sizeof(uint64_t)) != hipSuccess) return DC_ERR_OUT_OF_MEMORY;
    ctx->status = static_cast<uint64_t*>(p);
    ctx->status_words = want;
    DC_RETURN_IF(zero_async(ctx, ctx->status, want * sizeof(uint64_t)));
    ctx->epoch = 0;
  }
  ctx->epoch = (ctx->epoch + 1) & kEpochMask;
  if (ctx->epoch == 0) {  // wrapped: stale words could carry the next epochs; clear and restart at 1
    DC_RETURN_IF(zero_async(ctx, ctx->status, ctx->status_words * sizeof(uint64_t)));
    ctx->epoch = 1;
  }
  *epoch_out = ctx->epoch;
  return DC_OK;
}

int32_t ensure_round_counts(dc_hip_ctx* ctx, size_t words, uint32_t* epoch_out) {
  if (ctx->round_counts_words < words) {
    size_t want = std::max<size_t>(words, 16384);
    DC_RETURN_IF_HIP(hipStreamSynchronize(ctx->stream));
    if (ctx->round_counts) DC_RETURN_IF_HIP(hipFree(ctx->round_counts));
    ctx->round_counts = nullptr;
    ctx->round_counts_words = 0;
    void* p = nullptr;
    if (hipMalloc(&p, want * sizeof(uint32_t)) != hipSuccess) return DC_ERR_OUT_OF_MEMORY;
    ctx->round_counts = static_cast<uint32_t*>(p);
    ctx->round_counts_words = want;
    DC_RETURN_IF(zero_async(ctx, ctx->round_counts, want * sizeof(uint32_t)));
    ctx->round_epoch = 0;
  }
  ctx->round_epoch = (ctx->round_epoch + 1) & 0xFFFFu;
  if (ctx->round_epoch == 0) {  // wrapped: clear so no stale word can match the next epochs
    DC_RETURN_IF(zero_async(ctx, ctx->round_counts, ctx->round_counts_words * sizeof(uint32_t)));
    ctx->round_epoch = 1;
  }
  *epoch_out = ctx->round_epoch;
  return DC_OK;
}

namespace {
struct OrderSlot {
  std::mutex mu;
  dc_hip_ctx* last_ctx = nullptr;  // context whose order event marks the last launch of this kind
};
OrderSlot g_order[DC_ORDER_KINDS][64];
}  // namespace

ResidentLaunch::ResidentLaunch(dc_hip_ctx* ctx, int kind) : ctx_(ctx), kind_(kind) {
  if (ctx->device < 0 || ctx->device >= 64 || kind < 0 || kind >= DC_ORDER_KINDS) {
    status_ = DC_ERR_UNSUPPORTED;
    return;
  }
  OrderSlot& slot = g_order[kind][ctx->device];
  slot.mu.lock();
  mu_ = &slot.mu;
  dc_hip_ctx* prev = slot.last_ctx;
  if (!prev || prev == ctx) return;
  hipError_t e = hipSuccess;
  hipEvent_t& ev = prev->order_done[kind];
  // The no-alloc kind's events exist from context creation (that path creates nothing).
  if (!ev) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventRecord(ev, prev->stream);
  if (e == hipSuccess) e = hipStreamWaitEvent(ctx->stream, ev, 0);
  status_ = (int32_t)e;
}

ResidentLaunch::~ResidentLaunch() {
  if (mu_) mu_->unlock();
}

void ResidentLaunch::done() {
  if (mu_) g_order[kind_][ctx_->device].last_ctx = ctx_;
}

void resident_forget(dc_hip_ctx* ctx) {
  if (ctx->device < 0 || ctx->device >= 64) return;
  for (int kind = 0; kind < DC_ORDER_KINDS; ++kind) {
    OrderSlot& slot = g_order[kind][ctx->device];
    std::lock_guard<std::mutex> lock(slot.mu);
    if (slot.last_ctx == ctx) slot.last_ctx = nullptr;
    if (ctx->order_done[kind]) (void)hipEventDestroy(ctx->order_done[kind]);
    ctx->order_done[kind] = nullptr;
  }
}

}  // namespace dc

extern "C" {

DC_HIP_API const char* dc_hip_error_string(int32_t status) {
  switch (status) {
    case DC_OK: return "success";
    case DC_ERR_INVALID_ARGUMENT: return "invalid argument (null pointer, negative size or bad shape)";
    case DC_ERR_NO_DEVICE: return "no HIP device available (or device index out of range)";
    case DC_ERR_UNSUPPORTED: return "unsupported: device is not gfx950, or the operation/chain is not supported";
    case DC_ERR_OVERFLOW: return "Arithmetic operation resulted in an overflow.";
    case DC_ERR_MISALIGNED: return "pointer alignment requirement not met";
    case DC_ERR_DIMENSION: return "dimension mismatch";
    case DC_ERR_OUT_OF_MEMORY: return "out of memory";
    case DC_ERR_NOT_FOUND: return "module or function not found";
    case DC_ERR_COMPILE: return "run-time compilation of the LINQ program failed";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown DotCompute HIP status";
}

DC_HIP_API int32_t dc_hip_abi_version(void) { return DC_HIP_ABI_VERSION; }

DC_HIP_API int32_t dc_hip_device_count(int32_t* count) {
  if (!count) return DC_ERR_INVALID_ARGUMENT;
  int c = 0;
  hipError_t e = hipGetDeviceCount(&c);
  if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) {
    *count = 0;
    return DC_OK;
  }
  if (e != hipSuccess) {
    *count = 0;
    return (int32_t)e;
  }
  *count = c;
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_device_info_get(int32_t device, dc_hip_device_info* info) {
  if (!info) return DC_ERR_INVALID_ARGUMENT;
  int32_t count = 0;
  DC_RETURN_IF(dc_hip_device_count(&count));
  if (device < 0 || device >= count) return DC_ERR_NO_DEVICE;
  hipDeviceProp_t prop;
  DC_RETURN_IF_HIP(hipGetDeviceProperties(&prop, device));
  std::memset(info, 0, sizeof(*info));
  std::strncpy(info->name, prop.name, sizeof(info->name) - 1);
  std::strncpy(info->gcn_arch_name, prop.gcnArchName, sizeof(info->gcn_arch_name) - 1);
  info->device_id = device;
  info->compute_units = prop.multiProcessorCount;
  info->wave_size = prop.warpSize;
  info->max_threads_per_block = prop.maxThreadsPerBlock;
  info->clock_khz = prop.clockRate;
  info->memory_clock_khz = prop.memoryClockRate;
  info->memory_bus_width_bits = prop.memoryBusWidth;
  info->l2_cache_bytes = prop.l2CacheSize;
  info->total_global_mem = (int64_t)prop.totalGlobalMem;
  info->lds_per_block = (int64_t)prop.sharedMemPerBlock;
  info->pci_bus_id = prop.pciBusID;
  info->is_gfx950 = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_ctx_create(int32_t device, dc_hip_ctx** out) {
  if (!out) return DC_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  dc_hip_device_info info;
  DC_RETURN_IF(dc_hip_device_info_get(device, &info));
  // The kernels are built for gfx950 only; refuse other devices instead of failing at launch.
  if (!info.is_gfx950) return DC_ERR_UNSUPPORTED;
  DC_RETURN_IF_HIP(hipSetDevice(device));
  (void)hipGetLastError();  // start from a clean error slot: the launch checks below read it
  dc_hip_ctx* ctx = new dc_hip_ctx();
  ctx->device = device;
  ctx->cu_count = info.compute_units;
  hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return (int32_t)e;
  }
  void* c = nullptr;
  e = hipMalloc(&c, DC_SLOT_COUNT * sizeof(uint32_t));
  if (e != hipSuccess) {
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return (int32_t)e;
  }
  ctx->counters = static_cast<uint32_t*>(c);
  void* sc = nullptr;
  e = hipMalloc(&sc, 64 * sizeof(double));
  if (e != hipSuccess) {
    (void)hipFree(ctx->counters);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return (int32_t)e;
  }
  ctx->scalars = static_cast<double*>(sc);
  int32_t st = dc::zero_async(ctx, ctx->counters, DC_SLOT_COUNT * sizeof(uint32_t));
  if (st == DC_OK) st = (int32_t)hipStreamSynchronize(ctx->stream);
  if (st != DC_OK) {
    (void)hipFree(ctx->scalars);
    (void)hipFree(ctx->counters);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return st;
  }
  // Set-up of the allocation-free entry point (device current): its status is kept and returned by
  // that entry point, so a failed lookup does not stop the context from serving everything else.
  ctx->noalloc_status = dc::linq_noalloc_setup(ctx);
  if (ctx->noalloc_status == DC_OK)  // the event that orders no-alloc calls across contexts
    ctx->noalloc_status = (int32_t)hipEventCreateWithFlags(&ctx->order_done[dc::kOrderNoAlloc], hipEventDisableTiming);
  *out = ctx;
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_ctx_destroy(dc_hip_ctx* ctx) {
  if (!ctx) return DC_ERR_INVALID_ARGUMENT;
  {
    std::lock_guard<std::mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->partials) (void)hipFree(ctx->partials);
    if (ctx->status) (void)hipFree(ctx->status);
    if (ctx->round_counts) (void)hipFree(ctx->round_counts);
    dc::resident_forget(ctx);
    if (ctx->counters) (void)hipFree(ctx->counters);
    if (ctx->scalars) (void)hipFree(ctx->scalars);
    if (ctx->spmv_windows) (void)hipFree(ctx->spmv_windows);
    if (ctx->spmv_plan_mem) (void)hipFree(ctx->spmv_plan_mem);
    (void)hipStreamDestroy(ctx->stream);
  }
  delete ctx;
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_ctx_device(const dc_hip_ctx* ctx, int32_t* device) {
  if (!ctx || !device) return DC_ERR_INVALID_ARGUMENT;
  *device = ctx->device;
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_synchronize(dc_hip_ctx* ctx) {
  DC_CTX_ENTER(ctx);
  DC_RETURN_IF_HIP(hipStreamSynchronize(ctx->stream));
  return DC_OK;
}

// ---- memory ---------------------------------------------------------------------------------

DC_HIP_API int32_t dc_hip_malloc(dc_hip_ctx* ctx, size_t bytes, void** device_ptr) {
  if (!device_ptr) return DC_ERR_INVALID_ARGUMENT;
  *device_ptr = nullptr;
  DC_CTX_ENTER(ctx);
  if (bytes == 0) return DC_OK;
  hipError_t e = hipMalloc(device_ptr, bytes);
  if (e == hipErrorOutOfMemory) return DC_ERR_OUT_OF_MEMORY;
  DC_RETURN_IF_HIP(e);
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_free(dc_hip_ctx* ctx, void* device_ptr) {
  DC_CTX_ENTER(ctx);
  if (!device_ptr) return DC_OK;
  // Queued kernels may still use the buffer; hipFree itself synchronises the device.
  DC_RETURN_IF_HIP(hipFree(device_ptr));
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_malloc_host(dc_hip_ctx* ctx, size_t bytes, void** host_ptr) {
  if (!host_ptr) return DC_ERR_INVALID_ARGUMENT;
  *host_ptr = nullptr;
  DC_CTX_ENTER(ctx);
  if (bytes == 0) return DC_OK;
  DC_RETURN_IF_HIP(hipHostMalloc(host_ptr, bytes, hipHostMallocDefault));
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_host_device_pointer(dc_hip_ctx* ctx, void* host_ptr, void** device_ptr) {
  if (!host_ptr || !device_ptr) return DC_ERR_INVALID_ARGUMENT;
  *device_ptr = nullptr;
  DC_CTX_ENTER(ctx);
  DC_RETURN_IF_HIP(hipHostGetDevicePointer(device_ptr, host_ptr, 0));
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_free_host(dc_hip_ctx* ctx, void* host_ptr) {
  DC_CTX_ENTER(ctx);
  if (!host_ptr) return DC_OK;
  DC_RETURN_IF_HIP(hipHostFree(host_ptr));
  return DC_OK;
}

static int32_t copy_async(dc_hip_ctx* ctx, void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
  DC_CTX_ENTER(ctx);
  if (bytes == 0) return DC_OK;
  if (!dst || !src) return DC_ERR_INVALID_ARGUMENT;
  DC_RETURN_IF_HIP(hipMemcpyAsync(dst, src, bytes, kind, ctx->stream));
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_memcpy_h2d_async(dc_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  return copy_async(ctx, dst, src, bytes, hipMemcpyHostToDevice);
}
DC_HIP_API int32_t dc_hip_memcpy_d2h_async(dc_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  return copy_async(ctx, dst, src, bytes, hipMemcpyDeviceToHost);
}
DC_HIP_API int32_t dc_hip_memcpy_d2d_async(dc_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  return copy_async(ctx, dst, src, bytes, hipMemcpyDeviceToDevice);
}

DC_HIP_API int32_t dc_hip_memset_async(dc_hip_ctx* ctx, void* dst, int32_t value, size_t bytes) {
  DC_CTX_ENTER(ctx);
  return fill_bytes(ctx, dst, static_cast<uint8_t>(value & 0xFF), bytes);
}

DC_HIP_API int32_t dc_hip_mem_info(dc_hip_ctx* ctx, size_t* free_bytes, size_t* total_bytes) {
  if (!free_bytes || !total_bytes) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  DC_RETURN_IF_HIP(hipMemGetInfo(free_bytes, total_bytes));
  return DC_OK;
}

// ---- events ---------------------------------------------------------------------------------

DC_HIP_API int32_t dc_hip_event_create(dc_hip_ctx* ctx, dc_hip_event** event) {
  if (!event) return DC_ERR_INVALID_ARGUMENT;
  *event = nullptr;
  DC_CTX_ENTER(ctx);
  dc_hip_event* ev = new dc_hip_event();
  ev->device = ctx->device;
  hipError_t e = hipEventCreate(&ev->ev);
  if (e != hipSuccess) {
    delete ev;
    return (int32_t)e;
  }
  *event = ev;
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_event_destroy(dc_hip_event* event) {
  if (!event) return DC_ERR_INVALID_ARGUMENT;
  (void)hipSetDevice(event->device);
  hipError_t e = hipEventDestroy(event->ev);
  delete event;
  return (int32_t)e;
}

DC_HIP_API int32_t dc_hip_event_record(dc_hip_ctx* ctx, dc_hip_event* event) {
  if (!event) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  DC_RETURN_IF_HIP(hipEventRecord(event->ev, ctx->stream));
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_event_synchronize(dc_hip_event* event) {
  if (!event) return DC_ERR_INVALID_ARGUMENT;
  DC_RETURN_IF_HIP(hipSetDevice(event->device));
  DC_RETURN_IF_HIP(hipEventSynchronize(event->ev));
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_event_elapsed_ms(dc_hip_event* start, dc_hip_event* stop, float* ms) {
  if (!start || !stop || !ms) return DC_ERR_INVALID_ARGUMENT;
  DC_RETURN_IF_HIP(hipSetDevice(start->device));
  DC_RETURN_IF_HIP(hipEventElapsedTime(ms, start->ev, stop->ev));
  return DC_OK;
}

// ---- modules and generic launch ---------------------------------------------------------------

DC_HIP_API int32_t dc_hip_module_load(dc_hip_ctx* ctx, const char* path, dc_hip_module** module) {
  if (!path || !module) return DC_ERR_INVALID_ARGUMENT;
  *module = nullptr;
  DC_CTX_ENTER(ctx);
  struct stat st;
  if (stat(path, &st) != 0) return DC_ERR_NOT_FOUND;
  hipModule_t m = nullptr;
  DC_RETURN_IF_HIP(hipModuleLoad(&m, path));
  *module = new dc_hip_module{m, ctx->device};
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_module_load_data(dc_hip_ctx* ctx, const void* image, dc_hip_module** module) {
  if (!image || !module) return DC_ERR_INVALID_ARGUMENT;
  *module = nullptr;
  DC_CTX_ENTER(ctx);
  hipModule_t m = nullptr;
  DC_RETURN_IF_HIP(hipModuleLoadData(&m, image));
  *module = new dc_hip_module{m, ctx->device};
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_module_unload(dc_hip_module* module) {
  if (!module) return DC_ERR_INVALID_ARGUMENT;
  (void)hipSetDevice(module->device);
  hipError_t e = hipModuleUnload(module->mod);
  delete module;
  return (int32_t)e;
}

DC_HIP_API int32_t dc_hip_module_get_function(dc_hip_module* module, const char* name, void** function) {
  if (!module || !name || !function) return DC_ERR_INVALID_ARGUMENT;
  *function = nullptr;
  DC_RETURN_IF_HIP(hipSetDevice(module->device));
  hipFunction_t f = nullptr;
  hipError_t e = hipModuleGetFunction(&f, module->mod, name);
  if (e != hipSuccess) (void)hipGetLastError();  // a failed lookup must not surface in a later call
  if (e == hipErrorNotFound) return DC_ERR_NOT_FOUND;
  DC_RETURN_IF_HIP(e);
  *function = reinterpret_cast<void*>(f);
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_launch_kernel(dc_hip_ctx* ctx, void* function, uint32_t grid_x, uint32_t grid_y,
                                        uint32_t grid_z, uint32_t block_x, uint32_t block_y, uint32_t block_z,
                                        uint32_t shared_mem_bytes, void** args) {
  if (!function) return DC_ERR_INVALID_ARGUMENT;
  if (grid_x == 0 || grid_y == 0 || grid_z == 0 || block_x == 0 || block_y == 0 || block_z == 0)
    return DC_ERR_INVALID_ARGUMENT;
  if ((uint64_t)block_x * block_y * block_z > 1024) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  DC_RETURN_IF_HIP(hipModuleLaunchKernel(reinterpret_cast<hipFunction_t>(function), grid_x, grid_y, grid_z,
                                         block_x, block_y, block_z, shared_mem_bytes, ctx->stream, args,
                                         nullptr));
  return DC_OK;
}

DC_HIP_API const char* dc_hip_default_module_path(void) {
  static std::string path = [] {
    Dl_info info;
    if (dladdr(reinterpret_cast<void*>(&dc_hip_abi_version), &info) == 0 || !info.dli_fname) return std::string();
    std::string lib(info.dli_fname);
    size_t slash = lib.find_last_of('/');
    std::string dir = slash == std::string::npos ? std::string(".") : lib.substr(0, slash);
    std::string p = dir + "/dc_kernels_gfx950.hsaco";
    struct stat st;
    return stat(p.c_str(), &st) == 0 ? p : std::string();
  }();
  return path.c_str();
}

// ---- generators -------------------------------------------------------------------------------

DC_HIP_API int32_t dc_hip_fill_uniform_f32(dc_hip_ctx* ctx, float* dst, int64_t n, uint64_t seed, uint32_t stream,
                                           int32_t unit_interval) {
  if (n < 0 || (n > 0 && !dst)) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  if (n == 0) return DC_OK;
  fill_uniform_f32_kernel<<<grid_for(n, 256, 16384), 256, 0, ctx->stream>>>(dst, n, seed, stream, unit_interval);
  return dc::last_launch_status();
}

DC_HIP_API int32_t dc_hip_fill_uniform_i32(dc_hip_ctx* ctx, int32_t* dst, int64_t n, uint64_t seed, uint32_t stream,
                                           int32_t lo, int32_t hi) {
  if (n < 0 || (n > 0 && !dst) || hi < lo) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  if (n == 0) return DC_OK;
  uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
  fill_uniform_i32_kernel<<<grid_for(n, 256, 16384), 256, 0, ctx->stream>>>(dst, n, seed, stream, lo, span);
  return dc::last_launch_status();
}

DC_HIP_API int32_t dc_gen_uniform_f32(float* dst, int64_t n, uint64_t seed, uint32_t stream, int32_t unit_interval) {
  if (n < 0 || (n > 0 && !dst)) return DC_ERR_INVALID_ARGUMENT;
  for (int64_t i = 0; i < n; ++i) dst[i] = dc::gen_f32(dc::splitmix64(dc::gen_key(seed, stream, (uint64_t)i)), unit_interval);
  return DC_OK;
}

DC_HIP_API int32_t dc_gen_uniform_i32(int32_t* dst, int64_t n, uint64_t seed, uint32_t stream, int32_t lo, int32_t hi) {
  if (n < 0 || (n > 0 && !dst) || hi < lo) return DC_ERR_INVALID_ARGUMENT;
  uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
  for (int64_t i = 0; i < n; ++i) dst[i] = dc::gen_i32(dc::splitmix64(dc::gen_key(seed, stream, (uint64_t)i)), lo, span);
  return DC_OK;
}

static unsigned gen_threads() {
  unsigned t = std::thread::hardware_concurrency();
  return std::max(1u, std::min(t, 16u));
}

DC_HIP_API int32_t dc_gen_zipf_csr_rowptr(int64_t rows, double alpha, int32_t max_degree, uint64_t seed,
                                          int32_t* row_pointers) {
  if (rows < 0 || max_degree < 1 || !row_pointers || !(alpha > 0.0)) return DC_ERR_INVALID_ARGUMENT;
  // Inverse CDF of Zipf(alpha) on [1, max_degree], accumulated in the same order as the CPU checker.
  std::vector<double> cdf((size_t)max_degree + 1);
  double total = 0.0;
  for (int32_t d = 1; d <= max_degree; ++d) total += std::pow((double)d, -alpha);
  double acc = 0.0;
  cdf[0] = 0.0;
  for (int32_t d = 1; d <= max_degree; ++d) {
    acc += std::pow((double)d, -alpha);
    cdf[d] = acc / total;
  }
  cdf[max_degree] = 1.0;
  // Degrees in parallel (counter-based: row r uses stream 3, key r), then a sequential scan.
  std::vector<int32_t> deg((size_t)rows);
  unsigned T = gen_threads();
  std::vector<std::thread> th;
  for (unsigned t = 0; t < T; ++t) {
    th.emplace_back([&, t] {
      int64_t r0 = rows * t / T, r1 = rows * (t + 1) / T;
      for (int64_t r = r0; r < r1; ++r) {
        uint64_t z = dc::splitmix64(dc::gen_key(seed, 3u, (uint64_t)r));
        double u = (double)(z >> 11) * 0x1p-53;
        int32_t lo = 1, hi = max_degree;
        while (lo < hi) {
          int32_t mid = lo + (hi - lo) / 2;
          if (cdf[mid] > u) hi = mid; else lo = mid + 1;
        }
        deg[r] = lo;
      }
    });
  }
  for (auto& x : th) x.join();
  int64_t nnz = 0;
  row_pointers[0] = 0;
  for (int64_t r = 0; r < rows; ++r) {
    nnz += deg[r];
    if (nnz > 2147483647LL) return DC_ERR_OVERFLOW;  // CsrMatrix<T> uses int32 row pointers
    row_pointers[r + 1] = (int32_t)nnz;
  }
  return DC_OK;
}

DC_HIP_API int32_t dc_gen_zipf_csr_fill(int64_t rows, int64_t cols, uint64_t seed, const int32_t* row_pointers,
                                        int32_t* col_indices, float* values) {
  if (rows < 0 || cols < 2 || !row_pointers) return DC_ERR_INVALID_ARGUMENT;
  if (row_pointers[rows] > 0 && (!col_indices || !values)) return DC_ERR_INVALID_ARGUMENT;
  const uint64_t span = (uint64_t)(cols - 1);
  unsigned T = gen_threads();
  std::vector<std::thread> th;
  for (unsigned t = 0; t < T; ++t) {
    th.emplace_back([&, t] {
      int64_t r0 = rows * t / T, r1 = rows * (t + 1) / T;
      for (int64_t r = r0; r < r1; ++r) {
        int32_t b = row_pointers[r], e = row_pointers[r + 1];
        float v = 1.0f / (float)(e - b);
        for (int32_t j = b; j < e; ++j) {
          uint64_t z = dc::splitmix64(dc::gen_key(seed, 4u, (uint64_t)j));
          int64_t c = (int64_t)(((z >> 32) * span) >> 32);
          if (c >= r) c += 1;
          col_indices[j] = (int32_t)c;
          values[j] = v;
        }
      }
    });
  }
  for (auto& x : th) x.join();
  return DC_OK;
}

}  // extern "C"
