// dc_internal.hpp — shared host-side state of libdotcompute_hip.so (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <mutex>

#include "../../include/dotcompute_hip.h"

// One device + one in-order stream + the scratch memory the kernels need.
struct dc_hip_ctx {
  int device = 0;
  int cu_count = 0;
  hipStream_t stream = nullptr;
  std::mutex mu;

  // Fixed 4 KiB block of counters (tile tickets, last-block tickets). Zeroed at creation; every
  // kernel that takes a ticket puts its counter back to zero before it exits.
  uint32_t* counters = nullptr;

  // Per-block partial results of the reductions (double or int64 each; grows on demand).
  void* partials = nullptr;
  size_t partials_bytes = 0;

  // SpMV scratch: the list of long rows (handled a workgroup per row) and small device scalars.
  int32_t* spmv_windows = nullptr;  // first row of each nonzero window
  size_t spmv_windows_cap = 0;
  double* scalars = nullptr;  // 64 doubles
  // Device memory of the tiled SpMV plan built by dc_hip_spmv_power_iterate_f32 (grows).
  void* spmv_plan_mem = nullptr;
  size_t spmv_plan_bytes = 0;

  // Decoupled-lookback status words, one uint64 per tile (grows on demand). A word is valid only
  // when its epoch field equals the launch's epoch, so the array never needs clearing between
  // launches; it is cleared once when allocated and again whenever the epoch counter wraps.
  uint64_t* status = nullptr;
  size_t status_words = 0;
  uint32_t epoch = 0;

  // Per-round tile counts of the round-robin compaction kernel: one 32-bit word per tile,
  // (epoch16 << 16) | count, so a word left from an earlier launch never reads as current. Cleared
  // once when allocated and again whenever the 16-bit epoch wraps.
  uint32_t* round_counts = nullptr;
  size_t round_counts_words = 0;
  uint32_t round_epoch = 0;
  // Whether one 1024-thread workgroup of each round-robin kernel fits on a CU: -1 not yet asked.
  int rounds_fit = -1;
  // Recorded on this context's stream when another context's launch of the same kind must follow
  // this one's (dc::ResidentLaunch): [kOrderResident] resident grids, [kOrderNoAlloc] the calls
  // that share a device's static no-alloc scratch (that event is created with the context, since
  // the no-alloc path creates nothing).
  hipEvent_t order_done[2] = {nullptr, nullptr};
  // Launches of run-time compiled LINQ kernels on this context, and compilations that failed
  // (whose programs then ran on the interpreter); see dc_hip_linq_compile_stats.
  int64_t jit_launches = 0;
  int64_t jit_failures = 0;

  // Device address of the static scratch array of dc_hip_linq_where_select_sum_f32_noalloc on this
  // context's device (resolved once per device at context creation), and the status of that lookup.
  void* noalloc_scratch = nullptr;
  int32_t noalloc_status = DC_ERR_NOT_FOUND;
};

struct dc_hip_event {
  hipEvent_t ev = nullptr;
  int device = 0;
};

struct dc_hip_module {
  hipModule_t mod = nullptr;
  int device = 0;
};

#define DC_ORDER_KINDS 2

// Counter slots inside ctx->counters.
enum dc_counter_slot : int {
  DC_SLOT_LINQ_TICKET = 0,   // tile ticket of the compaction kernel (returned to 0 by the kernel)
  // slot 1: unused
  DC_SLOT_LINQ_DONE = 2,     // finished-workgroup word of the round-robin compaction (returned to 0)
  DC_SLOT_REDUCE_DONE = 3,   // finished-workgroup word of the one-launch reductions (returned to 0)
  DC_SLOT_LINQ_FAULT = 4,    // 64-bit (slots 4-5): first exception of an int32 LINQ ToArray, ~(4 * index +
                             // kind), 0 when none (returned to 0 by the kernel that reports it)
  DC_SLOT_COUNT = 1024
};

#define DC_RETURN_IF_HIP(expr)                         \
  do {                                                 \
    hipError_t dc_e_ = (expr);                         \
    if (dc_e_ != hipSuccess) return (int32_t)dc_e_;    \
  } while (0)

#define DC_RETURN_IF(status_expr)                      \
  do {                                                 \
    int32_t dc_s_ = (status_expr);                     \
    if (dc_s_ != DC_OK) return dc_s_;                  \
  } while (0)

// Lock the context and make its device current; every op entry point starts with this.
// hipGetLastError() also clears the runtime's sticky last-error slot, so a failed lookup in an
// earlier call (e.g. a missing module function) is not reported by this call's launch check.
#define DC_CTX_ENTER(ctx)                                      \
  if (!(ctx)) return DC_ERR_INVALID_ARGUMENT;                  \
  std::lock_guard<std::mutex> dc_lock_((ctx)->mu);             \
  DC_RETURN_IF_HIP(hipSetDevice((ctx)->device));               \
  (void)hipGetLastError()

namespace dc {

// Grows ctx->partials to at least `bytes` (caller holds the lock).
int32_t ensure_partials(dc_hip_ctx* ctx, size_t bytes);
// The round-robin ToArray kernel compiled at run time for one (validated) program over float32
// (is_int false) or int32 elements, for the context's device: compiled once per process and
// device and cached. nullptr when the compilation failed (counted in ctx->jit_failures).
hipFunction_t linq_jit_rounds(dc_hip_ctx* ctx, const dc_linq_chain& chain, bool is_int);
// Grows ctx->status to at least `words` and returns the epoch to use for the next launch.
int32_t ensure_status(dc_hip_ctx* ctx, size_t words, uint32_t* epoch_out);
// Grows ctx->round_counts to at least `words` and returns the 16-bit epoch for the next launch.
int32_t ensure_round_counts(dc_hip_ctx* ctx, size_t words, uint32_t* epoch_out);
// Launches that must not overlap another launch of the same kind on a device, from any context of
// the process. kOrderResident: resident grids (kernels whose workgroups wait for each other,
// launched with one workgroup per CU): two such grids could each hold half of the CUs while
// waiting for workgroups that cannot start. kOrderNoAlloc: the allocation-free LINQ Sum, whose
// partials live in one static array per device. A ResidentLaunch holds the device's slot lock of
// its kind from construction to destruction, so those enqueues on a device never interleave; when
// the previous launch of the kind came from another context, the constructor records an event on
// that context's stream (behind its launch) and makes this context's stream wait for it. A context
// that follows itself records nothing. The caller holds the context lock, enqueues the launch,
// then calls done(). (Other processes on the same device are not covered; the resident kernels'
// waits are bounded and report a failure instead of hanging.)
constexpr int kOrderResident = 0;
constexpr int kOrderNoAlloc = 1;
class ResidentLaunch {
 public:
  explicit ResidentLaunch(dc_hip_ctx* ctx, int kind = kOrderResident);
  ~ResidentLaunch();
  ResidentLaunch(const ResidentLaunch&) = delete;
  ResidentLaunch& operator=(const ResidentLaunch&) = delete;
  int32_t status() const { return status_; }
  void done();  // the grid is enqueued: this context now holds the device's last resident grid

 private:
  dc_hip_ctx* ctx_;
  int kind_;
  std::mutex* mu_ = nullptr;
  int32_t status_ = 0;
};
// Forgets the context's order events (context destruction).
void resident_forget(dc_hip_ctx* ctx);
// Looks up the device address of the no-alloc LINQ Sum's static scratch for ctx->device (the
// device must be current) and stores it in ctx->noalloc_scratch. Calls no allocator.
int32_t linq_noalloc_setup(dc_hip_ctx* ctx);
// Grow ctx->spmv_windows to at least `count` entries (caller holds the lock).
int32_t ensure_spmv_windows(dc_hip_ctx* ctx, size_t count);
int32_t ensure_spmv_plan_mem(dc_hip_ctx* ctx, size_t bytes);
// Two-pass deterministic float64 sum of n floats into *sum_out (device), on the ctx stream.
int32_t launch_reduce_sum_f32(dc_hip_ctx* ctx, const float* input, int64_t n, double* sum_out);
// *sum_out = partials[0] + ... + partials[count-1] (float64, fixed order; one workgroup).
int32_t launch_reduce_partials_f64(dc_hip_ctx* ctx, const double* partials, int count, double* sum_out);
// Fills device memory with zero bytes using a kernel (capture-safe).
int32_t zero_async(dc_hip_ctx* ctx, void* dst, size_t bytes);
inline int32_t last_launch_status() { return (int32_t)hipGetLastError(); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace dc
