// dc_device.hpp — device-side building blocks shared by the gfx950 kernels: counter-based
// generator, wave64 DPP reductions, block reductions and agent-scope atomics.
#pragma once

#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#endif

#include <cstdint>

namespace dc {

constexpr int kWave = 64;

// SplitMix64 finaliser (Steele, Lea, Flood, OOPSLA 2014).
__host__ __device__ inline uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__host__ __device__ inline uint64_t gen_key(uint64_t seed, uint32_t stream, uint64_t i) {
  return seed ^ (static_cast<uint64_t>(stream) << 40) ^ i;
}

// [-1,1) with 2^-23 spacing, or [0,1) with 2^-24 spacing; both exact in float32.
__host__ __device__ inline float gen_f32(uint64_t r, int unit_interval) {
  float u = static_cast<float>(static_cast<uint32_t>(r >> 40));
  return unit_interval ? u * 0x1p-24f : u * 0x1p-23f - 1.0f;
}

__host__ __device__ inline int32_t gen_i32(uint64_t r, int32_t lo, uint64_t span) {
  return static_cast<int32_t>(static_cast<int64_t>(lo) + static_cast<int64_t>(((r >> 32) * span) >> 32));
}

// ---- DPP wave reductions (result valid in lane 63, then broadcast with readlane) -------------
// DPP control words (GFX9 encoding): quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E,
// row_half_mirror = 0x141, row_mirror = 0x140, row_bcast:15 = 0x142, row_bcast:31 = 0x143.

template <int CTRL, int ROW_MASK>
__device__ inline uint32_t dpp_u32(uint32_t v) {
  // Lanes in rows outside ROW_MASK receive `old` = 0, so an add of the result is a no-op there.
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROW_MASK, 0xF, false));
}

template <int CTRL, int ROW_MASK>
__device__ inline uint64_t dpp_u64(uint64_t v) {
  uint32_t lo = dpp_u32<CTRL, ROW_MASK>(static_cast<uint32_t>(v));
  uint32_t hi = dpp_u32<CTRL, ROW_MASK>(static_cast<uint32_t>(v >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ inline uint64_t readlane_u64(uint64_t v, int lane) {
  uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), lane));
  uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v >> 32)), lane));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

template <typename T>
__device__ inline uint64_t as_u64(T v) { return __builtin_bit_cast(uint64_t, v); }
template <typename T>
__device__ inline T from_u64(uint64_t v) { return __builtin_bit_cast(T, v); }

// Sum over the 64 lanes of a wave for 64-bit T (double or int64); every lane must be active.
// Fixed combination tree, so the result is deterministic for a given lane assignment.
template <typename T>
__device__ inline T wave_sum64(T v) {
  static_assert(sizeof(T) == 8, "64-bit lanes only");
  v = v + from_u64<T>(dpp_u64<0xB1, 0xF>(as_u64(v)));   // lanes xor 1
  v = v + from_u64<T>(dpp_u64<0x4E, 0xF>(as_u64(v)));   // lanes xor 2  -> quad sums
  v = v + from_u64<T>(dpp_u64<0x141, 0xF>(as_u64(v)));  // half-row mirror -> 8-lane sums
  v = v + from_u64<T>(dpp_u64<0x140, 0xF>(as_u64(v)));  // row mirror -> 16-lane row sums
  v = v + from_u64<T>(dpp_u64<0x142, 0xA>(as_u64(v)));  // lane 15 of rows 0/2 into rows 1/3
  v = v + from_u64<T>(dpp_u64<0x143, 0xC>(as_u64(v)));  // lane 31 into rows 2/3
  return from_u64<T>(readlane_u64(as_u64(v), 63));
}

// Inclusive prefix sum over the 64 lanes of a wave (lane i gets v_0 + ... + v_i) for 64-bit T:
// row_shr 1, 2, 4, 8 scan each row of 16 lanes, then row_bcast 15 / 31 carry the row totals
// forward. Every lane must be active.
template <typename T>
__device__ inline T wave_inclusive_scan64(T v) {
  static_assert(sizeof(T) == 8, "64-bit lanes only");
  v = v + from_u64<T>(dpp_u64<0x111, 0xF>(as_u64(v)));  // row_shr:1
  v = v + from_u64<T>(dpp_u64<0x112, 0xF>(as_u64(v)));  // row_shr:2
  v = v + from_u64<T>(dpp_u64<0x114, 0xF>(as_u64(v)));  // row_shr:4
  v = v + from_u64<T>(dpp_u64<0x118, 0xF>(as_u64(v)));  // row_shr:8
  v = v + from_u64<T>(dpp_u64<0x142, 0xA>(as_u64(v)));  // row_bcast:15 into rows 1 and 3
  v = v + from_u64<T>(dpp_u64<0x143, 0xC>(as_u64(v)));  // row_bcast:31 into rows 2 and 3
  return v;
}

// Block-wide sum for BLOCK threads (multiple of 64). Fixed order: wave sums, then waves 0..W-1
// in order. Result valid in every thread. Uses `scratch` (W elements of shared memory).
template <int BLOCK, typename T>
__device__ inline T block_sum64(T v, T* scratch) {
  constexpr int W = BLOCK / kWave;
  T w = wave_sum64(v);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  if (lane == 0) scratch[wave] = w;
  __syncthreads();
  T total = scratch[0];
#pragma unroll
  for (int i = 1; i < W; ++i) total = total + scratch[i];
  __syncthreads();
  return total;
}

// ---- agent-scope atomics used by the grid combines --------------------------------------------
__device__ inline uint64_t load_agent_u64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void store_agent_u64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t fetch_add_agent_u32(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t load_agent_u32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void store_agent_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t fetch_add_relaxed_agent_u32(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until this wave's outstanding memory operations, stores included, have completed. After an
// agent-scope atomic store (which writes through the XCD's L2) this makes the store visible to
// every XCD before what follows, without the L2 write-back of an agent-scope release fence.
__device__ inline void wait_memory_ops() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ inline void fence_release_agent() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent"); }
__device__ inline void fence_acquire_agent() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }

// Native 4-wide vectors (16-byte global loads/stores).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Streaming 16-byte load that does not displace reusable cache lines.
__device__ inline f32x4 load_stream(const f32x4* p) { return __builtin_nontemporal_load(p); }
__device__ inline i32x4 load_stream(const i32x4* p) { return __builtin_nontemporal_load(p); }

// Buffer resource over [p, p + bytes) (bytes < 4 GiB): loads past the end return 0 and stores past
// it are dropped by the hardware range check, without touching memory, so code can issue a fixed
// set of accesses with no branches around them.
__device__ inline __amdgpu_buffer_rsrc_t range_rsrc(const void* p, int32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}
constexpr int kBufNt = 2;  // buffer cache policy: non-temporal (streamed once)

}  // namespace dc
