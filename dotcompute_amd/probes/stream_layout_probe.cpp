// stream_layout_probe.cpp — measurement-only program (not linked into any library): how the access
// layout of a read-1-GiB / write-512-MiB stream changes what HBM delivers on MI355X. It backs the
// ceiling analysis of the round-robin Where/Select kernel (a persistent grid, one workgroup per CU)
// against the covering-grid streaming probes. Build and run (one GPU, about a second):
//   hipcc --offload-arch=gfx950 -O3 -std=c++20 -Xclang -target-feature -Xclang -packed-fp32-ops \
//         dotcompute_amd/probes/stream_layout_probe.cpp -o /tmp/stream_layout_probe && /tmp/stream_layout_probe
// Every kernel reads 2 vectors for each one it writes (the 50 %-kept mix), non-temporal, 16-byte
// vectors, over 1000 MiB of input; times are HIP events over 50 launches after 3 warm-up launches.
// The persistent variants also record each workgroup's start and end (wall_clock64, 100 MHz) and
// print per-XCD mean end times (workgroup b runs on XCD b mod 8).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <utility>
#include <vector>

typedef float f32x4 __attribute__((ext_vector_type(4)));
#define CK(x)                                                                \
  do {                                                                       \
    hipError_t e_ = (x);                                                     \
    if (e_ != hipSuccess) {                                                  \
      std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      std::exit(1);                                                          \
    }                                                                        \
  } while (0)

namespace {

template <class F, int... U>
__device__ __attribute__((always_inline)) inline void each(F&& f, std::integer_sequence<int, U...>) {
  (f(std::integral_constant<int, U>{}), ...);
}

// Covering grid, two read streams h4 vectors apart and one write stream, all advancing together.
__global__ __launch_bounds__(256) void cover_two_streams(const f32x4* __restrict__ in, f32x4* __restrict__ out, int64_t h4) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < h4)
    __builtin_nontemporal_store(__builtin_nontemporal_load(in + i) + __builtin_nontemporal_load(in + h4 + i), out + i);
}

// Covering grid, one read stream: each block reads VEC consecutive 4 KiB pieces and writes VEC / 2
// (the read stream advances twice as fast as the write stream, as in a compaction).
template <int VEC>
__global__ __launch_bounds__(256) void cover_one_stream(const f32x4* __restrict__ in, f32x4* __restrict__ out) {
  const f32x4* p = in + (int64_t)blockIdx.x * 256 * VEC;
  f32x4 e[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) e[j] = __builtin_nontemporal_load(p + j * 256 + threadIdx.x);
  f32x4* o = out + (int64_t)blockIdx.x * 128 * VEC;
#pragma unroll
  for (int j = 0; j < VEC / 2; ++j) __builtin_nontemporal_store(e[2 * j] + e[2 * j + 1], o + j * 256 + threadIdx.x);
}

// Persistent grid with the round-robin kernel's layout: P workgroups of WAVES worker waves (+ one
// idle wave, as the control wave), tile of round r at position w = r * P + w (positions dealt out
// XCD by XCD), VEC vectors per lane per tile, loads AHEAD rounds ahead in registers, one barrier per
// round. `rounds` is a multiple of AHEAD + 1.
template <int WAVES, int VEC, int AHEAD>
__global__ __launch_bounds__(64 * (WAVES + 1)) void persistent(const f32x4* __restrict__ in, f32x4* __restrict__ out,
                                                               int64_t rounds, uint32_t P, uint64_t* stamps) {
  // The launch's dynamic LDS size (unused by the code) sets how many workgroups fit per CU.
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t w = (P % 8u == 0u) ? (blockIdx.x % 8u) * (P / 8u) + blockIdx.x / 8u : blockIdx.x;
  constexpr int CH4 = 64 * VEC, TILE4 = WAVES * CH4, NB = AHEAD + 1;
  const uint64_t t0 = wall_clock64();
  if (wave < WAVES) {
    f32x4 e[NB][VEC];
    auto load = [&](f32x4 (&b)[VEC], int64_t r) __attribute__((always_inline)) {
      const f32x4* p = in + (r * P + w) * TILE4 + wave * CH4;
#pragma unroll
      for (int j = 0; j < VEC; ++j) b[j] = __builtin_nontemporal_load(p + j * 64 + lane);
    };
    each([&](auto U) __attribute__((always_inline)) { load(e[U.value], min((int64_t)U.value, rounds - 1)); },
         std::make_integer_sequence<int, AHEAD>{});
    int64_t r = 0;
    auto step = [&](f32x4 (&ec)[VEC], f32x4 (&en)[VEC]) __attribute__((always_inline)) {
      load(en, min(r + AHEAD, rounds - 1));
      f32x4* o = out + (r * P + w) * (TILE4 / 2) + wave * (CH4 / 2);
#pragma unroll
      for (int j = 0; j < VEC / 2; ++j) __builtin_nontemporal_store(ec[2 * j] + ec[2 * j + 1], o + j * 64 + lane);
      __syncthreads();
      ++r;
    };
    for (int64_t it = rounds / NB; it > 0; --it)
      each([&](auto U) __attribute__((always_inline)) { step(e[U.value], e[(U.value + AHEAD) % NB]); },
           std::make_integer_sequence<int, NB>{});
  } else {
    for (int64_t r = 0; r < rounds; ++r) __syncthreads();
  }
  if (threadIdx.x == 0) {
    stamps[2 * blockIdx.x] = t0;
    stamps[2 * blockIdx.x + 1] = wall_clock64();
  }
}

// Persistent grid with dynamic balancing between XCDs: blocks of 32 tiles are claimed from a global
// counter by the first workgroup of each XCD and published (tagged with the launch's epoch) in
// claims[x][k]; workgroup i of XCD x processes tile 32 b + i of every block b its XCD claimed. A
// claim that does not arrive within the bounded wait ends the workgroup's loop and is counted.
constexpr int kMaxClaims = 4096;
template <int WAVES, int VEC, int AHEAD>
__global__ __launch_bounds__(64 * (WAVES + 1)) void persistent_xcd_claims(
    const f32x4* __restrict__ in, f32x4* __restrict__ out, int64_t nblocks, unsigned long long* counter,
    unsigned long long* claims, unsigned long long epoch, uint64_t* stamps, unsigned* gave_up) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int x = blockIdx.x & 7, li = blockIdx.x >> 3;
  const bool leader = li == 0;
  unsigned long long* mine = claims + (size_t)x * kMaxClaims;
  constexpr int CH4 = 64 * VEC, TILE4 = WAVES * CH4, NB = AHEAD + 1, NT = 16;
  __shared__ int64_t s_b[NT];
  const uint64_t t0 = wall_clock64();
  const int64_t ntiles = nblocks * 32;
  auto claim = [&](int64_t k) -> int64_t {
    if (leader) {
      const unsigned long long b = atomicAdd(counter, 1ull);
      __hip_atomic_store(mine + k, (epoch << 32) | b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return (int64_t)b;
    }
    for (int spin = 0; spin < (1 << 20); ++spin) {
      const unsigned long long v = __hip_atomic_load(mine + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((v >> 32) == epoch) return (int64_t)(v & 0xFFFFFFFFull);
      __builtin_amdgcn_s_sleep(2);
    }
    atomicAdd(gave_up, 1u);
    return nblocks;
  };
  if (wave == WAVES && lane == 0)
    for (int k = 0; k < AHEAD + 2; ++k) s_b[k] = claim(k);
  __syncthreads();
  f32x4 e[NB][VEC];
  auto load = [&](f32x4 (&b)[VEC], int64_t blk) __attribute__((always_inline)) {
    const f32x4* p = in + min(blk * 32 + li, ntiles - 1) * TILE4 + wave * CH4;
#pragma unroll
    for (int j = 0; j < VEC; ++j) b[j] = __builtin_nontemporal_load(p + j * 64 + lane);
  };
  if (wave < WAVES)
    each([&](auto U) __attribute__((always_inline)) { load(e[U.value], s_b[U.value]); },
         std::make_integer_sequence<int, AHEAD>{});
  int64_t s = 0;
  bool go = s_b[0] < nblocks;
  auto step = [&](f32x4 (&ec)[VEC], f32x4 (&en)[VEC]) __attribute__((always_inline)) {
    const int64_t bc = s_b[s % NT];
    if (wave < WAVES) {
      load(en, s_b[(s + AHEAD) % NT]);
      if (bc < nblocks) {
        f32x4* o = out + (bc * 32 + li) * (TILE4 / 2) + wave * (CH4 / 2);
#pragma unroll
        for (int j = 0; j < VEC / 2; ++j) __builtin_nontemporal_store(ec[2 * j] + ec[2 * j + 1], o + j * 64 + lane);
      }
    } else if (lane == 0) {
      s_b[(s + AHEAD + 2) % NT] = claim(s + AHEAD + 2);
    }
    __syncthreads();
    ++s;
    go = s_b[s % NT] < nblocks;
  };
  while (go && s + AHEAD + 2 + NB < kMaxClaims)
    each([&](auto U) __attribute__((always_inline)) { step(e[U.value], e[(U.value + AHEAD) % NB]); },
         std::make_integer_sequence<int, NB>{});
  __syncthreads();
  if (threadIdx.x == 0) {
    stamps[2 * blockIdx.x] = t0;
    stamps[2 * blockIdx.x + 1] = wall_clock64();
    if (atomicAdd(counter + 1, 1ull) == gridDim.x - 1) {  // the last one out resets the counter
      counter[0] = 0;
      counter[1] = 0;
    }
  }
}

template <class L>
float time_us(L&& launch, int reps) {
  hipEvent_t a, b;
  CK(hipEventCreate(&a));
  CK(hipEventCreate(&b));
  for (int i = 0; i < 3; ++i) launch();
  CK(hipDeviceSynchronize());
  CK(hipEventRecord(a, 0));
  for (int i = 0; i < reps; ++i) launch();
  CK(hipEventRecord(b, 0));
  CK(hipEventSynchronize(b));
  float ms = 0;
  CK(hipEventElapsedTime(&ms, a, b));
  CK(hipEventDestroy(a));
  CK(hipEventDestroy(b));
  return 1000.0f * ms / reps;
}

// Start/end stamps of the last launch: start spread, and mean end per XCD.
void print_stamps(const uint64_t* dstamps, int groups) {
  std::vector<uint64_t> h(2 * groups);
  CK(hipMemcpy(h.data(), dstamps, 16 * (size_t)groups, hipMemcpyDeviceToHost));
  uint64_t s0 = ~0ull, s1 = 0;
  for (int g = 0; g < groups; ++g) {
    s0 = std::min(s0, h[2 * g]);
    s1 = std::max(s1, h[2 * g]);
  }
  std::printf("      starts within %.1f us; mean end per XCD (us):", (s1 - s0) / 100.0);
  for (int x = 0; x < 8; ++x) {
    double sum = 0;
    int cnt = 0;
    for (int g = x; g < groups; g += 8, ++cnt) sum += (h[2 * g + 1] - s0) / 100.0;
    std::printf(" %.1f", sum / cnt);
  }
  double e0 = 1e30, e1 = 0;
  for (int g = 0; g < groups; ++g) {
    e0 = std::min(e0, (h[2 * g + 1] - s0) / 100.0);
    e1 = std::max(e1, (h[2 * g + 1] - s0) / 100.0);
  }
  std::printf("; first end %.1f, last %.1f\n", e0, e1);
}

}  // namespace

int main() {
  const int64_t bytes = 125ll * 256 * 32768;  // 1000 MiB of input
  const int64_t n4 = bytes / 16;
  const int reps = 50;
  f32x4 *in, *out;
  uint64_t* stamps;
  unsigned long long *counter, *claims;
  unsigned* gave_up;
  CK(hipMalloc(&in, bytes));
  CK(hipMalloc(&out, bytes / 2));
  CK(hipMalloc(&stamps, 16 * 1024));
  CK(hipMalloc(&counter, 16));
  CK(hipMalloc(&claims, 8 * kMaxClaims * sizeof(unsigned long long)));
  CK(hipMalloc(&gave_up, 4));
  CK(hipMemset(in, 0, bytes));
  CK(hipMemset(counter, 0, 16));
  CK(hipMemset(claims, 0, 8 * kMaxClaims * sizeof(unsigned long long)));
  CK(hipMemset(gave_up, 0, 4));
  auto report = [&](const char* name, float us, double read_bytes) {
    std::printf("%-44s %7.1f us  %6.1f us per GiB read\n", name, us, us * 1073741824.0 / read_bytes);
  };
  report("covering grid, two read streams", time_us([&] {
    cover_two_streams<<<(unsigned)(n4 / 2 / 256), 256>>>(in, out, n4 / 2); }, reps), bytes);
  report("covering grid, one read stream, 8 KiB blocks", time_us([&] {
    cover_one_stream<2><<<(unsigned)(n4 / 512), 256>>>(in, out); }, reps), bytes);
  report("covering grid, one read stream, 16 KiB blocks", time_us([&] {
    cover_one_stream<4><<<(unsigned)(n4 / 1024), 256>>>(in, out); }, reps), bytes);
  // persistent: 8 workers x 4 vectors (32 KiB tiles) x 4 rounds ahead, as the headline kernel
  auto k844 = persistent<8, 4, 4>;
  CK(hipFuncSetAttribute((const void*)k844, hipFuncAttributeMaxDynamicSharedMemorySize, 140 * 1024));
  report("persistent 256 x (8 waves x 4 vec), 4 ahead", time_us([&] {
    k844<<<256, 576, 130 * 1024>>>(in, out, 125, 256, stamps); }, reps), bytes);
  print_stamps(stamps, 256);
  report("persistent 512 x (8 waves x 4 vec), 70 KiB LDS", time_us([&] {
    k844<<<512, 576, 70 * 1024>>>(in, out, 60, 512, stamps); }, reps), 60.0 * 512 * 32768);
  print_stamps(stamps, 512);
  auto k822 = persistent<8, 2, 2>;
  report("persistent 256 x (8 waves x 2 vec), 2 ahead", time_us([&] {
    k822<<<256, 576, 0>>>(in, out, 249, 256, stamps); }, reps), 249.0 * 256 * 16384);
  print_stamps(stamps, 256);
  unsigned long long epoch = 0;
  report("persistent 256 x (8 x 4), XCD-block claims", time_us([&] {
    ++epoch;
    persistent_xcd_claims<8, 4, 4><<<256, 576>>>(in, out, 1000, counter, claims, epoch, stamps, gave_up); }, reps),
         bytes);
  print_stamps(stamps, 256);
  unsigned g = 0;
  CK(hipMemcpy(&g, gave_up, 4, hipMemcpyDeviceToHost));
  std::printf("claims that did not arrive: %u\n", g);
  CK(hipFree(in));
  CK(hipFree(out));
  CK(hipFree(stamps));
  CK(hipFree(counter));
  CK(hipFree(claims));
  CK(hipFree(gave_up));
  return 0;
}
