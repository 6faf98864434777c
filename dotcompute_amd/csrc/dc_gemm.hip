// dc_gemm.hip — dense row-major GEMM C[m×n] = A[m×k]·B[k×n] on the gfx950 matrix cores.
//
// fp32: v_mfma_f32_32x32x2_f32 (fp32 inputs, fp32 accumulate).
// bf16: v_mfma_f32_32x32x16_bf16 (bf16 inputs, fp32 accumulate).
//
// Kernels, by the shapes that take them:
//   - gemm_f32_dma_kernel<T>: fp32 full tiles (m, n multiples of T = 128, or 64 when 128-tiles
//     cannot fill the CUs; k a multiple of 32). Direct-to-LDS loads, double-buffered LDS, 4 waves
//     of (T/2)×(T/2), two workgroups per CU.
//   - gemm_bf16_big_kernel: bf16 with m, n multiples of 256 and k a multiple of 64. 256×256 macro
//     tile, direct-to-LDS loads of row-major A and B, B fragments through transposing LDS reads,
//     8 waves of 128×64, one workgroup per CU.
//   - gemm_f32_kernel / gemm_bf16_kernel: every other shape (bounds-checked where a tile is
//     ragged). Block tile 128×128, 4 waves of 64×64; the next tile's global loads go to registers
//     before the current tile's MFMAs and are stored to the other LDS buffer afterwards, with B
//     transposed on the way in (Bs[n][k], row pitch BK+4 floats), so a lane's operands for 8
//     MFMAs are two contiguous, bank-conflict-free 16-byte LDS reads.
//
// Operand layout. For a 32×32 MFMA lane l supplies row (A) / column (B) l % 32 and the k-group
// h = l / 32; the instruction pairs A and B values by (h, element index), so any assignment of
// actual k indices to (h, element) is valid as long as A and B agree. bf16: lane group h takes
// the 8 consecutive k's [8h, 8h+8) of each 16-wide k step; fp32 (one k per lane per MFMA): the
// kernels choose k orders that make each lane's LDS reads contiguous.
//
// Tile order: consecutive workgroups are dispatched round-robin over the 8 XCDs (each with its own
// L2). Block b is mapped to tile (b % 8) * (T / 8) + b / 8, so each XCD works on a contiguous
// range of tiles, and within it tiles are walked in groups of 8 tile-rows, column by column, so
// the blocks resident on one XCD share A row-panels and B column-panels in that XCD's L2.
#include <algorithm>

#include <cstddef>
#include <type_traits>

#include "dc_device.hpp"
#include "dc_internal.hpp"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kThreads = 256;
constexpr int kGroupM = 8;

struct TileCoord {
  int tm, tn;
};

__device__ inline TileCoord map_tile(int tiles_m, int tiles_n) {
  const int total = tiles_m * tiles_n;
  int b = blockIdx.x;
  int t = (total % 8 == 0) ? (b % 8) * (total / 8) + b / 8 : b;
  const int group = kGroupM * tiles_n;
  const int g = t / group;
  const int first_m = g * kGroupM;
  const int gm = min(tiles_m - first_m, kGroupM);
  const int in_g = t - g * group;
  return TileCoord{first_m + in_g % gm, in_g / gm};
}

// ---------------------------------------------------------------------------------------------
// fp32, full tiles (m, n multiples of T, k a multiple of 32): direct-to-LDS loads, no staging
// registers and no transposing LDS stores.
//   A tile [T rows][32 k] (128 B rows, unpadded): the 16-byte k-quad q of row R sits in slot
//   q ^ ((R >> 1) & 7), so a fragment read (16 lanes = rows R0..R0+15 at one quad) touches 16
//   distinct 16-byte bank groups.
//   B tile [32 k][T n] in its natural row-major layout: the n-quad Q of k-row k sits at quad
//   Q ^ (8·((k >> 3) & 1)). Lane (r, h) of MFMA step kk reads B[ks + 8h + kk][n = r] with a 4-byte
//   LDS load: the h = 0 and h = 1 halves read rows 8 apart and land in opposite 128-byte halves of
//   the bank window.
// A wave's direct-to-LDS load writes 1 KiB (lane L -> bytes 16·L): the swizzles are applied on
// the global side (each lane fetches the quad that belongs in its slot).
// Pipeline as in the bf16 large-tile kernel: step 0 (k 0..15) runs its MFMAs with step 1's
// fragment reads between them; then the tile's one barrier (which also waits for tile kt+1's
// loads, issued a tile earlier); the loads of tile kt+2 go out into the buffer tile kt finished
// with, and step 1's MFMAs run with tile kt+1's step-0 fragment reads between them.
// ---------------------------------------------------------------------------------------------
constexpr int kBKd = 32;

// One LDS buffer per (operand, stage) as a separate __shared__ object, so the compiler can tell that
// loads into one stage's buffers do not alias reads of the other's (and need no wait before them).
template <int T>
struct F32DmaSmem {
  float* a[2];
  float* b[2];
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Waits until this wave's direct-to-LDS loads have landed (vmcnt(0); expcnt and lgkmcnt left
// alone), then the workgroup barrier: after it every wave's loads issued before are visible.
__device__ inline void dma_barrier() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // gfx9 encoding: vmcnt = 0, expcnt = 7, lgkmcnt = 15
  __syncthreads();
}

template <int T, int BUF>
__device__ inline void f32_tile_to_lds(const F32DmaSmem<T>& sm, __amdgpu_buffer_rsrc_t ra, const float* __restrict__ B, int N,
                                       int K, int n0, int k0, int wave, uint32_t avoff, const uint32_t (&bvoff)[T / 32]) {
  // A: T/8 blocks of 8 rows; wave w issues blocks w, w + 4, ...
#pragma unroll
  for (int i = 0; i < T / 32; ++i) {
    const int row0 = 8 * (4 * i + wave);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(sm.a[BUF] + row0 * kBKd), 16, avoff,
                                             (row0 * K + k0) * (int)sizeof(float), 0, 0);
  }
  // B: T/8 blocks of 256/T k-rows (this k slice only, as its own buffer range)
  const auto rb = dc::range_rsrc(B + (size_t)k0 * N + n0, ((kBKd - 1) * N + T) * (int)sizeof(float));
  constexpr int kRowsPerBlock = 256 / T;
#pragma unroll
  for (int i = 0; i < T / 32; ++i) {
    const int krow0 = kRowsPerBlock * (4 * i + wave);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)(sm.b[BUF] + krow0 * T), 16, bvoff[i],
                                             krow0 * N * (int)sizeof(float), 0, 0);
  }
}

template <int T>
__global__ __launch_bounds__(kThreads, 2) void gemm_f32_dma_kernel(const float* __restrict__ A,
                                                                   const float* __restrict__ B, float* __restrict__ C,
                                                                   int M, int N, int K, int tiles_m, int tiles_n) {
  constexpr int kW = T / 2, kMT = T / 64;  // wave tile edge, MFMA tiles per wave edge
  constexpr int kQuads = T / 4;            // n-quads per B row
  __shared__ __align__(16) float lds_a0[T * kBKd], lds_a1[T * kBKd], lds_b0[kBKd * T], lds_b1[kBKd * T];
  const F32DmaSmem<T> sm{{lds_a0, lds_a1}, {lds_b0, lds_b1}};
  const TileCoord tc = map_tile(tiles_m, tiles_n);
  const int m0 = tc.tm * T, n0 = tc.tn * T;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int r = lane & 31, h = lane >> 5;

  // load side: A panel as a buffer range (T rows of K floats < 2 GiB, checked by the host)
  const auto ra = dc::range_rsrc(A + (size_t)m0 * K, T * K * (int)sizeof(float));
  // A block 4i + w holds rows 8(4i + w) + L/8: (row >> 1) & 7 = (4·(w & 1) + L/16) & 7
  const uint32_t avoff =
      (uint32_t)(((lane >> 3) * K + 4 * ((lane & 7) ^ ((4 * (wave & 1) + (lane >> 4)) & 7))) * (int)sizeof(float));
  uint32_t bvoff[T / 32];
#pragma unroll
  for (int i = 0; i < T / 32; ++i) {
    const int kr = lane / kQuads;                        // k-row within the block
    const int k = (256 / T) * (4 * i + wave) + kr;       // k-row within the slice
    const int q = (lane % kQuads) ^ (8 * ((k >> 3) & 1));
    bvoff[i] = (uint32_t)((kr * N + 4 * q) * (int)sizeof(float));
  }

  f32x16 acc[kMT][kMT];
#pragma unroll
  for (int i = 0; i < kMT; ++i)
#pragma unroll
    for (int j = 0; j < kMT; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int kt_count = K / kBKd;
  f32_tile_to_lds<T, 0>(sm, ra, B, N, K, n0, 0, wave, avoff, bvoff);
  dma_barrier();
  if (kt_count > 1) f32_tile_to_lds<T, 1>(sm, ra, B, N, K, n0, kBKd, wave, avoff, bvoff);

  // Fragments of one 16-wide k step: A quads (2 per MFMA tile row block), B scalars (8 per column block).
  const int aswz = (r >> 1) & 7;
  auto read_frags = [&](auto BUF, int ks, dc::f32x4 (&a)[kMT][2], float (&b)[kMT][8]) __attribute__((always_inline)) {
    constexpr int kB = decltype(BUF)::value;
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        a[mt][j] = *reinterpret_cast<const dc::f32x4*>(
            &(kB ? lds_a1 : lds_a0)[(wm * kW + mt * 32 + r) * kBKd + 4 * ((ks / 4 + 2 * h + j) ^ aswz)]);
#pragma unroll
    for (int nt = 0; nt < kMT; ++nt) {
      const int n = wn * kW + nt * 32 + r;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk)
        b[nt][kk] = (kB ? lds_b1 : lds_b0)[(ks + 8 * h + kk) * T + 4 * ((n >> 2) ^ (8 * h)) + (n & 3)];
    }
  };
  auto mfmas = [&](const dc::f32x4 (&a)[kMT][2], const float (&b)[kMT][8]) __attribute__((always_inline)) {
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
        for (int nt = 0; nt < kMT; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[mt][kk >> 2][kk & 3], b[nt][kk], acc[mt][nt], 0, 0, 0);
  };
  constexpr int kReads = 2 * kMT + 8 * kMT;  // LDS reads per step
  auto interleave_reads = []() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kReads; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
    }
  };
  dc::f32x4 fa0[kMT][2], fa1[kMT][2];
  float fb0[kMT][8], fb1[kMT][8];
  read_frags(std::integral_constant<int, 0>{}, 0, fa0, fb0);
  // Tile KT in LDS buffer BUF = KT % 2 (unrolled by two so buffer offsets are constants; a macro
  // keeps the fragment arrays plain registers). After the last tile the barrier and the reads of
  // the other buffer are harmless and unused.
#define DC_F32_TILE(BUF, KT)                                                                      \
  {                                                                                               \
    __builtin_amdgcn_sched_barrier(0);                                                            \
    read_frags(std::integral_constant<int, BUF>{}, 16, fa1, fb1);                                 \
    mfmas(fa0, fb0);                                                                              \
    interleave_reads();                                                                           \
    __builtin_amdgcn_sched_barrier(0);                                                            \
    dma_barrier(); /* tile KT+1 is in LDS; every wave is done reading buffer BUF */               \
    if ((KT) + 2 < kt_count) f32_tile_to_lds<T, BUF>(sm, ra, B, N, K, n0, ((KT) + 2) * kBKd, wave, avoff, bvoff); \
    __builtin_amdgcn_sched_barrier(0);                                                            \
    read_frags(std::integral_constant<int, 1 - (BUF)>{}, 0, fa0, fb0);                            \
    mfmas(fa1, fb1);                                                                              \
    interleave_reads();                                                                           \
    __builtin_amdgcn_sched_barrier(0);                                                            \
  }
  for (int kt = 0; kt < kt_count; kt += 2) {
    DC_F32_TILE(0, kt);
    if (kt + 1 < kt_count) DC_F32_TILE(1, kt + 1);
  }
#undef DC_F32_TILE

  // acc[mt][nt][v] holds C[row][col], row = 8*(v/4) + 4*h + v%4, col = r (within the 32×32 tile).
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int nt = 0; nt < kMT; ++nt) {
      const int col = n0 + wn * kW + nt * 32 + r;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * kW + mt * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        C[(size_t)row * N + col] = acc[mt][nt][v];
      }
    }
}

// ---------------------------------------------------------------------------------------------
// fp32. T = macro tile (128, or 64 when 128-tiles cannot occupy the CUs: 1024² has only 64 of
// them); 4 waves as 2×2, each wave (T/2)×(T/2) = (T/64)×(T/64) MFMA 32×32 tiles.
// ---------------------------------------------------------------------------------------------
template <int BK, int T>
struct F32Smem {
  static constexpr int kPitch = BK + 4;  // floats per LDS row
  float a[2][T][kPitch];
  float b[2][T][kPitch];
};

// Global -> register prefetch for one BK slice. A: (T rows × BK) as float4 slots,
// slot s -> row s / (BK/4), kq = s % (BK/4). B: (BK × T) as float4 slots, slot s ->
// nq = s / BK, k = s % BK (a wave covers 16 k-rows × 4 column quads, which spreads the transposed
// LDS writes over the banks).
template <int BK, bool CHECKED, int T>
struct F32Loader {
  static constexpr int kASlots = T * BK / 4 / kThreads;
  static constexpr int kBSlots = T * BK / 4 / kThreads;
  dc::f32x4 ra[kASlots];
  dc::f32x4 rb[kBSlots];

  __device__ inline void load(const float* __restrict__ A, const float* __restrict__ B, int M, int N, int K,
                              int m0, int n0, int k0, int tid) {
#pragma unroll
    for (int i = 0; i < kASlots; ++i) {
      const int s = tid + i * kThreads;
      const int row = s / (BK / 4), kq = s % (BK / 4);
      const int gm = m0 + row, gk = k0 + 4 * kq;
      if (!CHECKED) {
        ra[i] = *reinterpret_cast<const dc::f32x4*>(A + (size_t)gm * K + gk);
      } else {
        dc::f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (gm < M) {
          const float* p = A + (size_t)gm * K;
          if (gk + 0 < K) v.x = p[gk + 0];
          if (gk + 1 < K) v.y = p[gk + 1];
          if (gk + 2 < K) v.z = p[gk + 2];
          if (gk + 3 < K) v.w = p[gk + 3];
        }
        ra[i] = v;
      }
    }
#pragma unroll
    for (int i = 0; i < kBSlots; ++i) {
      const int s = tid + i * kThreads;
      const int nq = s / BK, k = s % BK;
      const int gk = k0 + k, gn = n0 + 4 * nq;
      if (!CHECKED) {
        rb[i] = *reinterpret_cast<const dc::f32x4*>(B + (size_t)gk * N + gn);
      } else {
        dc::f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (gk < K) {
          const float* p = B + (size_t)gk * N;
          if (gn + 0 < N) v.x = p[gn + 0];
          if (gn + 1 < N) v.y = p[gn + 1];
          if (gn + 2 < N) v.z = p[gn + 2];
          if (gn + 3 < N) v.w = p[gn + 3];
        }
        rb[i] = v;
      }
    }
  }

  __device__ inline void store(F32Smem<BK, T>& sm, int buf, int tid) {
#pragma unroll
    for (int i = 0; i < kASlots; ++i) {
      const int s = tid + i * kThreads;
      const int row = s / (BK / 4), kq = s % (BK / 4);
      *reinterpret_cast<dc::f32x4*>(&sm.a[buf][row][4 * kq]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < kBSlots; ++i) {
      const int s = tid + i * kThreads;
      const int nq = s / BK, k = s % BK;
      sm.b[buf][4 * nq + 0][k] = rb[i].x;
      sm.b[buf][4 * nq + 1][k] = rb[i].y;
      sm.b[buf][4 * nq + 2][k] = rb[i].z;
      sm.b[buf][4 * nq + 3][k] = rb[i].w;
    }
  }
};

template <int BK, bool CHECKED, int T>
__global__ __launch_bounds__(kThreads, 2) void gemm_f32_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                               float* __restrict__ C, int M, int N, int K, int tiles_m,
                                                               int tiles_n) {
  constexpr int kW = T / 2, kMT = T / 64;  // wave tile edge, MFMA tiles per wave edge
  __shared__ F32Smem<BK, T> sm;
  const TileCoord tc = map_tile(tiles_m, tiles_n);
  const int m0 = tc.tm * T, n0 = tc.tn * T;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int r = lane & 31, h = lane >> 5;

  f32x16 acc[kMT][kMT];
#pragma unroll
  for (int i = 0; i < kMT; ++i)
#pragma unroll
    for (int j = 0; j < kMT; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  F32Loader<BK, CHECKED, T> ld;
  const int kt_count = (K + BK - 1) / BK;
  ld.load(A, B, M, N, K, m0, n0, 0, tid);
  ld.store(sm, 0, tid);
  __syncthreads();

  for (int kt = 0; kt < kt_count; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < kt_count) ld.load(A, B, M, N, K, m0, n0, (kt + 1) * BK, tid);
#pragma unroll
    for (int ks = 0; ks < BK; ks += 16) {
      dc::f32x4 a[kMT][2], b[kMT][2];
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt) {
        const float* p = &sm.a[buf][wm * kW + mt * 32 + r][ks + 8 * h];
        a[mt][0] = *reinterpret_cast<const dc::f32x4*>(p);
        a[mt][1] = *reinterpret_cast<const dc::f32x4*>(p + 4);
      }
#pragma unroll
      for (int nt = 0; nt < kMT; ++nt) {
        const float* p = &sm.b[buf][wn * kW + nt * 32 + r][ks + 8 * h];
        b[nt][0] = *reinterpret_cast<const dc::f32x4*>(p);
        b[nt][1] = *reinterpret_cast<const dc::f32x4*>(p + 4);
      }
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
#pragma unroll
        for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
          for (int nt = 0; nt < kMT; ++nt)
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[mt][kk >> 2][kk & 3], b[nt][kk >> 2][kk & 3],
                                                               acc[mt][nt], 0, 0, 0);
      }
    }
    if (kt + 1 < kt_count) ld.store(sm, buf ^ 1, tid);
    __syncthreads();
  }

  // acc[mt][nt][v] holds C[row][col], row = 8*(v/4) + 4*h + v%4, col = r (within the 32×32 tile).
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int nt = 0; nt < kMT; ++nt) {
      const int col = n0 + wn * kW + nt * 32 + r;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * kW + mt * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        if (!CHECKED || (row < M && col < N)) C[(size_t)row * N + col] = acc[mt][nt][v];
      }
    }
}

// ---------------------------------------------------------------------------------------------
// bf16 (inputs as raw bf16 bit patterns), fp32 accumulate
// ---------------------------------------------------------------------------------------------
template <int BK>
struct Bf16Smem {
  static constexpr int kPitch = BK + 8;  // bf16 elements per LDS row (16-byte aligned rows)
  unsigned short a[2][kBM][kPitch];
  unsigned short b[2][kBN][kPitch];
};

template <int BK, bool CHECKED>
struct Bf16Loader {
  // 8 bf16 (16 bytes) per slot.
  static constexpr int kASlots = kBM * BK / 8 / kThreads;
  static constexpr int kBSlots = kBN * BK / 8 / kThreads;
  u16x8 ra[kASlots];
  u16x8 rb[kBSlots];

  __device__ inline void load(const unsigned short* __restrict__ A, const unsigned short* __restrict__ B, int M, int N,
                              int K, int m0, int n0, int k0, int tid) {
#pragma unroll
    for (int i = 0; i < kASlots; ++i) {
      const int s = tid + i * kThreads;
      const int row = s / (BK / 8), kq = s % (BK / 8);
      const int gm = m0 + row, gk = k0 + 8 * kq;
      if (!CHECKED) {
        ra[i] = *reinterpret_cast<const u16x8*>(A + (size_t)gm * K + gk);
      } else {
        u16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
        if (gm < M) {
          const unsigned short* p = A + (size_t)gm * K;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (gk + e < K) v[e] = p[gk + e];
        }
        ra[i] = v;
      }
    }
#pragma unroll
    for (int i = 0; i < kBSlots; ++i) {
      const int s = tid + i * kThreads;
      const int nq = s / BK, k = s % BK;
      const int gk = k0 + k, gn = n0 + 8 * nq;
      if (!CHECKED) {
        rb[i] = *reinterpret_cast<const u16x8*>(B + (size_t)gk * N + gn);
      } else {
        u16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
        if (gk < K) {
          const unsigned short* p = B + (size_t)gk * N;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (gn + e < N) v[e] = p[gn + e];
        }
        rb[i] = v;
      }
    }
  }

  __device__ inline void store(Bf16Smem<BK>& sm, int buf, int tid) {
#pragma unroll
    for (int i = 0; i < kASlots; ++i) {
      const int s = tid + i * kThreads;
      const int row = s / (BK / 8), kq = s % (BK / 8);
      *reinterpret_cast<u16x8*>(&sm.a[buf][row][8 * kq]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < kBSlots; ++i) {
      const int s = tid + i * kThreads;
      const int nq = s / BK, k = s % BK;
#pragma unroll
      for (int e = 0; e < 8; ++e) sm.b[buf][8 * nq + e][k] = rb[i][e];
    }
  }
};

template <int BK, bool CHECKED>
__global__ __launch_bounds__(kThreads, 2) void gemm_bf16_kernel(const unsigned short* __restrict__ A,
                                                                const unsigned short* __restrict__ B,
                                                                float* __restrict__ C, int M, int N, int K,
                                                                int tiles_m, int tiles_n) {
  __shared__ Bf16Smem<BK> sm;
  const TileCoord tc = map_tile(tiles_m, tiles_n);
  const int m0 = tc.tm * kBM, n0 = tc.tn * kBN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int r = lane & 31, h = lane >> 5;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  Bf16Loader<BK, CHECKED> ld;
  const int kt_count = (K + BK - 1) / BK;
  ld.load(A, B, M, N, K, m0, n0, 0, tid);
  ld.store(sm, 0, tid);
  __syncthreads();

  for (int kt = 0; kt < kt_count; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < kt_count) ld.load(A, B, M, N, K, m0, n0, (kt + 1) * BK, tid);
#pragma unroll
    for (int ks = 0; ks < BK; ks += 16) {
      bf16x8 a[2], b[2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
        a[mt] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8*>(&sm.a[buf][wm * 64 + mt * 32 + r][ks + 8 * h]));
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
        b[nt] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8*>(&sm.b[buf][wn * 64 + nt * 32 + r][ks + 8 * h]));
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[mt], b[nt], acc[mt][nt], 0, 0, 0);
    }
    if (kt + 1 < kt_count) ld.store(sm, buf ^ 1, tid);
    __syncthreads();
  }

#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int col = n0 + wn * 64 + nt * 32 + r;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * 64 + mt * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        if (!CHECKED || (row < M && col < N)) C[(size_t)row * N + col] = acc[mt][nt][v];
      }
    }
}

// ---------------------------------------------------------------------------------------------
// bf16, large tiles: C = A·B straight from row-major A[M][K] and B[K][N].
//
// Macro tile 256×256, BK = 64, double-buffered LDS (2 × (32 + 32) KiB = 128 KiB, one workgroup
// per CU). 512 threads as 2×4 waves of 128×64 (4×2 MFMA 32×32×16 tiles, 128 accumulators per
// lane), two waves per SIMD so one's LDS and barrier waits overlap the other's MFMAs.
//
// Global -> LDS: direct-to-LDS loads (buffer_load_dwordx4 ... lds): lane L of a wave's load
// writes LDS bytes 16·L of a 1 KiB block, so no registers stage the tile and a tile's loads can
// stay in flight for a whole tile of MFMAs. The swizzles below are applied on the global side:
// each lane fetches the 16 bytes that belong in its LDS slot.
// - A tile: 256 rows (m) of 64 k, 128 B per row. The 16-byte k-octet q of row R sits in slot
//   q ^ ((R >> 1) & 7), so a fragment read (ds_read_b128: rows R0..R0+15 at one octet for each 16
//   lanes) touches 16 distinct 16-byte bank groups.
// - B tile: 64 rows (k) of 256 n, 512 B per row, as B is stored. The 64-byte block b of row k
//   sits at block b ^ (k & 3). The MFMA wants 8 consecutive k of one column n per lane; the
//   transposing LDS read ds_read_b64_tr_b16 gives that: within each 16 lanes, source lane
//   s = 4j + p reads the 4 bf16 of row k0 + j at columns n0 + 4p..4p+3, and lane i receives
//   B[k0 + j][n0 + i] for j = 0..3 (two such reads give k0..k0+7). The 32 lanes of each half
//   wave read 4 rows × 64 B at four different 64-byte offsets modulo 256 B: no bank conflicts.
//
// Pipeline of tile kt (buffer kt & 1): steps 0..2 run their MFMAs with the next step's fragment
// reads between them; then the tile's one barrier (which also waits for tile kt+1's loads, issued
// a tile earlier); right after it the loads of tile kt+2 go out into the buffer tile kt just
// finished with, and the last step's MFMAs run with tile kt+1's step-0 fragment reads between
// them, so no LDS latency is exposed after the barrier.
// ---------------------------------------------------------------------------------------------
constexpr int kBM2 = 256, kBN2 = 256, kBK2 = 64;
constexpr int kBigThreads = 512;
constexpr int kWaveM = 128, kWaveN = 64;       // wave tile
constexpr int kMT = kWaveM / 32, kNT = kWaveN / 32;
constexpr int kARow = kBK2 * 2;                // bytes per A row in LDS (64 k)
constexpr int kBRow = kBN2 * 2;                // bytes per B row in LDS (256 n)

struct Bf16BigSmem {
  unsigned short a[2][kBM2 * kBK2];
  unsigned short b[2][kBK2 * kBN2];
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4* lds_s16x4_ptr;

// Issues the direct-to-LDS loads of one BK slice (k0..k0+63) of the workgroup's A panel (rows
// m0..m0+255, buffer resource `ra`) and B panel (columns n0..n0+255 of rows k0.., resource `rb`)
// into LDS buffer BUF. Wave w's load i fills A rows 8·(8i + w) .. +7 and B rows 2·(8i + w) .. +1
// (1 KiB each). `avoff` / `bvoff` are the lane's byte offsets inside such a block's global rows;
// the block's global row offset is uniform (scalar).
template <int BUF>
__device__ inline void bf16_tile_to_lds(Bf16BigSmem& sm, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb, int K,
                                        int N, int k0, int wave, uint32_t avoff, uint32_t bvoff) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int blk = 8 * i + wave;
    const int32_t asoff = (8 * blk * K + k0) * (int32_t)sizeof(unsigned short);
    const int32_t bsoff = (k0 + 2 * blk) * N * (int32_t)sizeof(unsigned short);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)&sm.a[BUF][blk * 512], 16, avoff, asoff, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)&sm.b[BUF][blk * 512], 16, bvoff, bsoff, 0, 0);
  }
}

__global__ __launch_bounds__(kBigThreads, 1) void gemm_bf16_big_kernel(const unsigned short* __restrict__ A,
                                                                       const unsigned short* __restrict__ B,
                                                                       float* __restrict__ C, int M, int N, int K,
                                                                       int tiles_m, int tiles_n) {
  __shared__ __align__(16) Bf16BigSmem sm;  // 128 KiB of static LDS (gfx950 has 160 KiB per CU)
  const TileCoord tc = map_tile(tiles_m, tiles_n);
  const int m0 = tc.tm * kBM2, n0 = tc.tn * kBN2;
  // wave index in a scalar register: the loads' LDS bases and scalar offsets derive from it
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / (kBN2 / kWaveN), wn = wave % (kBN2 / kWaveN);
  const int r = lane & 31, h = lane >> 5;
  // load side: A panel (256 rows of K) and B panel (K rows, 256 columns at row pitch N) as buffer
  // ranges (both < 2 GiB, checked by the host)
  const auto ra = dc::range_rsrc(A + (size_t)m0 * K, kBM2 * K * (int32_t)sizeof(unsigned short));
  const auto rb = dc::range_rsrc(B + n0, ((K - 1) * N + kBN2) * (int32_t)sizeof(unsigned short));
  // A: lane -> row L / 8 of the block, slot L % 8 = octet (L % 8) ^ ((row >> 1) % 8), where
  // (row >> 1) % 8 depends on w and L only
  const int arow = lane >> 3;
  const int aswz = ((8 * wave + arow) >> 1) & 7;
  const uint32_t avoff = (uint32_t)((arow * K + 8 * ((lane & 7) ^ aswz)) * (int)sizeof(unsigned short));
  // B: lane -> row L / 32 of the block pair, 16-byte slot c = L % 32 (64-byte block c / 4), which
  // holds global chunk 4·((c / 4) ^ (row & 3)) + c % 4; row & 3 = (2w + L / 32) & 3
  const int brow = lane >> 5, bc = lane & 31;
  const int bchunk = 4 * ((bc >> 2) ^ ((2 * wave + brow) & 3)) + (bc & 3);
  const uint32_t bvoff = (uint32_t)((brow * N + 8 * bchunk) * (int)sizeof(unsigned short));
  // read side, A: fragment rows R = 32·t + r (t: wave and tile offsets, multiples of 32), so the
  // swizzle is (r >> 1) % 8; k-octet 2·step + h. Byte offsets of step s in buffer 0 (buffer and mt
  // offsets are immediates).
  const int rswz = (r >> 1) & 7;
  uint32_t aoff[4];
#pragma unroll
  for (int st = 0; st < 4; ++st)
    aoff[st] = (uint32_t)(wm * kWaveM + r) * kARow + 16u * (uint32_t)((2 * st + h) ^ rswz);
  // read side, B: source lane s = L % 16 = 4j + p reads row 8h + j (+16·step, +4 for the upper
  // four k: immediates) at columns wn·64 + nt·32 + 16·((L / 16) & 1) + 4p, whose 64-byte block
  // 2·wn + nt sits at (2·wn + nt) ^ j since the row is ≡ j (mod 4)
  uint32_t boff[kNT];
  {
    const int j = (lane & 15) >> 2, p4 = lane & 3, cg = (lane >> 4) & 1;
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
      boff[nt] = (uint32_t)offsetof(Bf16BigSmem, b) + (uint32_t)((8 * h + j) * kBRow) +
                 64u * (uint32_t)((2 * wn + nt) ^ j) + (uint32_t)(32 * cg + 8 * p4);
  }

  f32x16 acc[kMT][kNT];
#pragma unroll
  for (int i = 0; i < kMT; ++i)
#pragma unroll
    for (int j = 0; j < kNT; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  constexpr int kSteps = kBK2 / 16;
  static_assert(kSteps == 4, "four 16-wide k steps per tile");
  const int kt_count = K / kBK2;
  const unsigned char* lds = reinterpret_cast<const unsigned char*>(&sm);
  // B fragments of a whole tile (4 steps × kNT × 2 transposing reads) in one burst. The compiler
  // cannot tell these intrinsic reads apart from the LDS the direct-to-LDS loads write, so it
  // waits for every load in flight before each of them: the burst is issued while none is (right
  // after a barrier that waited for them all, before the next tile's loads go out).
  auto read_b_tile = [&](auto BUF, bf16x8 (*b)[kNT]) __attribute__((always_inline)) {
    constexpr uint32_t kBufB = (uint32_t)decltype(BUF)::value * kBK2 * kBRow;
#pragma unroll
    for (int st = 0; st < kSteps; ++st)
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) {
        const unsigned char* q = lds + boff[nt] + kBufB + st * 16 * kBRow;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(q));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(q + 4 * kBRow));
        b[st][nt] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
  };
  auto read_a = [&](auto BUF, int step, bf16x8* a) __attribute__((always_inline)) {
    constexpr uint32_t kBufA = (uint32_t)decltype(BUF)::value * kBM2 * kARow;
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
      a[mt] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8*>(lds + aoff[step] + kBufA + mt * 32 * kARow));
  };
  auto mfmas = [&](const bf16x8* a, const bf16x8* b) __attribute__((always_inline)) {
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt)
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[mt], b[nt], acc[mt][nt], 0, 0, 0);
  };
  // One A read after each of the first kMT MFMAs of the region (the rest run back to back).
  auto interleave_reads = []() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kMT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
    }
  };
  bf16x8 fa[2][kMT], fb[2][kSteps][kNT];
  bf16_tile_to_lds<0>(sm, ra, rb, K, N, 0, wave, avoff, bvoff);
  dma_barrier();
  read_b_tile(std::integral_constant<int, 0>{}, fb[0]);
  read_a(std::integral_constant<int, 0>{}, 0, fa[0]);
  if (kt_count > 1) bf16_tile_to_lds<1>(sm, ra, rb, K, N, kBK2, wave, avoff, bvoff);
  // Tile kt in LDS buffer BUF = kt % 2 (the loop is unrolled by two, so buffer offsets are
  // constants; a macro rather than a lambda keeps the fragment arrays plain registers).
#define DC_BF16_TILE(BUF, KT)                                                                      \
  {                                                                                                \
    _Pragma("unroll") for (int step = 0; step + 1 < kSteps; ++step) {                              \
      const int cur = step & 1;                                                                    \
      __builtin_amdgcn_sched_barrier(0);                                                           \
      read_a(std::integral_constant<int, BUF>{}, step + 1, fa[cur ^ 1]);                           \
      mfmas(fa[cur], fb[BUF][step]);                                                               \
      interleave_reads();                                                                          \
      __builtin_amdgcn_sched_barrier(0);                                                           \
    }                                                                                              \
    /* tile KT+1 is in LDS; every wave is done reading buffer BUF (after the last tile the */     \
    /* barrier and the reads of the other buffer are harmless and unused) */                      \
    dma_barrier();                                                                                 \
    read_b_tile(std::integral_constant<int, 1 - (BUF)>{}, fb[1 - (BUF)]);                          \
    if ((KT) + 2 < kt_count)                                                                       \
      bf16_tile_to_lds<BUF>(sm, ra, rb, K, N, ((KT) + 2) * kBK2, wave, avoff, bvoff);              \
    __builtin_amdgcn_sched_barrier(0);                                                             \
    read_a(std::integral_constant<int, 1 - (BUF)>{}, 0, fa[0]);                                    \
    mfmas(fa[1], fb[BUF][kSteps - 1]);                                                             \
    interleave_reads();                                                                            \
    __builtin_amdgcn_sched_barrier(0);                                                             \
  }
  // K is a positive multiple of 64 (host check): at least one tile, and no zero-trip path that
  // would keep the accumulators' initial values live beside the loop
  __builtin_assume(kt_count > 0);
  int kt = 0;
  do {
    DC_BF16_TILE(0, kt);
    if (kt + 1 < kt_count) DC_BF16_TILE(1, kt + 1);
    kt += 2;
  } while (kt < kt_count);
#undef DC_BF16_TILE

  // acc[mt][nt][v] holds C[row][col], row = 8*(v/4) + 4*h + v%4, col = r (within the 32×32 tile).
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
      const int col = n0 + wn * kWaveN + nt * 32 + r;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * kWaveM + mt * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        C[(size_t)row * N + col] = acc[mt][nt][v];
      }
    }
}

// Round-to-nearest-even fp32 -> bf16 (quiet NaN kept NaN).
__global__ __launch_bounds__(256) void f32_to_bf16_kernel(const float* __restrict__ x, unsigned short* __restrict__ y,
                                                          int64_t n) {
  int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    uint32_t u = __builtin_bit_cast(uint32_t, x[i]);
    unsigned short h;
    if ((u & 0x7fffffffu) > 0x7f800000u) {
      h = (unsigned short)((u >> 16) | 0x0040u);
    } else {
      u += 0x7fffu + ((u >> 16) & 1u);
      h = (unsigned short)(u >> 16);
    }
    y[i] = h;
  }
}

constexpr int kBKf32 = 32;
constexpr int kBKbf16 = 64;

int32_t check_dims(int64_t m, int64_t n, int64_t k) {
  if (m < 0 || n < 0 || k < 0) return DC_ERR_INVALID_ARGUMENT;
  if (m > INT32_MAX / 2 || n > INT32_MAX / 2 || k > INT32_MAX / 2) return DC_ERR_INVALID_ARGUMENT;
  return DC_OK;
}

}  // namespace

extern "C" {

DC_HIP_API int32_t dc_hip_gemm_f32(dc_hip_ctx* ctx, const float* a, const float* b, float* c, int64_t m, int64_t n,
                                   int64_t k) {
  DC_RETURN_IF(check_dims(m, n, k));
  if (m == 0 || n == 0) return ctx ? DC_OK : DC_ERR_INVALID_ARGUMENT;
  if (!c || (k > 0 && (!a || !b))) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  if (k == 0) return dc::zero_async(ctx, c, (size_t)(m * n) * sizeof(float));
  // 128×128 tiles unless that leaves fewer than two per CU; then 64×64 (four times the tiles)
  const int64_t tiles128 = ((m + 127) / 128) * ((n + 127) / 128);
  const bool small = tiles128 < 2 * (int64_t)std::max(1, ctx->cu_count);
  const int T = small ? 64 : 128;
  const int tiles_m = (int)((m + T - 1) / T), tiles_n = (int)((n + T - 1) / T);
  const unsigned grid = (unsigned)(tiles_m * tiles_n);
  // full tiles take the direct-to-LDS kernel; its A panel (T rows of k floats) is one buffer range
  const bool full = (m % T == 0) && (n % T == 0) && (k % kBKd == 0) && dc::aligned16(a) && dc::aligned16(b) &&
                    (int64_t)T * k * 4 < ((int64_t)1 << 31) && ((int64_t)kBKd * n + T) * 4 < ((int64_t)1 << 31);
#define DC_GEMM_F32_DMA(TT) \
  gemm_f32_dma_kernel<TT><<<grid, kThreads, 0, ctx->stream>>>(a, b, c, (int)m, (int)n, (int)k, tiles_m, tiles_n)
#define DC_GEMM_F32_CHECKED(TT)                                                                                 \
  gemm_f32_kernel<kBKf32, true, TT><<<grid, kThreads, 0, ctx->stream>>>(a, b, c, (int)m, (int)n, (int)k, tiles_m, \
                                                                       tiles_n)
  if (small) {
    if (full) DC_GEMM_F32_DMA(64); else DC_GEMM_F32_CHECKED(64);
  } else {
    if (full) DC_GEMM_F32_DMA(128); else DC_GEMM_F32_CHECKED(128);
  }
#undef DC_GEMM_F32_DMA
#undef DC_GEMM_F32_CHECKED
  return dc::last_launch_status();
}

DC_HIP_API int32_t dc_hip_gemm_bf16(dc_hip_ctx* ctx, const uint16_t* a, const uint16_t* b, float* c, int64_t m,
                                    int64_t n, int64_t k) {
  DC_RETURN_IF(check_dims(m, n, k));
  if (m == 0 || n == 0) return ctx ? DC_OK : DC_ERR_INVALID_ARGUMENT;
  if (!c || (k > 0 && (!a || !b))) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  if (k == 0) return dc::zero_async(ctx, c, (size_t)(m * n) * sizeof(float));
  const int tiles_m = (int)((m + kBM - 1) / kBM), tiles_n = (int)((n + kBN - 1) / kBN);
  const unsigned grid = (unsigned)(tiles_m * tiles_n);
  const unsigned short* A = reinterpret_cast<const unsigned short*>(a);
  const unsigned short* B = reinterpret_cast<const unsigned short*>(b);
  // large tiles: the A panel (256 rows of k bf16) and the B panel (k rows at pitch n) as buffer
  // ranges, each < 2 GiB
  if ((m % kBM2 == 0) && (n % kBN2 == 0) && (k % kBK2 == 0) && dc::aligned16(a) && dc::aligned16(b) &&
      (int64_t)k * kBM2 * 2 < ((int64_t)1 << 31) && (int64_t)k * n * 2 < ((int64_t)1 << 31)) {
    const int tm2 = (int)(m / kBM2), tn2 = (int)(n / kBN2);
    gemm_bf16_big_kernel<<<(unsigned)(tm2 * tn2), kBigThreads, 0, ctx->stream>>>(
        A, B, c, (int)m, (int)n, (int)k, tm2, tn2);
    return dc::last_launch_status();
  }
  const bool full = (m % kBM == 0) && (n % kBN == 0) && (k % kBKbf16 == 0) && dc::aligned16(a) && dc::aligned16(b);
  if (full)
    gemm_bf16_kernel<kBKbf16, false><<<grid, kThreads, 0, ctx->stream>>>(A, B, c, (int)m, (int)n, (int)k, tiles_m, tiles_n);
  else
    gemm_bf16_kernel<kBKbf16, true><<<grid, kThreads, 0, ctx->stream>>>(A, B, c, (int)m, (int)n, (int)k, tiles_m, tiles_n);
  return dc::last_launch_status();
}

DC_HIP_API int32_t dc_hip_convert_f32_to_bf16(dc_hip_ctx* ctx, const float* input, uint16_t* output, int64_t n) {
  if (n < 0 || (n > 0 && (!input || !output))) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  if (n == 0) return DC_OK;
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, 16384));
  f32_to_bf16_kernel<<<grid, 256, 0, ctx->stream>>>(input, reinterpret_cast<unsigned short*>(output), n);
  return dc::last_launch_status();
}

}  // extern "C"
