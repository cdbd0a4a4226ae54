// Shared definitions of libekv_hip: status codes, error text, device properties, and the
// wave64 / workgroup primitives the kernels use (gfx950: 64-lane wavefronts).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/ekv_hip.h"

namespace ekv {

constexpr int kWave = 64;

// Records the message of the failing call on this thread; returns `status` for chaining.
int fail(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// Maps a HIP error to EKV_ELAUNCH with the call's name, or EKV_OK.
int check_hip(hipError_t err, const char *what);

// Number of compute units of the current device (cached per device).
int cu_count();

// ---------------------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------------------

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// A pointer read out of memory (a field of an argument struct indexed at run time, a table of
// pointers) is generic to the compiler, and its accesses become FLAT instructions.  A FLAT access
// counts against the LDS wait counter as well as the vector-memory one, so every later wait for
// an LDS result also waits for it: a key load issued before the LDS work of the previous chunk
// would be waited for by that work.  These casts state that the memory is global.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T *as_global(const T *p) {
  return (const __attribute__((address_space(1))) T *)p;
}
template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T *as_global(T *p) {
  return (__attribute__((address_space(1))) T *)p;
}

template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

// Max / sum over the four 16-lane rows of a wave (lanes l, l ^ 16, l ^ 32, l ^ 48), every lane
// receiving the result, on the VALU with no LDS round trip.  v_permlane16_swap of a register with
// a copy of itself returns rows (0, 0, 2, 2) and rows (1, 1, 3, 3); v_permlane32_swap returns the
// low half twice and the high half twice.  Each step combines the two results, so every lane gets
// the same bits as the xor-16 then xor-32 butterfly.
//
// Both the operand copy and the two results pass through empty asm statements.  Without them this
// compiler folds the exchange: given one value for both operands it takes the results to be equal,
// and where the two results meet in one expression it reads the first result twice (both seen in
// the generated code; the parity tests of every kernel that uses these catch either).
__device__ __forceinline__ void row_swap16(float v, float &a, float &b) {
  const uint32_t x = __builtin_bit_cast(uint32_t, v);
  uint32_t y = x;
  asm volatile("" : "+v"(y));
  const auto r = __builtin_amdgcn_permlane16_swap(x, y, false, false);
  uint32_t r0 = r[0], r1 = r[1];
  asm volatile("" : "+v"(r0), "+v"(r1));
  a = __builtin_bit_cast(float, r0);
  b = __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ void row_swap32(float v, float &a, float &b) {
  const uint32_t x = __builtin_bit_cast(uint32_t, v);
  uint32_t y = x;
  asm volatile("" : "+v"(y));
  const auto r = __builtin_amdgcn_permlane32_swap(x, y, false, false);
  uint32_t r0 = r[0], r1 = r[1];
  asm volatile("" : "+v"(r0), "+v"(r1));
  a = __builtin_bit_cast(float, r0);
  b = __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ float rows_max(float v) {
  float a, b;
  row_swap16(v, a, b);
  row_swap32(fmaxf(a, b), a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float rows_sum(float v) {
  float a, b;
  row_swap16(v, a, b);
  row_swap32(a + b, a, b);
  return a + b;
}

// Sum / max over all 64 lanes; every lane receives the result.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += shfl_xor(v, m);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor(v, m));
  return v;
}
// Integer sums and scans over a wave on DPP lane moves (no LDS round trip; a __shfl is a
// ds_bpermute, whose latency a chain of six pays six times).  Every lane of the wave must be
// active.  GFX9 DPP controls: quad_perm [1,0,3,2] and [2,3,0,1] (xor 1, xor 2 in each quad),
// row_shr:n = 0x110 + n, row_ror:n = 0x120 + n, row_bcast:15 = 0x142, row_bcast:31 = 0x143.
template <int CTRL, int ROW_MASK = 0xf, bool BOUND_ZERO = false>
__device__ __forceinline__ int dpp_move(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, BOUND_ZERO);
}
// each lane receives the sum of its 16-lane row
__device__ __forceinline__ int row_sum_int(int v) {
  v += dpp_move<0xB1>(v);
  v += dpp_move<0x4E>(v);
  v += dpp_move<0x124>(v);
  v += dpp_move<0x128>(v);
  return v;
}
__device__ __forceinline__ long long row_sum_i64(long long v) {
  auto step = [](long long x, long long y) { return x + y; };
  auto move = [](long long x, auto ctrl) {
    const int lo = dpp_move<decltype(ctrl)::value>((int)(uint32_t)x);
    const int hi = dpp_move<decltype(ctrl)::value>((int)(uint32_t)((uint64_t)x >> 32));
    return (long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
  };
  v = step(v, move(v, std::integral_constant<int, 0xB1>()));
  v = step(v, move(v, std::integral_constant<int, 0x4E>()));
  v = step(v, move(v, std::integral_constant<int, 0x124>()));
  v = step(v, move(v, std::integral_constant<int, 0x128>()));
  return v;
}
__device__ __forceinline__ int wave_sum_int(int v) {
  v = row_sum_int(v);
  return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
         __builtin_amdgcn_readlane(v, 48);
}
__device__ __forceinline__ long long wave_sum_i64(long long v) {
  v = row_sum_i64(v);
  long long s = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 16 * r);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), 16 * r);
    s += (long long)(((uint64_t)hi << 32) | lo);
  }
  return s;
}

// Inclusive scan of `v` across the 64 lanes of a wave: shifts within each 16-lane row, then the
// rows' totals carried forward (lane 15 into row 1 and row 3, then lane 31 into rows 2 and 3).
// Every lane of the wave must be active.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  v += dpp_move<0x111, 0xf, true>(v);
  v += dpp_move<0x112, 0xf, true>(v);
  v += dpp_move<0x114, 0xf, true>(v);
  v += dpp_move<0x118, 0xf, true>(v);
  v += dpp_move<0x142, 0xa>(v);
  v += dpp_move<0x143, 0xc>(v);
  return v;
}

// A workgroup barrier that orders LDS only: the wave's LDS requests complete, then every wave meets.
// __syncthreads() also orders global memory, so each wave first waits for every load it has in flight;
// a kernel whose waves share data only through LDS uses this one, and loads it issued ahead of their
// use (a table run wanted at the end) stay in flight across the barrier.  The memory clobber keeps the
// compiler from moving any memory access across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <bool LDS_ONLY>
__device__ __forceinline__ void workgroup_barrier() {
  if constexpr (LDS_ONLY) lds_barrier();
  else __syncthreads();
}

// Exclusive scan across a workgroup of NT threads; `total` receives the sum.
// `scratch` must hold NT / 64 ints of LDS.  Contains barriers (LDS-only ones with LDS_ONLY): every
// thread must call it.
template <int NT, bool LDS_ONLY = false>
__device__ __forceinline__ int block_exclusive_scan(int v, int *scratch, int &total) {
  constexpr int kWaves = NT / kWave;
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  int inc = wave_inclusive_scan(v);
  if (lane == kWave - 1) scratch[wave] = inc;
  workgroup_barrier<LDS_ONLY>();
  int base = 0, sum = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    int s = scratch[w];
    base += (w < wave) ? s : 0;
    sum += s;
  }
  workgroup_barrier<LDS_ONLY>();
  total = sum;
  return base + inc - v;
}

// Sum across a workgroup of NT threads (every thread receives it).  Contains barriers.
template <int NT, typename T>
__device__ __forceinline__ T block_sum(T v, T *scratch) {
  constexpr int kWaves = NT / kWave;
  if constexpr (std::is_same<T, int>::value) {
    v = wave_sum_int(v);
  } else if constexpr (std::is_same<T, long long>::value) {
    v = wave_sum_i64(v);
  } else {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += shfl_xor(v, m);
  }
  if (lane_id() == 0) scratch[threadIdx.x / kWave] = v;
  __syncthreads();
  T s = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) s += scratch[w];
  __syncthreads();
  return s;
}

}  // namespace ekv
