// Shared definitions of libekv_hip: status codes, error text, device properties, and the
// wave64 / workgroup primitives the kernels use (gfx950: 64-lane wavefronts).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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
__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += shfl_xor(v, m);
  return v;
}
__device__ __forceinline__ long long wave_sum_i64(long long v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += shfl_xor(v, m);
  return v;
}

// Inclusive scan of `v` across the 64 lanes of a wave.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  const int lane = lane_id();
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    int up = __shfl_up(v, d, kWave);
    if (lane >= d) v += up;
  }
  return v;
}

// Exclusive scan across a workgroup of NT threads; `total` receives the sum.
// `scratch` must hold NT / 64 ints of LDS.  Contains barriers: every thread must call it.
template <int NT>
__device__ __forceinline__ int block_exclusive_scan(int v, int *scratch, int &total) {
  constexpr int kWaves = NT / kWave;
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  int inc = wave_inclusive_scan(v);
  if (lane == kWave - 1) scratch[wave] = inc;
  __syncthreads();
  int base = 0, sum = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    int s = scratch[w];
    base += (w < wave) ? s : 0;
    sum += s;
  }
  __syncthreads();
  total = sum;
  return base + inc - v;
}

// Sum across a workgroup of NT threads (every thread receives it).  Contains barriers.
template <int NT, typename T>
__device__ __forceinline__ T block_sum(T v, T *scratch) {
  constexpr int kWaves = NT / kWave;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += shfl_xor(v, m);
  if (lane_id() == 0) scratch[threadIdx.x / kWave] = v;
  __syncthreads();
  T s = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) s += scratch[w];
  __syncthreads();
  return s;
}

}  // namespace ekv
