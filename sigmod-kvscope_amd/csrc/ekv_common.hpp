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
