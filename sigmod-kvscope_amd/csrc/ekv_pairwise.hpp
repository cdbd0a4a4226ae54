// NumPy's float64 sum, reproduced bit for bit on the device (shared by the `uniform`, `sum` and
// `maxmin` rankings, whose shares divide by it: observe/allocation.py:46-52).
//
// NumPy adds the pairwise sums of successive runs of at most 8192 values (its reduction buffer) to
// 0.0; a run's pairwise sum takes pieces of at most 128 values with eight accumulators and splits
// longer pieces at n / 2 rounded down to a multiple of 8 (NumPy's published pairwise summation,
// numpy/_core/src/umath/loops_utils.h.src; checked against NumPy 2.2.6).  One wave evaluates it:
// the leaves are summed in parallel and combined in the recursion's order.
#pragma once

#include "ekv_common.hpp"

namespace ekv {

constexpr int kMaxLeaves = 128;  // pairwise leaves of one run of at most kChunk values (65 at most)

// np.maximum(s, 0.0): NaN stays NaN, -0.0 stays -0.0
__device__ __forceinline__ double clamp0(double s) { return (s >= 0.0 || s != s) ? s : 0.0; }

// ---- NumPy's sum of n values get(i), by one wave; every lane returns it -----------------------
// The reduction hands its inner loop at most kChunk values at a time and adds each run's pairwise
// sum to the result in turn, starting from the identity 0.0.  A run's recursion splits a piece of
// more than 128 values at n2 = len / 2 rounded down to a multiple of 8; the left part is at most
// len / 2 and the right one at most len / 2 + 8, so a run of at most 8192 values reaches pieces of
// at most 128 within kPairDepth = 7 levels.  The recursion is unrolled at compile time (no stack
// arrays, whose dynamic indexing made one lane's walk of the tree take tens of microseconds).
constexpr int kChunk = 8192;
constexpr int kPairDepth = 7;

template <int D>
__device__ __forceinline__ void plan_leaves(int s, int len, int &leaves, int *s_start, int *s_len) {
  if constexpr (D > 0) {
    if (len > 128) {
      int n2 = len / 2;
      n2 -= n2 % 8;
      plan_leaves<D - 1>(s, n2, leaves, s_start, s_len);
      plan_leaves<D - 1>(s + n2, len - n2, leaves, s_start, s_len);
      return;
    }
  }
  s_start[leaves] = s;
  s_len[leaves] = len;
  ++leaves;
}

template <int D>
__device__ __forceinline__ double combine_leaves(int len, int &next, const double *s_leaf) {
  if constexpr (D > 0) {
    if (len > 128) {
      int n2 = len / 2;
      n2 -= n2 % 8;
      const double left = combine_leaves<D - 1>(n2, next, s_leaf);
      const double right = combine_leaves<D - 1>(len - n2, next, s_leaf);
      return left + right;
    }
  }
  return s_leaf[next++];
}

template <class Get>
__device__ double numpy_sum(Get get, int n, int *s_start, int *s_len, double *s_leaf) {
  const int lane = lane_id();
  __shared__ int s_nleaves;
  double total = 0.0;
  // the runs one at a time: each run's leaves (at most 65, of at most 128 values each; fewer for
  // a short run) planned by lane 0, summed by the wave, combined in the recursion's order by lane 0
  // and added to the total in turn
  for (int c0 = 0; c0 < max(n, 1); c0 += kChunk) {
    const int run = n > 0 ? min(n - c0, kChunk) : 0;
    if (lane == 0) {
      int leaves = 0;
      plan_leaves<kPairDepth>(c0, run, leaves, s_start, s_len);
      s_nleaves = leaves;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const int leaves = s_nleaves;
    for (int j = lane; j < leaves; j += kWave) {  // a leaf: eight accumulators, then the rest in order
      const int s = s_start[j], len = s_len[j];
      double res;
      if (len < 8) {
        res = 0.0;
        for (int i = 0; i < len; ++i) res += get(s + i);
      } else {
        double r[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) r[k] = get(s + k);
        int i = 8;
        for (; i < len - (len % 8); i += 8) {
#pragma unroll
          for (int k = 0; k < 8; ++k) r[k] += get(s + i + k);
        }
        res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        for (; i < len; ++i) res += get(s + i);
      }
      s_leaf[j] = res;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (lane == 0) {
      int next = 0;
      total += combine_leaves<kPairDepth>(run, next, s_leaf);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // the leaf arrays are free for the next run
  }
  return __shfl(total, 0, kWave);
}

}  // namespace ekv
