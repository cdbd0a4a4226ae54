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

// ---- NumPy's sum of n values get(i), by a workgroup of NT threads; every thread returns it -----
// The same runs, leaves and combination as numpy_sum, evaluated in parallel over the recursion's
// tree.  The tree has at most kPairDepth + 1 levels, so its nodes fit a heap of 255 entries (node v's
// halves are 2v and 2v + 1); thread v - 1 finds node v by walking from the run down the bits of v,
// and it is a leaf when its length is at most 128 (or it lies at the last level), absent when an
// ancestor is a leaf.  Eight consecutive threads take a leaf of at least 8 values, thread k adding
// values k, k + 8, ... of its first len - len % 8 in order (NumPy's eight accumulators); the
// accumulators then combine as ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7)) over lane exchanges
// (IEEE addition commutes, so lanes k and k ^ 1 hold the same bits of a pair's sum), and thread 0 of
// the eight adds the leaf's last len % 8 values in order (all of a leaf shorter than 8, from 0.0).
// The inner nodes then add their halves' sums, a level at a time from the deepest.  Each thread
// loads the values of two leaves' accumulators before it adds any, so with NT = 256 a run of 8192
// values costs one memory latency.  get(i) is also called for i = 0 when n is 0.  Contains barriers:
// every thread of the workgroup calls it.
constexpr int kPairNodes = 1 << (kPairDepth + 1);  // heap slots 1 .. 255
struct PairwiseLds {
  int start[kMaxLeaves], len[kMaxLeaves], node_of[kMaxLeaves];
  double node[kPairNodes];
  int scan[16];
};

template <int NT, class Get>
__device__ double block_numpy_sum(Get get, int n, PairwiseLds &lds) {
  static_assert(NT % kWave == 0 && NT >= kPairNodes && NT <= 1024, "whole waves, a thread per tree node");
  constexpr int kPer = 16;  // values per accumulator in a leaf of at most 128
  const int t = threadIdx.x, k = t & 7;
  const int v = t + 1;  // this thread's tree node (heap numbering), when v < kPairNodes
  const int depth = v < kPairNodes ? 31 - __clz(v) : 0;
  double total = 0.0;
  for (int c0 = 0; c0 < max(n, 1); c0 += kChunk) {
    const int run = n > 0 ? min(n - c0, kChunk) : 0;
    // node v of this run's tree: its values [vs, vs + vlen), and whether it is a leaf or an inner node
    int vs = c0, vlen = run;
    bool exists = v < kPairNodes;
    for (int i = depth - 1; i >= 0 && exists; --i) {
      if (vlen <= 128) {
        exists = false;  // an ancestor is a leaf
      } else {
        const int n2 = (vlen / 2) & ~7;
        if ((v >> i) & 1) {
          vs += n2;
          vlen -= n2;
        } else {
          vlen = n2;
        }
      }
    }
    const bool leaf = exists && (vlen <= 128 || depth == kPairDepth);
    const bool inner = exists && !leaf;
    int leaves;
    const int li = block_exclusive_scan<NT, true>(leaf ? 1 : 0, lds.scan, leaves);
    if (leaf) {
      lds.start[li] = vs;
      lds.len[li] = vlen;
      lds.node_of[li] = v;
    }
    lds_barrier();
    const int chains = 8 * leaves;  // a multiple of 8: the eight threads of a leaf go together
    for (int c = t; c < chains; c += 2 * NT) {
      double x[2][kPer], tail[2][7];
      int m[2], rest[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {  // chains c and c + NT: every load issued before any add
        const int cc = c + h * NT;
        const int j = cc < chains ? cc >> 3 : 0;
        const int s = lds.start[j], len = cc < chains ? lds.len[j] : 0;
        m[h] = len >> 3;
        rest[h] = len - 8 * m[h];
        // every load issued, the unused ones reading value c0 (a load under a condition is followed
        // by a wait for every load before it)
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
          const double y = get(i < m[h] ? s + k + 8 * i : c0);
          x[h][i] = i < m[h] ? y : 0.0;
        }
#pragma unroll
        for (int i = 0; i < 7; ++i) {
          const bool used = k == 0 && i < rest[h];
          const double y = get(used ? s + 8 * m[h] + i : c0);
          tail[h][i] = used ? y : 0.0;
        }
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int cc = c + h * NT;
        if (cc >= chains) continue;  // uniform over the eight threads of a leaf
        double res = 0.0;
        if (m[h] > 0) {
          double r = x[h][0];
#pragma unroll
          for (int i = 1; i < kPer; ++i)
            if (i < m[h]) r += x[h][i];
          r = r + __shfl_xor(r, 1, kWave);
          r = r + __shfl_xor(r, 2, kWave);
          r = r + __shfl_xor(r, 4, kWave);
          res = r;
        }
        if (k == 0) {
#pragma unroll
          for (int i = 0; i < 7; ++i)
            if (i < rest[h]) res += tail[h][i];
          lds.node[lds.node_of[cc >> 3]] = res;
        }
      }
    }
    // the inner nodes, deepest first: left half + right half, as the recursion returns them
#pragma unroll
    for (int d = kPairDepth - 1; d >= 0; --d) {
      lds_barrier();
      if (inner && depth == d) lds.node[v] = lds.node[2 * v] + lds.node[2 * v + 1];
    }
    lds_barrier();
    total += lds.node[1];  // every thread adds the runs in order
    lds_barrier();         // node 1 is read before the next run writes it
  }
  return total;
}

}  // namespace ekv
