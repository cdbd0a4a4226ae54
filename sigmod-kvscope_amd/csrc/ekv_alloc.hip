// The `sum` and `maxmin` budget splits across requests, on the device.
// Semantics: allocate(..., "sum" | "maxmin"), observe/allocation.py:55-166, with Request.shares
// and pinned_mask (observe/allocation.py:39-52).
//
// Every request's shares are max(s, 0) / total in float64, total being NumPy's sum of the clamped
// scores (equal shares 1 / n when total <= 0).  The totals are reproduced bit for bit: NumPy adds
// the pairwise sums of successive runs of at most 8192 values (its reduction buffer) to 0.0, a
// run's pairwise sum taking pieces of at most 128 values with eight accumulators and splitting
// longer pieces at n / 2 rounded down to a multiple of 8 (NumPy's published pairwise summation,
// numpy/_core/src/umath/loops_utils.h.src; checked against NumPy 2.2.6) -- which a wave evaluates
// with the leaves summed in parallel and combined in the recursion's order.
//
// sum: keep the `free` unpinned blocks of highest weight * share, a tie going to the newer block,
// then to the earlier request.  The threshold is found by a radix select over order-preserving
// 64-bit keys of the float64 gains (eight passes of 8 bits over every open block, the gains
// recomputed in each pass), then among the blocks at the threshold by a select over
// (block desc, request asc) (four passes).  All state lives in a caller-provided workspace that a
// kernel clears first, so the launches need no host synchronisation and no memset.
#pragma clang fp contract(off)

#include <math.h>

#include "ekv_common.hpp"

namespace ekv {
namespace alloc {

constexpr int kThreads = 256;
constexpr int kMaxLeaves = 256;  // pairwise leaves of a row of at most 12288 blocks
constexpr int kMaxWidth = 12288;
constexpr int kMaxRows = 65535;  // the tie key holds the request in 16 bits

enum Mode : int { kSelect = 0, kKeepAll = 1, kKeepOpen = 2, kPinnedOnly = 3 };

struct State {
  unsigned long long hist[256];
  unsigned long long prefix, mask, threshold;  // threshold: the gain key at the cut
  long long k_rem, free_blocks, must, sizes, open_total, requests, budget;
  int mode, error;
};

struct RowStat {
  double total;  // NumPy's sum of the clamped scores
  int n, pinned, open, pad;
};

struct Params {
  const double *scores;
  int64_t scores_stride;
  const int32_t *blocks;
  const double *weights;  // per request, or null (1.0)
  const uint8_t *pinned;
  int64_t pinned_stride;
  int32_t rows, width;
  long long budget;
  uint8_t *keep;
  int64_t keep_stride;
  int64_t *summary;
  State *state;
  RowStat *row_stat;
};

__device__ __forceinline__ int row_blocks(const Params &p, int r) { return min(max(p.blocks[r], 0), p.width); }

// Request.pinned_mask: the explicit mask, else the first and the last block
__device__ __forceinline__ bool pinned_at(const Params &p, int r, int b, int n) {
  if (p.pinned != nullptr) return p.pinned[(int64_t)r * p.pinned_stride + b] != 0;
  return b == 0 || b == n - 1;
}

// np.maximum(s, 0.0): NaN stays NaN, -0.0 stays -0.0
__device__ __forceinline__ double clamp0(double s) { return (s >= 0.0 || s != s) ? s : 0.0; }

// ---- NumPy's sum of n values get(i), by one wave; every lane returns it -----------------------
// The reduction hands its inner loop at most kChunk values at a time and adds each run's pairwise
// sum to the result in turn, starting from the identity 0.0.
constexpr int kChunk = 8192;

template <class Get>
__device__ double numpy_sum(Get get, int n, int *s_start, int *s_len, double *s_leaf) {
  const int lane = lane_id();
  __shared__ int s_nleaves;
  if (lane == 0) {  // the leaves of every run, left to right: pieces of at most 128 values
    int leaves = 0;
    for (int c0 = 0; c0 < max(n, 1); c0 += kChunk) {
      int stack_s[16], stack_n[16], sp = 0;
      stack_s[0] = c0;
      stack_n[0] = n > 0 ? min(n - c0, kChunk) : 0;
      while (sp >= 0) {
        const int s = stack_s[sp], len = stack_n[sp];
        --sp;
        if (len <= 128) {
          s_start[leaves] = s;
          s_len[leaves] = len;
          ++leaves;
        } else {
          int n2 = len / 2;
          n2 -= n2 % 8;
          stack_s[++sp] = s + n2;  // right half second
          stack_n[sp] = len - n2;
          stack_s[++sp] = s;
          stack_n[sp] = n2;
        }
      }
    }
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
  double total = 0.0;
  if (lane == 0) {  // every run combined in its recursion's order, the runs added in turn
    int next = 0;
    for (int c0 = 0; c0 < max(n, 1); c0 += kChunk) {
      int st_len[16], st_stage[16];
      double st_left[16];
      int sp = 0;
      double ret = 0.0;
      st_len[0] = n > 0 ? min(n - c0, kChunk) : 0;
      st_stage[0] = 0;
      while (sp >= 0) {
        const int len = st_len[sp];
        if (len <= 128) {
          ret = s_leaf[next++];
          --sp;
          continue;
        }
        int n2 = len / 2;
        n2 -= n2 % 8;
        if (st_stage[sp] == 0) {
          st_stage[sp] = 1;
          ++sp;
          st_len[sp] = n2;
          st_stage[sp] = 0;
        } else if (st_stage[sp] == 1) {
          st_left[sp] = ret;
          st_stage[sp] = 2;
          ++sp;
          st_len[sp] = len - n2;
          st_stage[sp] = 0;
        } else {
          ret = st_left[sp] + ret;
          --sp;
        }
      }
      total += ret;
    }
  }
  return __shfl(total, 0, kWave);
}

// order-preserving key of a float64 gain: larger gain, larger key; both zeros one key; NaN the
// lowest key (1); key 0 marks a block that is not open
__device__ __forceinline__ unsigned long long gain_key(double g) {
  if (g != g) return 1ull;
  if (g == 0.0) g = 0.0;
  const unsigned long long bits = __builtin_bit_cast(unsigned long long, g);
  const unsigned long long k = (bits >> 63) ? ~bits : (bits | (1ull << 63));
  return k < 2ull ? 2ull : k;  // keep 0 and 1 free (only the most negative NaN-free values would map there)
}

__device__ __forceinline__ double share_of(const Params &p, const RowStat &st, int r, int b) {
  if (!(st.total > 0.0) && st.total == st.total) return 1.0 / (double)max(st.n, 1);  // total <= 0
  return clamp0(p.scores[(int64_t)r * p.scores_stride + b]) / st.total;
}

__device__ __forceinline__ double weight_of(const Params &p, int r) { return p.weights != nullptr ? p.weights[r] : 1.0; }

__global__ __launch_bounds__(kThreads) void clear_kernel(State *s) {
  unsigned long long *w = (unsigned long long *)s;
  for (int i = threadIdx.x; i < (int)(sizeof(State) / 8); i += kThreads) w[i] = 0ull;
}

// one wave per request: its total, its pinned and open blocks
__global__ __launch_bounds__(kWave) void prepare_kernel(const Params p) {
  __shared__ int s_start[kMaxLeaves], s_len[kMaxLeaves];
  __shared__ double s_leaf[kMaxLeaves];
  const int r = blockIdx.x;
  const int lane = lane_id();
  const int n = row_blocks(p, r);
  const double *srow = p.scores + (int64_t)r * p.scores_stride;
  const double total = numpy_sum([&](int i) { return clamp0(srow[i]); }, n, s_start, s_len, s_leaf);
  int pinned = 0;
  for (int b = lane; b < n; b += kWave) pinned += pinned_at(p, r, b, n) ? 1 : 0;
  pinned = wave_sum_int(pinned);
  if (lane == 0) {
    RowStat st;
    st.total = total;
    st.n = n;
    st.pinned = pinned;
    st.open = n - pinned;
    st.pad = 0;
    p.row_stat[r] = st;
    atomicAdd((unsigned long long *)&p.state->must, (unsigned long long)pinned);
    atomicAdd((unsigned long long *)&p.state->sizes, (unsigned long long)n);
    atomicAdd((unsigned long long *)&p.state->open_total, (unsigned long long)(n - pinned));
    atomicAdd((unsigned long long *)&p.state->requests, 1ull);
  }
}

// the budget's mode (allocation.py:57-76) and the select's start
__global__ void decide_kernel(const Params p) {
  if (threadIdx.x != 0) return;
  State *s = p.state;
  const long long must = s->must, sizes = s->sizes, budget = p.budget;
  s->budget = budget;
  s->error = (must > budget && budget < sizes) ? 1 : 0;
  const long long free_blocks = budget - must;
  s->free_blocks = free_blocks;
  int mode;
  if (budget >= sizes) mode = kKeepAll;
  else if (free_blocks <= 0) mode = kPinnedOnly;
  else if (free_blocks >= s->open_total) mode = kKeepOpen;
  else mode = kSelect;
  s->mode = mode;
  s->k_rem = free_blocks;
  s->prefix = 0ull;
  s->mask = 0ull;
  if (p.summary != nullptr) {
    p.summary[0] = budget;
    p.summary[1] = sizes;
    p.summary[2] = must;
    p.summary[3] = s->error;
    p.summary[4] = s->requests;
    p.summary[5] = free_blocks;
  }
}

// the select's two keys of an open block
__device__ __forceinline__ unsigned long long key_at(const Params &p, const RowStat &st, int r, int b) {
  return gain_key(weight_of(p, r) * share_of(p, st, r, b));
}
__device__ __forceinline__ unsigned long long tie_key(int r, int b) {
  return ((unsigned long long)b << 16) | (unsigned long long)(0xFFFF - r);  // newer block, then earlier request
}

// one radix pass: the digit histogram of the open blocks whose key matches the prefix so far
// (tie passes: the blocks at the gain threshold, over the tie key)
template <bool TIE>
__global__ __launch_bounds__(kThreads) void hist_kernel(const Params p, int shift) {
  __shared__ unsigned int s_hist[256];
  const State *s = p.state;
  if (s->mode != kSelect || s->error) return;
  s_hist[threadIdx.x] = 0u;
  __syncthreads();
  const unsigned long long prefix = s->prefix, mask = s->mask, threshold = s->threshold;
  const int r = blockIdx.y;
  const RowStat st = p.row_stat[r];
  for (int b = blockIdx.x * kThreads + threadIdx.x; b < st.n; b += gridDim.x * kThreads) {
    if (pinned_at(p, r, b, st.n)) continue;
    const unsigned long long k = key_at(p, st, r, b);
    unsigned long long key = k;
    if constexpr (TIE) {
      if (k != threshold) continue;
      key = tie_key(r, b);
    }
    if ((key & mask) == prefix) atomicAdd(&s_hist[(key >> shift) & 255], 1u);
  }
  __syncthreads();
  const unsigned int c = s_hist[threadIdx.x];
  if (c) atomicAdd(&p.state->hist[threadIdx.x], (unsigned long long)c);
}

// the digit where the k_rem-th largest key lies; the next pass's prefix
__global__ __launch_bounds__(kThreads) void pick_kernel(const Params p, int shift, int last_gain_pass) {
  __shared__ long long s_scan[kThreads / kWave];
  State *s = p.state;
  if (s->mode != kSelect || s->error) return;
  const int t = threadIdx.x;
  const long long h = (long long)s->hist[255 - t];  // thread t looks at digit 255 - t
  // inclusive scan over the threads: the keys at digits >= 255 - t
  const int lane = lane_id(), wave = t / kWave;
  long long inc = h;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const long long up = __shfl_up(inc, d, kWave);
    if (lane >= d) inc += up;
  }
  if (lane == kWave - 1) s_scan[wave] = inc;
  __syncthreads();
  long long base = 0;
  for (int w = 0; w < wave; ++w) base += s_scan[w];
  inc += base;
  const long long before = inc - h;
  const long long k_rem = s->k_rem;
  __syncthreads();
  if (before < k_rem && inc >= k_rem) {
    s->prefix |= (unsigned long long)(255 - t) << shift;
    s->k_rem = k_rem - before;
  }
  s->hist[t] = 0ull;
  __syncthreads();
  if (t == 0) {
    s->mask |= 255ull << shift;
    if (last_gain_pass) {  // the gain threshold is complete: the tie passes start
      s->threshold = s->prefix;
      s->prefix = 0ull;
      s->mask = 0ull;
    }
  }
}

__global__ __launch_bounds__(kThreads) void sum_keep_kernel(const Params p) {
  const int r = blockIdx.x;
  const State *s = p.state;
  const RowStat st = p.row_stat[r];
  const int mode = s->mode;
  const bool error = s->error != 0;
  const unsigned long long threshold = s->threshold, tie = s->prefix;
  uint8_t *krow = p.keep + (int64_t)r * p.keep_stride;
  for (int b = threadIdx.x; b < p.width; b += kThreads) {
    uint8_t k;
    if (error || b >= st.n || mode == kKeepAll || pinned_at(p, r, b, st.n)) k = 1;
    else if (mode == kKeepOpen) k = 1;
    else if (mode == kPinnedOnly) k = 0;
    else {
      const unsigned long long key = key_at(p, st, r, b);
      k = (key > threshold || (key == threshold && tie_key(r, b) >= tie)) ? 1 : 0;
    }
    krow[b] = k;
  }
}

}  // namespace alloc
}  // namespace ekv

using namespace ekv;

extern "C" size_t ekv_rank_sum_workspace(int32_t rows) {
  return sizeof(alloc::State) + (size_t)(rows > 0 ? rows : 0) * sizeof(alloc::RowStat) + 256;
}

extern "C" int ekv_rank_sum(const double *scores, int64_t scores_stride, const int32_t *blocks,
                            const double *weights, const uint8_t *pinned, int64_t pinned_stride, int32_t rows,
                            int32_t width, int64_t budget, uint8_t *keep, int64_t keep_stride, int64_t *summary,
                            void *workspace, size_t workspace_bytes, void *stream) {
  if (scores == nullptr || blocks == nullptr || keep == nullptr || workspace == nullptr)
    return fail(EKV_EINVAL, "ekv_rank_sum: null pointer");
  if (rows < 0 || rows > alloc::kMaxRows || width < 1 || width > alloc::kMaxWidth)
    return fail(EKV_EINVAL, "ekv_rank_sum: rows %d (max %d), width %d (max %d)", rows, alloc::kMaxRows, width,
                alloc::kMaxWidth);
  if (budget < 0) return fail(EKV_EINVAL, "ekv_rank_sum: the budget cannot be negative");
  if (workspace_bytes < ekv_rank_sum_workspace(rows))
    return fail(EKV_EINVAL, "ekv_rank_sum: a workspace of %zu bytes is below the %zu needed", workspace_bytes,
                ekv_rank_sum_workspace(rows));
  if (rows == 0) return EKV_OK;
  alloc::Params p{};
  p.scores = scores;
  p.scores_stride = scores_stride;
  p.blocks = blocks;
  p.weights = weights;
  p.pinned = pinned;
  p.pinned_stride = pinned_stride;
  p.rows = rows;
  p.width = width;
  p.budget = budget;
  p.keep = keep;
  p.keep_stride = keep_stride;
  p.summary = summary;
  const uintptr_t base = ((uintptr_t)workspace + 255) & ~(uintptr_t)255;
  p.state = (alloc::State *)base;
  p.row_stat = (alloc::RowStat *)(base + sizeof(alloc::State));
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(alloc::clear_kernel, dim3(1), dim3(alloc::kThreads), 0, s, p.state);
  hipLaunchKernelGGL(alloc::prepare_kernel, dim3(rows), dim3(kWave), 0, s, p);
  hipLaunchKernelGGL(alloc::decide_kernel, dim3(1), dim3(kWave), 0, s, p);
  const dim3 grid((width + alloc::kThreads - 1) / alloc::kThreads, rows);
  for (int pass = 0; pass < 8; ++pass) {  // the gain threshold, 8 bits at a time from the top
    hipLaunchKernelGGL(alloc::hist_kernel<false>, grid, dim3(alloc::kThreads), 0, s, p, 56 - 8 * pass);
    hipLaunchKernelGGL(alloc::pick_kernel, dim3(1), dim3(alloc::kThreads), 0, s, p, 56 - 8 * pass, pass == 7);
  }
  for (int pass = 0; pass < 4; ++pass) {  // among the blocks at the threshold: newer block, earlier request
    hipLaunchKernelGGL(alloc::hist_kernel<true>, grid, dim3(alloc::kThreads), 0, s, p, 24 - 8 * pass);
    hipLaunchKernelGGL(alloc::pick_kernel, dim3(1), dim3(alloc::kThreads), 0, s, p, 24 - 8 * pass, 0);
  }
  hipLaunchKernelGGL(alloc::sum_keep_kernel, dim3(rows), dim3(alloc::kThreads), 0, s, p);
  return check_hip(hipGetLastError(), "ekv_rank_sum launch");
}
