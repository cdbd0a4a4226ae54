// The `uniform` budget split and per-row ranking, on the device.
// Semantics: Controller._allocate's pins and budget (observe/controller.py:398-451), then
// allocate(..., "uniform") (observe/allocation.py:55-91) with Request.shares / pinned_mask
// (observe/allocation.py:39-52).
//
// One workgroup per row.  Every workgroup first recomputes, from the per-row block counts, the
// budget, the pinned floor and the largest-remainder quota of its own row: the quotas are
// floor(free * open_i / open_total) in IEEE double (Python's int / int true division is the
// correctly rounded quotient, and so is the double division of these exactly representable
// operands), and the `free - sum(floor)` leftover blocks go to the rows ranked first by
// (-(exact_i - floor_i), i).  That is O(rows) work per workgroup and needs no second kernel.
// The row then keeps its quota of open blocks by (share desc, block index asc), found by an
// 8-bit radix select over order-preserving keys in LDS and a prefix count of the tied keys.
//
// Keys.  The reference ranks `max(s, 0) / total` in float64 with a stable argsort.  For float32
// scores this order equals the order of max(s, 0) itself: distinct float32 values differ by at
// least 2^-24 relative and the float64 division by one positive total rounds at 2^-53, so it
// can neither merge nor swap them.  The special totals are reproduced: a NaN score makes
// every share NaN (all tie -> index order); a +inf score makes the total +inf, so the finite
// blocks get share 0 (tie, first) and the +inf blocks NaN (last); a total <= 0 gives equal
// shares (index order).
#pragma clang fp contract(off)

#include <math.h>

#include "ekv_common.hpp"

namespace ekv {
namespace rank {

constexpr int kThreads = 512;
constexpr int kMaxWidth = 12288;  // 5 bytes of LDS per block
constexpr uint32_t kClosed = 0xFFFFFFFFu;  // key of a block that is not open

struct Params {
  const float *scores;
  int64_t scores_stride;
  const int32_t *blocks;
  const uint8_t *measured;
  const uint8_t *pinned;
  int64_t pinned_stride;
  const int32_t *pin_from;
  int32_t recent;
  const uint8_t *released;
  int64_t released_stride;
  const int32_t *counts;  // [rows][2] existing and pinned-existing blocks, when masks are given
  int32_t rows, width;
  double fraction;
  int64_t budget_in;
  uint8_t *keep;
  int64_t keep_stride;
  int64_t *summary;
};

struct RowInfo {
  int n;        // blocks of the row, clipped to the width
  int part;     // takes part in the allocation
  int pin_at;   // structural pins: block 0 and blocks >= pin_at
  int exist;    // blocks that still exist
  int pinned;   // pinned blocks that exist
};

__device__ __forceinline__ RowInfo row_info(const Params &p, int r) {
  RowInfo ri;
  ri.n = min(max(p.blocks[r], 0), p.width);
  ri.part = (p.measured == nullptr || p.measured[r] != 0) && ri.n > 0;
  int a = max(0, ri.n - 1 - p.recent);  // controller.py:422
  if (p.pin_from != nullptr) a = min(a, min(max(p.pin_from[r], 0), ri.n));  // controller.py:424
  ri.pin_at = a;
  if (p.counts != nullptr) {
    ri.exist = p.counts[2 * r];
    ri.pinned = p.counts[2 * r + 1];
  } else {
    ri.exist = ri.n;
    ri.pinned = ri.n == 0 ? 0 : (ri.n - a) + (a > 0 ? 1 : 0);
  }
  return ri;
}

__device__ __forceinline__ bool is_pinned(const Params &p, const RowInfo &ri, int r, int b) {
  if (p.pinned != nullptr) return p.pinned[(int64_t)r * p.pinned_stride + b] != 0;
  return b == 0 || b >= ri.pin_at;
}

__device__ __forceinline__ bool exists(const Params &p, int r, int b) {
  return p.released == nullptr || p.released[(int64_t)r * p.released_stride + b] == 0;
}

// Existing and pinned-existing blocks of each row, when explicit masks are given.
__global__ __launch_bounds__(256) void count_kernel(const Params p, int32_t *counts) {
  __shared__ int s_red[256 / kWave];
  const int r = blockIdx.x;
  const RowInfo ri = row_info(p, r);
  int ex = 0, pn = 0;
  for (int b = threadIdx.x; b < ri.n; b += 256) {
    if (exists(p, r, b)) {
      ++ex;
      pn += is_pinned(p, ri, r, b) ? 1 : 0;
    }
  }
  ex = block_sum<256>(ex, s_red);
  pn = block_sum<256>(pn, s_red);
  if (threadIdx.x == 0) {
    counts[2 * r] = ex;
    counts[2 * r + 1] = pn;
  }
}

__global__ __launch_bounds__(kThreads) void rank_kernel(const Params p) {
  extern __shared__ uint32_t s_keys[];  // [width] keys, then [width] keep bytes
  __shared__ long long s_red64[kThreads / kWave];
  __shared__ int s_red[kThreads / kWave];
  __shared__ int s_scan[kThreads / kWave];
  __shared__ int s_hist[256];
  __shared__ int s_digit, s_krem;
  uint8_t *s_keep = (uint8_t *)(s_keys + p.width);

  const int row = blockIdx.x;
  const int tid = threadIdx.x;

  // ---- totals over every row: controller.py:435-437, allocation.py:57-67 -----------------
  long long total = 0, floor_pins = 0, sizes = 0, open_total = 0, nreq = 0;
  for (int r = tid; r < p.rows; r += kThreads) {
    const RowInfo ri = row_info(p, r);
    if (!ri.part) continue;
    total += ri.n;
    floor_pins += ri.pinned;
    sizes += ri.exist;
    open_total += ri.exist - ri.pinned;
    nreq += 1;
  }
  total = block_sum<kThreads>(total, s_red64);
  floor_pins = block_sum<kThreads>(floor_pins, s_red64);
  sizes = block_sum<kThreads>(sizes, s_red64);
  open_total = block_sum<kThreads>(open_total, s_red64);
  nreq = block_sum<kThreads>(nreq, s_red64);

  long long budget = p.budget_in;
  if (budget < 0) {
    const long long want = (long long)ceil(p.fraction * (double)total);
    budget = want > floor_pins ? want : floor_pins;
  }
  const bool error = floor_pins > budget && budget < sizes;  // allocation.py:64-65
  const bool keep_all = budget >= sizes;                      // allocation.py:66-67
  const long long free_blocks = budget - floor_pins;
  if (row == 0 && tid == 0 && p.summary != nullptr) {
    p.summary[0] = budget;
    p.summary[1] = total;
    p.summary[2] = floor_pins;
    p.summary[3] = error ? 1 : 0;
    p.summary[4] = nreq;
    p.summary[5] = free_blocks;
  }

  const RowInfo me = row_info(p, row);
  uint8_t *keep_row = p.keep + (int64_t)row * p.keep_stride;
  if (!me.part || error) {  // rows without evidence read in full, controller.py:401
    for (int b = tid; b < p.width; b += kThreads) keep_row[b] = 1;
    return;
  }

  // ---- this row's quota: largest remainder in IEEE double, allocation.py:79-86 ---------------
  const long long my_open = me.exist - me.pinned;
  long long quota = 0;
  if (keep_all) {
    quota = my_open;
  } else {
    const double my_exact = open_total > 0 ? (double)(free_blocks * my_open) / (double)open_total : 0.0;
    const long long my_floor = (long long)my_exact;
    const double my_frac = my_exact - (double)my_floor;
    long long floors = 0, ahead = 0;
    for (int r = tid; r < p.rows; r += kThreads) {
      const RowInfo ri = row_info(p, r);
      if (!ri.part) continue;
      const long long open = ri.exist - ri.pinned;
      const double exact = open_total > 0 ? (double)(free_blocks * open) / (double)open_total : 0.0;
      const long long fl = (long long)exact;
      const double frac = exact - (double)fl;
      floors += fl;
      ahead += (frac > my_frac || (frac == my_frac && r < row)) ? 1 : 0;
    }
    floors = block_sum<kThreads>(floors, s_red64);
    ahead = block_sum<kThreads>(ahead, s_red64);
    const long long leftover = free_blocks - floors;
    quota = my_floor + (ahead < leftover ? 1 : 0);
  }

  // ---- key mode of the row's shares: allocation.py:46-52 over the existing blocks -----------
  const float *srow = p.scores + (int64_t)row * p.scores_stride;
  int has_nan = 0, has_inf = 0, has_pos = 0;
  for (int b = tid; b < me.n; b += kThreads) {
    if (!exists(p, row, b)) continue;
    const float s = srow[b];
    has_nan |= __builtin_isnan(s) ? 1 : 0;
    has_inf |= (__builtin_isinf(s) && s > 0.0f) ? 1 : 0;
    has_pos |= s > 0.0f ? 1 : 0;
  }
  has_nan = block_sum<kThreads>(has_nan, s_red);
  has_inf = block_sum<kThreads>(has_inf, s_red);
  has_pos = block_sum<kThreads>(has_pos, s_red);
  const int mode = has_nan ? 0 : (has_inf ? 2 : (has_pos ? 1 : 0));  // 0 tie, 1 by value, 2 inf last

  // ---- keys of the open blocks, and the pinned / released part of the keep row -------------
  int open_count = 0;
  for (int b = tid; b < p.width; b += kThreads) {
    uint32_t key = kClosed;
    uint8_t k = 1;
    if (b < me.n) {
      if (!exists(p, row, b)) {
        k = 0;
      } else if (!is_pinned(p, me, row, b)) {
        k = 0;  // decided below
        const float s = srow[b];
        if (mode == 1) key = s > 0.0f ? __builtin_bit_cast(uint32_t, s) : 0u;
        else if (mode == 2) key = (__builtin_isinf(s) && s > 0.0f) ? 0u : 1u;
        else key = 0u;
        ++open_count;
      }
    }
    s_keys[b] = key;
    s_keep[b] = k;
  }
  open_count = block_sum<kThreads>(open_count, s_red);
  // (block_sum ends with a barrier, so the LDS rows are complete)

  if (quota >= open_count) {
    for (int b = tid; b < me.n; b += kThreads)
      if (s_keys[b] != kClosed) s_keep[b] = 1;
  } else if (quota > 0) {
    // radix select of the quota-th largest key, 8 bits at a time from the top
    uint32_t prefix = 0, mask = 0;
    int k_rem = (int)quota;
    for (int shift = 24; shift >= 0; shift -= 8) {
      if (tid < 256) s_hist[tid] = 0;
      __syncthreads();
      for (int b = tid; b < me.n; b += kThreads) {
        const uint32_t key = s_keys[b];
        if (key != kClosed && (key & mask) == prefix) atomicAdd(&s_hist[(key >> shift) & 255], 1);
      }
      __syncthreads();
      // thread t looks at digit 255 - t: an inclusive scan gives the count of digits >= it
      const int h = tid < 256 ? s_hist[255 - tid] : 0;
      int scan_total;
      const int before = block_exclusive_scan<kThreads>(h, s_scan, scan_total);
      if (tid < 256 && before < k_rem && before + h >= k_rem) {
        s_digit = 255 - tid;
        s_krem = k_rem - before;
      }
      __syncthreads();
      prefix |= (uint32_t)s_digit << shift;
      mask |= 255u << shift;
      k_rem = s_krem;
      __syncthreads();
    }
    // keep every key above the threshold and the first k_rem equal keys by block index
    const int chunk = (me.n + kThreads - 1) / kThreads;
    const int b0 = tid * chunk, b1 = min(b0 + chunk, me.n);
    int eq = 0;
    for (int b = b0; b < b1; ++b) eq += s_keys[b] == prefix ? 1 : 0;
    int eq_total;
    int rank_eq = block_exclusive_scan<kThreads>(eq, s_scan, eq_total);
    for (int b = b0; b < b1; ++b) {
      const uint32_t key = s_keys[b];
      if (key == kClosed) continue;
      if (key > prefix) {
        s_keep[b] = 1;
      } else if (key == prefix) {
        if (rank_eq < k_rem) s_keep[b] = 1;
        ++rank_eq;
      }
    }
  }
  __syncthreads();
  for (int b = tid; b < p.width; b += kThreads) keep_row[b] = s_keep[b];
}

}  // namespace rank
}  // namespace ekv

using namespace ekv;

extern "C" int ekv_rank_uniform(const float *scores, int64_t scores_stride, const int32_t *blocks,
                                const uint8_t *measured, const uint8_t *pinned, int64_t pinned_stride,
                                const int32_t *pin_from, int32_t recent_blocks, const uint8_t *released,
                                int64_t released_stride, int32_t rows, int32_t width, double fraction,
                                int64_t budget, uint8_t *keep, int64_t keep_stride, int64_t *summary,
                                void *stream) {
  return ekv_rank_uniform_ws(scores, scores_stride, blocks, measured, pinned, pinned_stride, pin_from,
                             recent_blocks, released, released_stride, rows, width, fraction, budget, keep,
                             keep_stride, summary, nullptr, stream);
}

extern "C" int ekv_rank_uniform_ws(const float *scores, int64_t scores_stride, const int32_t *blocks,
                                   const uint8_t *measured, const uint8_t *pinned, int64_t pinned_stride,
                                   const int32_t *pin_from, int32_t recent_blocks, const uint8_t *released,
                                   int64_t released_stride, int32_t rows, int32_t width, double fraction,
                                   int64_t budget, uint8_t *keep, int64_t keep_stride, int64_t *summary,
                                   int32_t *workspace, void *stream) {
  if (scores == nullptr || blocks == nullptr || keep == nullptr)
    return fail(EKV_EINVAL, "ekv_rank_uniform: null pointer");
  if (rows < 0 || width < 1 || width > rank::kMaxWidth)
    return fail(EKV_EINVAL, "ekv_rank_uniform: rows %d, width %d (at most %d)", rows, width, rank::kMaxWidth);
  if (recent_blocks < 0) return fail(EKV_EINVAL, "ekv_rank_uniform: recent_blocks %d < 0", recent_blocks);
  if (budget < 0 && !(fraction > 0.0 && fraction <= 1.0))
    return fail(EKV_EINVAL, "ekv_rank_uniform: the budget fraction %g is not in (0, 1]", fraction);
  if ((pinned != nullptr || released != nullptr) && workspace == nullptr)
    return fail(EKV_EINVAL, "ekv_rank_uniform: pinned or released masks need a workspace of 2 * rows ints");
  if (rows == 0) return EKV_OK;
  rank::Params p{};
  p.scores = scores;
  p.scores_stride = scores_stride;
  p.blocks = blocks;
  p.measured = measured;
  p.pinned = pinned;
  p.pinned_stride = pinned_stride;
  p.pin_from = pin_from;
  p.recent = recent_blocks;
  p.released = released;
  p.released_stride = released_stride;
  p.counts = nullptr;
  p.rows = rows;
  p.width = width;
  p.fraction = fraction;
  p.budget_in = budget;
  p.keep = keep;
  p.keep_stride = keep_stride;
  p.summary = summary;
  if (pinned != nullptr || released != nullptr) {
    hipLaunchKernelGGL(rank::count_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, p, workspace);
    int rc = check_hip(hipGetLastError(), "ekv_rank_uniform count launch");
    if (rc != EKV_OK) return rc;
    p.counts = workspace;
  }
  const size_t lds = (size_t)width * sizeof(uint32_t) + (size_t)width;
  hipLaunchKernelGGL(rank::rank_kernel, dim3(rows), dim3(rank::kThreads), lds, (hipStream_t)stream, p);
  return check_hip(hipGetLastError(), "ekv_rank_uniform launch");
}
