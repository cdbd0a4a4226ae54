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
// 8-bit radix select over order-preserving keys (a row's keys stay in registers, block
// tid + 512 i in slot i of thread tid; 256-bin LDS histograms, scanned by one wave) and a
// ballot / scan count of the tied keys before each block.
//
// Keys.  The reference ranks `max(s, 0) / total` in float64 with a stable argsort.  For float32
// scores this order equals the order of max(s, 0) itself: distinct float32 values differ by at
// least 2^-24 relative and the float64 division by one positive total rounds at 2^-53, so it
// can neither merge nor swap them.  The special totals are reproduced: a NaN score makes
// every share NaN (all tie -> index order); a +inf score makes the total +inf, so the finite
// blocks get share 0 (tie, first) and the +inf blocks NaN (last); a total <= 0 gives equal
// shares (index order).
//
// float64 scores (ekv_rank_uniform64) rank the float64 shares themselves: there two distinct
// scores can divide to one share and tie, so a per-row kernel first takes each request's total
// over its existing blocks with NumPy's own pairwise summation, and the ranking keys are the shares
// clamp(s) / total (1 / n when total <= 0; NaN last), 64 bits wide, selected 8 bits a pass.
#pragma clang fp contract(off)

#include <limits.h>
#include <math.h>

#include <type_traits>

#include "ekv_common.hpp"
#include "ekv_pairwise.hpp"

namespace ekv {
namespace rank {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxPer = 24;                  // blocks per thread, block tid + kThreads i
constexpr int kMaxWidth = kThreads * kMaxPer;  // 12288: a row lives in registers
static_assert(kMaxWidth < 65536, "a row's block counts fit 16-bit fields");
constexpr int kRowRegs = 4;                  // rows per thread whose open count stays in registers

struct Params {
  const float *scores;
  int64_t scores_stride;
  const double *scores64;  // float64 scores (ekv_rank_uniform64), with each request's NumPy total
  const double *totals;
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
  // the view built from the keep (ekv_rank_uniform_view only)
  const int32_t *table;
  int64_t table_stride;
  const int32_t *seq_lens;
  int32_t block_size;
  int32_t *view_table;
  int64_t view_stride;
  int32_t *view_lens;
  long long *view_counts;  // [rows][5] DecodeView's read counters, accumulated (NULL: none)
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

// row_info from a row's loaded values, without explicit masks: its block count, whether it is
// measured, and its pin start (INT_MAX: none)
__device__ __forceinline__ RowInfo row_info_of(const Params &p, int blocks, bool measured, int pin_from) {
  RowInfo ri;
  ri.n = min(max(blocks, 0), p.width);
  ri.part = measured && ri.n > 0;
  ri.pin_at = min(max(0, ri.n - 1 - p.recent), min(max(pin_from, 0), ri.n));  // controller.py:422-424
  ri.exist = ri.n;
  ri.pinned = ri.n == 0 ? 0 : (ri.n - ri.pin_at) + (ri.pin_at > 0 ? 1 : 0);
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

// Each request's float64 total for ekv_rank_uniform64: NumPy's sum of the clamped scores of its
// existing blocks, in block order (Request.shares over the scores the controller passes, which
// leave released blocks out: observe/allocation.py:46-52, observe/controller.py:425-431).  One
// wave per row; with a released mask the existing blocks are listed in LDS first.
__global__ __launch_bounds__(kWave) void total64_kernel(const Params p, double *totals) {
  __shared__ int s_start[kMaxLeaves], s_len[kMaxLeaves];
  __shared__ double s_leaf[kMaxLeaves];
  __shared__ int s_map[kMaxWidth];
  const int r = blockIdx.x;
  const int lane = lane_id();
  const int n = min(max(p.blocks[r], 0), p.width);
  const double *srow = p.scores64 + (int64_t)r * p.scores_stride;
  double total;
  if (p.released == nullptr) {
    total = numpy_sum([&](int i) { return clamp0(srow[i]); }, n, s_start, s_len, s_leaf);
  } else {
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    int m = 0;
    for (int base = 0; base < n; base += kWave) {
      const int b = base + lane;
      const bool e = b < n && exists(p, r, b);
      const uint64_t ballot = __ballot(e);
      if (e) s_map[m + __popcll(ballot & below)] = b;
      m += __popcll(ballot);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    total = numpy_sum([&](int i) { return clamp0(srow[s_map[i]]); }, m, s_start, s_len, s_leaf);
  }
  if (lane == 0) totals[r] = total;
}

// Sum of N values over the workgroup in one pass (every thread receives the sums).
template <int N>
__device__ __forceinline__ void block_sums(long long (&v)[N], long long (*scratch)[kWaves]) {
  const int wave = threadIdx.x / kWave;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    v[j] = wave_sum_i64(v[j]);
    if (lane_id() == 0) scratch[j][wave] = v[j];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < N; ++j) {
    long long s = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) s += scratch[j][w];
    v[j] = s;
  }
  __syncthreads();
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 16-byte loads of one row through a buffer descriptor whose extent is the row's first `entries`
// 4-byte words: a group at or past the extent reads as zeros (the memory unit's range check), so
// every load is issued without a per-thread branch, and none can reach past the row.  The caller
// keeps the extent a multiple of 4 words from a 16-byte aligned base, so that no group straddles it.
// A negative `first` is a group outside the extent too (its offset is set past any extent): it reads
// zeros, and a store there writes nothing.
struct RowLoader {
  __amdgpu_buffer_rsrc_t rsrc;
  __device__ __forceinline__ RowLoader(const void *base, int entries)
      : rsrc(__builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, entries * 4, kRawBufferFormat)) {}
  static __device__ __forceinline__ int offset(int first) { return first >= 0 ? first * 4 : kPastExtent; }
  __device__ __forceinline__ u32x4 load(int first) const {
    return __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset(first), 0, 0);
  }
  __device__ __forceinline__ void store(int first, u32x4 v) const {
    __builtin_amdgcn_raw_buffer_store_b128(v, rsrc, offset(first), 0, 0);
  }
  // 32-bit data format, the word selects left at zero (the format word of a raw gfx9 buffer)
  static constexpr int kRawBufferFormat = 0x00020000;
  static constexpr int kPastExtent = INT_MIN;  // 2^31 as the unsigned offset: past every extent
};

// The view row's tail.  compact_block_table keeps no block at or past the row's block count nv
// (block_view.py:49-51) and orders the row stably, kept first: every kept block lies below nv, so each
// block from nv on stays at its own index.  From the first whole 16-byte group at or past nv (the
// value returned) the view row is the table row; the width when the rows are not whole 16-byte groups.
__device__ __forceinline__ int view_tail_from(const Params &p, int row, int L) {
  const int W = p.width;
  const uintptr_t trow = (uintptr_t)(p.table + (int64_t)row * p.table_stride);
  const uintptr_t vrow = (uintptr_t)(p.view_table + (int64_t)row * p.view_stride);
  const long long n64 = L > 0 ? ((long long)L + p.block_size - 1) / p.block_size : 0;  // block_view.py:49
  const bool whole_groups = (W & 3) == 0 && ((trow | vrow) & 15) == 0;
  return whole_groups ? (int)min((n64 + 3) & ~3LL, (long long)W) : W;
}

// compact_block_table (runtime/block_view.py:36-56) of the row on the keep bytes in LDS, which the
// ranking has just decided: keep'[b] = (keep[b] | b == 0 | b == n-1) & b < n for n = ceil(L / bs)
// from the row's token length; the row's entries stably partitioned, keep' first, then the rest,
// each in original order.  Thread t takes the contiguous run of PER entries from t * PER (16-byte
// table loads), one block scan of the threads' kept counts places every entry, the row is assembled
// in LDS and written with 16-byte stores.  (Loading the run at the kernel's entry, beside the
// scores, was slower: 49 against 46 us at 1024 rows x 8192 blocks.)
// With 16-byte loads (width a multiple of 4, the row aligned) only the groups below `extent` (a
// multiple of 4, at most the width) are read; the rest of the run reads as zeros.
template <int PER>
__device__ __forceinline__ void load_run(const Params &p, int row, int32_t (&entry)[PER], int extent) {
  static_assert(PER % 4 == 0, "runs of whole 16-byte groups");
  const int W = p.width;
  const int32_t *trow = p.table + (int64_t)row * p.table_stride;
  const int b0 = threadIdx.x * PER;
  if ((W & 3) == 0 && ((uintptr_t)trow & 15) == 0) {
    // one test for the whole workgroup; the groups past the extent read as zeros
    const RowLoader rl(trow, extent);
#pragma unroll
    for (int g = 0; g < PER / 4; ++g) {
      const u32x4 t4 = rl.load(b0 + 4 * g);
      entry[4 * g] = (int32_t)t4.x;
      entry[4 * g + 1] = (int32_t)t4.y;
      entry[4 * g + 2] = (int32_t)t4.z;
      entry[4 * g + 3] = (int32_t)t4.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < PER; ++i) entry[i] = b0 + i < W ? trow[b0 + i] : 0;
  }
}

template <int PER>
__device__ __forceinline__ void view_row(const Params &p, int row, int L, const long long (&c_in)[5],
                                         const int32_t (&entry)[PER], const uint8_t *s_keep, int32_t *s_out,
                                         int *s_scan) {
  const int tid = threadIdx.x;
  const int W = p.width;
  const long long n64 = L > 0 ? ((long long)L + p.block_size - 1) / p.block_size : 0;  // block_view.py:49
  const int n = n64 > W + 1LL ? W + 1 : (int)n64;
  const int b0 = tid * PER;
  uint32_t kept_bits = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int b = b0 + i;
    const bool k = b < W && s_keep[b] != 0;
    kept_bits |= (b < W && (k || b == 0 || b == n - 1) && b < n) ? (1u << i) : 0u;
  }
  int total_kept;
  int before = block_exclusive_scan<kThreads>(__popc(kept_bits), s_scan, total_kept);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    // kept: at its rank among the kept; dropped: after the kept ones, in order (one store either way)
    const int b = b0 + i;
    const bool kept = (kept_bits >> i) & 1u;
    if (b < W) s_out[kept ? before : total_kept + (b - before)] = entry[i];
    before += kept ? 1 : 0;
  }
  __syncthreads();
  int32_t *vrow = p.view_table + (int64_t)row * p.view_stride;
  if (((uintptr_t)vrow & 15) == 0) {
    for (int q = tid; 4 * q < W; q += kThreads) {
      if (4 * q + 3 < W) {
        *reinterpret_cast<int4 *>(vrow + 4 * q) =
            make_int4(s_out[4 * q], s_out[4 * q + 1], s_out[4 * q + 2], s_out[4 * q + 3]);
      } else {
        for (int b = 4 * q; b < W; ++b) vrow[b] = s_out[b];
      }
    }
  } else {
    for (int b = tid; b < W; b += kThreads) vrow[b] = s_out[b];
  }
  if (tid == 0) {  // block_view.py:53-55
    const int bs = p.block_size;
    const int last = L - (int)(n64 - 1) * bs;
    const int view_len = n64 > 0 ? (total_kept - 1) * bs + last : 0;
    p.view_lens[row] = view_len;
    if (p.view_counts != nullptr) {
      // DecodeView._count for a live decoding row outside the audit (block_view.py:313-329): blocks
      // read, blocks in full, none audited, reads of a whole row, none expired
      const long long read = view_len > 0 ? ((long long)view_len + bs - 1) / bs : 0;
      long long *c = p.view_counts + 5LL * row;
      long long before[5];
#pragma unroll
      for (int k = 0; k < 5; ++k) before[k] = PER <= 16 ? c_in[k] : c[k];
      c[0] = before[0] + read;
      c[1] = before[1] + n64;
      c[2] = before[2];
      c[3] = before[3] + (view_len == L ? read : 0);
      c[4] = before[4];
    }
  }
}

// PER: blocks per thread (the row's width is at most kThreads * PER).  VIEW: also build the row's
// view from the keep it decides (ekv_rank_uniform_view).
template <int PER, bool VIEW = false, bool F64 = false>
__global__ __launch_bounds__(kThreads) void rank_kernel(const Params p) {
  constexpr int kPer = PER;
  using Score = typename std::conditional<F64, double, float>::type;
  using Key = typename std::conditional<F64, unsigned long long, uint32_t>::type;
  constexpr Key kClosedKey = ~Key(0);  // key of a block that is not open
  constexpr int kPasses = F64 ? 8 : 4;  // 8-bit digits
  __shared__ uint8_t s_keep[VIEW ? kPer * kThreads : 1];
  __shared__ int32_t s_out[VIEW ? kPer * kThreads : 1];
  __shared__ long long s_red[5][kWaves];
  __shared__ int s_hist[2][256];
  __shared__ int s_count[kPer * kWaves];  // equal keys per (load, wave), then their exclusive scan
  __shared__ int s_scan[kWaves];
  __shared__ int s_digit, s_krem, s_whole;

  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;

  // ---- the row's blocks: scores and masks into registers (block tid + kThreads i) -----------
  // The loads are issued first and bounded by the width only, so that they overlap the row
  // counts' loads and reductions below instead of waiting for them.
  const RowInfo me = row_info(p, row);
  const int view_len_in = VIEW ? p.seq_lens[row] : 0;
  // the row's own counter slot, loaded with the row's other loads (thread 0 updates it); at 24 blocks
  // per thread its registers would cost a workgroup per CU, so it is loaded at the end there
  long long c_in[5] = {0, 0, 0, 0, 0};
  if (VIEW && kPer <= 16 && tid == 0 && p.view_counts != nullptr) {
#pragma unroll
    for (int k = 0; k < 5; ++k) c_in[k] = p.view_counts[5LL * row + k];
  }
  const Score *srow;
  if constexpr (F64) srow = p.scores64 + (int64_t)row * p.scores_stride;
  else srow = p.scores + (int64_t)row * p.scores_stride;
  const double row_total = F64 ? p.totals[row] : 0.0;
  Score sv[kPer];
  uint32_t gone_bits = 0, pin_mask_bits = 0;  // released / explicitly pinned, from the masks
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int b = tid + i * kThreads;
    const bool in = b < p.width;
    sv[i] = in ? srow[b] : Score(0);
    if (p.released != nullptr)
      gone_bits |= (in && p.released[(int64_t)row * p.released_stride + b] != 0) ? (1u << i) : 0u;
    if (p.pinned != nullptr)
      pin_mask_bits |= (in && p.pinned[(int64_t)row * p.pinned_stride + b] != 0) ? (1u << i) : 0u;
  }

  // ---- totals over every row: controller.py:435-437, allocation.py:57-67 -----------------
  // the open blocks of the first kRowRegs * kThreads rows stay in registers for the quota pass
  long long open_reg[kRowRegs];
  long long t5[5] = {0, 0, 0, 0, 0};  // total, floor_pins, sizes, open_total, requests
#pragma unroll
  for (int i = 0; i < kRowRegs; ++i) {
    const int r = tid + i * kThreads;
    open_reg[i] = -1;  // not taking part
    if (r < p.rows) {
      const RowInfo ri = row_info(p, r);
      if (ri.part) {
        t5[0] += ri.n;
        t5[1] += ri.pinned;
        t5[2] += ri.exist;
        t5[3] += ri.exist - ri.pinned;
        t5[4] += 1;
        open_reg[i] = ri.exist - ri.pinned;
      }
    }
  }
  for (int r = tid + kRowRegs * kThreads; r < p.rows; r += kThreads) {
    const RowInfo ri = row_info(p, r);
    if (!ri.part) continue;
    t5[0] += ri.n;
    t5[1] += ri.pinned;
    t5[2] += ri.exist;
    t5[3] += ri.exist - ri.pinned;
    t5[4] += 1;
  }
  block_sums(t5, s_red);
  const long long total = t5[0], floor_pins = t5[1], sizes = t5[2], open_total = t5[3], nreq = t5[4];

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

  uint8_t *keep_row = p.keep + (int64_t)row * p.keep_stride;
  if (!me.part || error) {  // rows without evidence read in full, controller.py:401
    for (int b = tid; b < p.width; b += kThreads) {
      keep_row[b] = 1;
      if constexpr (VIEW) s_keep[b] = 1;
    }
    if constexpr (VIEW) {
      int32_t entry[kPer];
      load_run<kPer>(p, row, entry, p.width);
      __syncthreads();
      view_row<kPer>(p, row, view_len_in, c_in, entry, s_keep, s_out, s_scan);
    }
    return;
  }

  // the row's existing and pinned blocks (is_pinned / exists over the loaded masks)
  uint32_t exist_bits = 0, pin_bits = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int b = tid + i * kThreads;
    const bool in = b < me.n;
    const bool pinned = p.pinned != nullptr ? ((pin_mask_bits >> i) & 1u) != 0 : (b == 0 || b >= me.pin_at);
    exist_bits |= (in && !((gone_bits >> i) & 1u)) ? (1u << i) : 0u;
    pin_bits |= (in && pinned) ? (1u << i) : 0u;
  }

  // ---- this row's quota: largest remainder in IEEE double, allocation.py:79-86 ---------------
  const long long my_open = me.exist - me.pinned;
  const double my_exact = open_total > 0 ? (double)(free_blocks * my_open) / (double)open_total : 0.0;
  const long long my_floor = (long long)my_exact;
  const double my_frac = my_exact - (double)my_floor;
  // [0] floors, [1] rows ahead in the leftover order, [2] four counts of the row's blocks in
  // 16-bit fields (a row has at most kMaxWidth < 2^16 blocks): existing blocks with a NaN score,
  // with a +inf score, with a positive score, and open blocks
  long long q3[3] = {0, 0, 0};
  if (!keep_all) {
    auto visit = [&](int r, long long open) {
      const double exact = open_total > 0 ? (double)(free_blocks * open) / (double)open_total : 0.0;
      const long long fl = (long long)exact;
      const double frac = exact - (double)fl;
      q3[0] += fl;
      q3[1] += (frac > my_frac || (frac == my_frac && r < row)) ? 1 : 0;
    };
#pragma unroll
    for (int i = 0; i < kRowRegs; ++i)
      if (open_reg[i] >= 0) visit(tid + i * kThreads, open_reg[i]);
    for (int r = tid + kRowRegs * kThreads; r < p.rows; r += kThreads) {
      const RowInfo ri = row_info(p, r);
      if (ri.part) visit(r, ri.exist - ri.pinned);
    }
  }
  // key mode of the row's shares: allocation.py:46-52 over the existing blocks
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    if (!F64 && ((exist_bits >> i) & 1u)) {
      const float s = (float)sv[i];
      q3[2] += __builtin_isnan(s) ? 1ll : 0ll;
      q3[2] += (__builtin_isinf(s) && s > 0.0f) ? 1ll << 16 : 0ll;
      q3[2] += s > 0.0f ? 1ll << 32 : 0ll;
    }
    q3[2] += (((exist_bits & ~pin_bits) >> i) & 1u) ? 1ll << 48 : 0ll;
  }
  block_sums(q3, s_red);
  long long quota;
  if (keep_all) {
    quota = my_open;
  } else {
    const long long leftover = free_blocks - q3[0];
    quota = my_floor + (q3[1] < leftover ? 1 : 0);
  }
  const long long has_nan = q3[2] & 0xffff, has_inf = (q3[2] >> 16) & 0xffff, has_pos = (q3[2] >> 32) & 0xffff;
  const long long open_count = (q3[2] >> 48) & 0xffff;
  const int mode = has_nan ? 0 : (has_inf ? 2 : (has_pos ? 1 : 0));  // 0 tie, 1 by value, 2 inf last

  // ---- keys of the open blocks (order-preserving, larger first), kClosedKey elsewhere -------
  Key key[kPer];
  if constexpr (F64) {
    // the request's float64 shares, allocation.py:46-52: clamp(s) / total, or 1 / n for a total <= 0
    // (n its existing blocks); a NaN share sorts last (key 0), +0 and -0 are one key
    const double uniform = 1.0 / (double)(me.exist > 0 ? me.exist : 1);
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      key[i] = kClosedKey;
      if (((exist_bits & ~pin_bits) >> i) & 1u) {
        double v = row_total <= 0.0 ? uniform : clamp0((double)sv[i]) / row_total;
        if (v == 0.0) v = 0.0;
        key[i] = v != v ? 0ull : __builtin_bit_cast(unsigned long long, v) + 1ull;
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      key[i] = kClosedKey;
      if (((exist_bits & ~pin_bits) >> i) & 1u) {
        const float s = (float)sv[i];
        if (mode == 1) key[i] = s > 0.0f ? __builtin_bit_cast(uint32_t, s) : 0u;
        else if (mode == 2) key[i] = (__builtin_isinf(s) && s > 0.0f) ? 0u : 1u;
        else key[i] = 0u;
      }
    }
  }

  // keep: blocks past the row's end 1, released 0, pinned 1, open blocks decided here
  uint32_t open_keep = 0;
  if (quota >= open_count) {
    open_keep = ~0u;
  } else if (quota > 0) {
    // radix select of the quota-th largest key, 8 bits at a time from the top; the histogram is
    // double-buffered so that clearing the next one needs no extra barrier.  The select stops
    // early once the quota ends exactly at the end of a digit's bucket: every key with that
    // prefix is kept and no tie needs ranking.
    Key prefix = 0, mask = 0;
    int k_rem = (int)quota;
    bool whole = false;
    if (tid < 256) s_hist[0][tid] = 0;
    __syncthreads();
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
      const int shift = 8 * (kPasses - 1) - 8 * pass;
      int *hist = s_hist[pass & 1];
#pragma unroll
      for (int i = 0; i < kPer; ++i)
        if (key[i] != kClosedKey && (key[i] & mask) == prefix) atomicAdd(&hist[(int)(key[i] >> shift) & 255], 1);
      if (tid < 256) s_hist[(pass & 1) ^ 1][tid] = 0;
      __syncthreads();
      if (wave == 0) {
        // lane l holds digits 255 - 4l .. 252 - 4l; a scan over the lanes counts the keys above
        int c[4], s4 = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          c[j] = hist[255 - 4 * lane - j];
          s4 += c[j];
        }
        const int inc = wave_inclusive_scan(s4);
        int acc = inc - s4;
        if (acc < k_rem && inc >= k_rem) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (acc < k_rem && acc + c[j] >= k_rem) {
              s_digit = 255 - 4 * lane - j;
              s_krem = k_rem - acc;
              s_whole = acc + c[j] == k_rem ? 1 : 0;
            }
            acc += c[j];
          }
        }
      }
      __syncthreads();
      prefix |= (Key)s_digit << shift;
      mask |= (Key)255 << shift;
      k_rem = s_krem;
      whole = __builtin_amdgcn_readfirstlane(s_whole) != 0;
      if (whole) break;
    }
    if (whole) {
      // the quota is every key whose top bits are at least the prefix
#pragma unroll
      for (int i = 0; i < kPer; ++i)
        open_keep |= (key[i] != kClosedKey && (key[i] & mask) >= prefix) ? (1u << i) : 0u;
    } else {
      // keep every key above the threshold and the first k_rem equal keys by block index
      const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
      int eq_rank[kPer];
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const uint64_t eq = __ballot(key[i] == prefix);
        eq_rank[i] = __popcll(eq & below);
        if (lane == 0) s_count[i * kWaves + wave] = __popcll(eq);
      }
      __syncthreads();
      const int v = tid < kPer * kWaves ? s_count[tid] : 0;
      int eq_total;
      const int excl = block_exclusive_scan<kThreads>(v, s_scan, eq_total);
      if (tid < kPer * kWaves) s_count[tid] = excl;
      __syncthreads();
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const bool kept = key[i] != kClosedKey &&
                          (key[i] > prefix || (key[i] == prefix && s_count[i * kWaves + wave] + eq_rank[i] < k_rem));
        open_keep |= kept ? (1u << i) : 0u;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int b = tid + i * kThreads;
    if (b >= p.width) continue;
    uint8_t k;
    if (b >= me.n) k = 1;
    else if (!((exist_bits >> i) & 1u)) k = 0;
    else if ((pin_bits >> i) & 1u) k = 1;
    else k = (open_keep >> i) & 1u;
    keep_row[b] = k;
    if constexpr (VIEW) s_keep[b] = k;
  }
  if constexpr (VIEW) {
    int32_t entry[kPer];
    load_run<kPer>(p, row, entry, p.width);
    __syncthreads();
    view_row<kPer>(p, row, view_len_in, c_in, entry, s_keep, s_out, s_scan);
  }
}


// The fused ranking and view for float scores without masks (ekv_rank_uniform_view), sized for four
// 512-thread workgroups per compute unit (at most 64 VGPRs), so that 1024 rows run in one round.
// Every workgroup takes the controller's budget and its row's largest-remainder quota from every
// row's counts (32-bit sums: the launch routes rows * width >= 2^31 to rank_kernel), keeps the
// quota's best open blocks by a radix select, and builds the view on that keep.  Thread t owns the
// contiguous run of blocks t * PER .. t * PER + PER - 1 of both the scores and the table: both are
// read with 16-byte loads (the scores' live part only), the keep decisions stay in the thread's
// registers for the view, and the ties of the select and the view's placement are each one
// workgroup scan of the threads' counts.  During the select the keys wait in LDS, lane-consecutive
// (slot i of thread t at i * kThreads + t), which leaves the registers to the table run, and the
// same LDS then holds the view row being assembled.  The decisions are those of rank_kernel<PER,
// true>.  (One workgroup computing every row's quota first was slower: 11 us for it against the ~5
// us of the sums it saves each workgroup.)
template <int PER>
__device__ __forceinline__ void load_scores_run(const Params &p, int row, int n, uint32_t (&key)[PER]) {
  const float *srow = p.scores + (int64_t)row * p.scores_stride;
  const int b0 = threadIdx.x * PER;
  if ((p.width & 3) == 0 && ((uintptr_t)srow & 15) == 0) {
    // one test for the whole workgroup; the extent is the live blocks rounded up to a whole group
    // (at most the width), the groups past it read as zeros
    const RowLoader rl(srow, min((n + 3) & ~3, p.width));
#pragma unroll
    for (int g = 0; g < PER / 4; ++g) {
      const u32x4 v = rl.load(b0 + 4 * g);
      key[4 * g] = v.x;
      key[4 * g + 1] = v.y;
      key[4 * g + 2] = v.z;
      key[4 * g + 3] = v.w;
    }
  } else {
    // the run's own entries, clipped to the row's last (block 0 for an empty row)
    const float *run = srow + min(b0, max(n - 1, 0));
    const int last = max(n - 1 - b0, 0);
#pragma unroll
    for (int i = 0; i < PER; ++i) key[i] = __builtin_bit_cast(uint32_t, run[min(i, last)]);
  }
}

// Sum of N values over a workgroup of NT threads in one pass (every thread receives the sums).
template <int NT, int N, class T, bool LDS_ONLY = false>
__device__ __forceinline__ void block_sums_n(T (&v)[N], T (*scratch)[NT / kWave]) {
  constexpr int NW = NT / kWave;
  const int wave = threadIdx.x / kWave;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    if constexpr (std::is_same<T, int>::value) v[j] = wave_sum_int(v[j]);
    else v[j] = wave_sum_i64(v[j]);
    if (lane_id() == 0) scratch[j][wave] = v[j];
  }
  workgroup_barrier<LDS_ONLY>();
#pragma unroll
  for (int j = 0; j < N; ++j) {
    T s = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) s += scratch[j][w];
    v[j] = s;
  }
  workgroup_barrier<LDS_ONLY>();
}

// bits [0, k) of a word (k clipped to [0, 32]), and bits [lo, hi)
__device__ __forceinline__ uint32_t bits_below(int k) { return k <= 0 ? 0u : (k >= 32 ? ~0u : (1u << k) - 1u); }
__device__ __forceinline__ uint32_t bit_range(int lo, int hi) { return bits_below(hi) & ~bits_below(lo); }

// max of an int over a wave (signed or as unsigned), every lane receiving it: DPP within each
// 16-lane row, then the four rows' lanes 0
template <bool SIGNED>
__device__ __forceinline__ int wave_max_int(int v) {
  auto mx = [](int a, int b) { return SIGNED ? max(a, b) : (int)max((uint32_t)a, (uint32_t)b); };
  v = mx(v, dpp_move<0xB1>(v));
  v = mx(v, dpp_move<0x4E>(v));
  v = mx(v, dpp_move<0x124>(v));
  v = mx(v, dpp_move<0x128>(v));
  return mx(mx(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
            mx(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// The budget of the controller's rule over every row taking part (controller.py:435-437,
// allocation.py:64-67), from the rows' block counts.
struct Budget {
  long long total, floor_pins, sizes, open_total, nreq, budget, free_blocks;
  bool error, keep_all;
};

// The quota of one row: largest remainder in IEEE double (allocation.py:79-86).
struct Quota {
  long long open, floor;
  double frac;
};

__device__ __forceinline__ Quota quota_of(const Budget &bg, const RowInfo &me) {
  Quota q;
  q.open = me.exist - me.pinned;
  const double exact = bg.open_total > 0 ? (double)(bg.free_blocks * q.open) / (double)bg.open_total : 0.0;
  q.floor = (long long)exact;
  q.frac = exact - (double)q.floor;
  return q;
}

// The key mode of a row's shares (allocation.py:46-52) from two maxima over its live scores (0 past
// the row): of the bits without the sign, above +inf's 0x7f800000 only for a NaN, and of the bits as
// a signed int, which is +inf's at most without a NaN and above 0 for a positive score.
// 0: all tie, 1: by value, 2: +inf last.
__device__ __forceinline__ int key_mode(uint32_t mag, int sgn) {
  return mag > 0x7f800000u ? 0 : (sgn == 0x7f800000 ? 2 : (sgn > 0 ? 1 : 0));
}

// One row's keep (the quota's best open blocks) and its view, from the raw score bits and the
// table run the thread holds: the radix select over the keys in LDS, the keep bytes, then
// compact_block_table (runtime/block_view.py:36-56) on that keep, the row assembled in the same LDS.
template <int PER>
__device__ __forceinline__ void keep_and_view(const Params &p, int row, const RowInfo &me, int L,
                                              const uint32_t (&key)[PER], bool decide, long long quota, int mode, uint32_t *s_row,
                                              int *s_hist, int *s_scan, int *s_sel) {
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const int W = p.width;
  const int b0 = tid * PER;
  // open blocks: existing (every block below n) and not pinned (block 0, blocks >= pin_at <= n);
  // the thread's run is contiguous, so they are one range of its bits
  const uint32_t open_bits = bit_range(max(1, b0) - b0, min(me.pin_at - b0, PER));
  uint32_t keep_bits = ~0u;  // rows without evidence read in full, controller.py:401
  const bool any_open = open_bits != 0u;
  const int open_count = (int)(me.exist - me.pinned);
  const bool select = decide && quota > 0 && quota < open_count;
  const int copy = lane & 3;
  if (decide) {
    // keys, larger first: an open block's is at least 1 (by value: the score's bits + 1 for a
    // positive score, else 1; inf last: 1 for +inf, else 2; tie: 1), a closed block's is 0 and is
    // never counted.  Slot i of thread t sits at i * kThreads + t: lane-consecutive, free of bank
    // conflicts.  A thread whose run holds no open block (past a short row) neither writes nor
    // reads its slots.  When the select runs, the keys' top digits are counted as they are
    // written, so that its first pass reads nothing back.
    if (any_open) {
      // the key of a raw score under the row's mode, the mode's test outside the loop
      const uint32_t fin_k = mode == 2 ? 2u : 1u;
      const bool by_value = mode == 1;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const uint32_t k = by_value ? (uint32_t)max((int)key[i], 0) + 1u : (key[i] == 0x7f800000u ? 1u : fin_k);
        const bool open = (open_bits >> i) & 1u;
        s_row[i * kThreads + tid] = open ? k : 0u;
        if (select && open) atomicAdd(&s_hist[(k >> 24) * 4 + copy], 1);
      }
    }
  }
  // the table run, requested once the raw scores are no longer needed (with both held, from the
  // kernel's entry on, the registers spill); the barriers up to the view row's assembly order LDS
  // only, so it streams in while the select runs
  int32_t entry[PER];
  load_run<PER>(p, row, entry, W);
  if (decide) {
    uint32_t open_keep = 0;
    if (quota >= open_count) {
      open_keep = ~0u;
    } else if (quota > 0) {
      // radix select of the quota-th largest key over the open blocks, 8 bits at a time from the
      // top; wave 0 scans the counts and clears them for the next pass, and the select stops once
      // the quota ends at the end of a digit's bucket
      uint32_t prefix = 0, mask = 0;
      int k_rem = (int)quota;
      bool whole = false;
#pragma unroll 1
      for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        if (pass > 0 && any_open) {
          // four keys read before their counts are added: an LDS atomic holds back every later
          // LDS read, so reads issued one by one would each wait a full LDS latency
#pragma unroll
          for (int g = 0; g < PER; g += 4) {
            uint32_t kk[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) kk[j] = s_row[(g + j) * kThreads + tid];
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (kk[j] != 0u && (kk[j] & mask) == prefix) atomicAdd(&s_hist[((kk[j] >> shift) & 255) * 4 + copy], 1);
          }
        }
        lds_barrier();
        if (wave == 0) {
          // lane l holds digits 255 - 4l .. 252 - 4l, the four bins' copies 64 contiguous bytes
          // from one address; a scan over the lanes counts the keys above.  (The lane's digits are
          // derived in each pass, not held across the select: the empty asm keeps them from being
          // hoisted out of the loop into registers the table run needs.)
          int l = lane;
          asm volatile("" : "+v"(l));
          int4 *h = reinterpret_cast<int4 *>(&s_hist[4 * (252 - 4 * l)]);
          int c[4], s4 = 0;
#pragma unroll
          for (int j = 0; j < 4; ++j) {  // digit 255 - 4l - j
            const int4 h4 = h[3 - j];
            c[j] = h4.x + h4.y + h4.z + h4.w;
            s4 += c[j];
            asm volatile("" ::: "memory");  // one bin's copies in registers at a time
          }
          const int inc = wave_inclusive_scan(s4);
          int acc = inc - s4;
          if (acc < k_rem && inc >= k_rem) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              if (acc < k_rem && acc + c[j] >= k_rem) {
                s_sel[0] = 255 - 4 * l - j;
                s_sel[1] = k_rem - acc;
                s_sel[2] = acc + c[j] == k_rem ? 1 : 0;
              }
              acc += c[j];
            }
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) h[j] = make_int4(0, 0, 0, 0);  // cleared for the next pass
        }
        lds_barrier();
        prefix |= (uint32_t)s_sel[0] << shift;
        mask |= 255u << shift;
        k_rem = s_sel[1];
        whole = __builtin_amdgcn_readfirstlane(s_sel[2]) != 0;
        if (whole) break;
      }
      if (whole) {
        if (any_open) {
#pragma unroll
          for (int i = 0; i < PER; ++i) {
            const uint32_t k = s_row[i * kThreads + tid];
            open_keep |= (k != 0u && (k & mask) >= prefix) ? (1u << i) : 0u;
          }
        }
      } else {
        // every key above the threshold (at least 1: closed keys are below it) and the first k_rem
        // equal keys by block index: the equal keys before a thread's run are one scan of the
        // threads' counts
        uint32_t eq_bits = 0, above_bits = 0;
        if (any_open) {
#pragma unroll
          for (int i = 0; i < PER; ++i) {
            const uint32_t k = s_row[i * kThreads + tid];
            eq_bits |= k == prefix ? (1u << i) : 0u;
            above_bits |= k > prefix ? (1u << i) : 0u;
          }
        }
        int eq_total;
        int before = block_exclusive_scan<kThreads, true>(__popc(eq_bits), s_scan, eq_total);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const bool eq = (eq_bits >> i) & 1u;
          const bool kept = ((above_bits >> i) & 1u) || (eq && before < k_rem);
          before += eq ? 1 : 0;
          open_keep |= kept ? (1u << i) : 0u;
        }
      }
    }
    keep_bits = ~open_bits | open_keep;  // past the row, pinned: 1; open: decided
  }
  // The view row's tail (view_tail_from) is the table row: the thread's groups there go from its
  // registers to the view row, in place; its other groups are assembled in LDS below.  (Stored before
  // the keep bytes, whose stores a wait for the run's loads would wait for as well.  The tail's
  // start and the rows' addresses are recomputed rather than held across the select, whose registers
  // are all taken: the empty asm hides that the values are the same.)
  L = __builtin_amdgcn_readfirstlane(L);  // both uniform; in scalar registers for the asm
  row = __builtin_amdgcn_readfirstlane(row);
  asm volatile("" : "+s"(L), "+s"(row));
  const int tail_from = view_tail_from(p, row, L);
  {
    const RowLoader tail(p.view_table + (int64_t)row * p.view_stride + tail_from, W - tail_from);
#pragma unroll
    for (int g = 0; g < PER / 4; ++g) {
      const u32x4 v = {(uint32_t)entry[4 * g], (uint32_t)entry[4 * g + 1], (uint32_t)entry[4 * g + 2],
                       (uint32_t)entry[4 * g + 3]};
      tail.store(b0 + 4 * g - tail_from, v);  // below the tail: a negative index, no store
    }
  }
  uint8_t *keep_row = p.keep + (int64_t)row * p.keep_stride;
  if (b0 + PER <= W && ((uintptr_t)(keep_row + b0) & 3) == 0) {
#pragma unroll
    for (int g = 0; g < PER / 4; ++g) {
      const uint32_t k4 = ((keep_bits >> (4 * g)) & 1u) | (((keep_bits >> (4 * g + 1)) & 1u) << 8) |
                          (((keep_bits >> (4 * g + 2)) & 1u) << 16) | (((keep_bits >> (4 * g + 3)) & 1u) << 24);
      *reinterpret_cast<uint32_t *>(keep_row + b0 + 4 * g) = k4;
    }
  } else {
    uint8_t *run = keep_row + b0;
    const int in_row = W - b0;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (i < in_row) run[i] = (keep_bits >> i) & 1u;
  }
  lds_barrier();  // every key is read before the view row overwrites them

  // ---- compact_block_table (runtime/block_view.py:36-56) of the row on that keep, blocks below
  // tail_from (the tail is stored above) ---------------------------------------------------------
  int32_t *s_out = reinterpret_cast<int32_t *>(s_row);
  const int bs = p.block_size;
  const long long n64 = L > 0 ? ((long long)L + bs - 1) / bs : 0;  // block_view.py:49
  const int nv = n64 > W + 1LL ? W + 1 : (int)n64;
  // keep' = (keep | b == 0 | b == nv - 1) & b < min(nv, W), as bits of the thread's run
  const int last_at = nv - 1 - b0;
  const uint32_t kept_bits = (keep_bits | (b0 == 0 ? 1u : 0u) | (last_at >= 0 && last_at < PER ? 1u << last_at : 0u)) &
                             bits_below(min(min(nv, W) - b0, PER));
  int total_kept;
  int before = block_exclusive_scan<kThreads, true>(__popc(kept_bits), s_scan, total_kept);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    // kept: at its rank among the kept; dropped: after the kept ones, in order (one store either way)
    const int b = b0 + i;
    const bool kept = (kept_bits >> i) & 1u;
    if (b < tail_from) s_out[kept ? before : total_kept + (b - before)] = entry[i];
    before += kept ? 1 : 0;
  }
  lds_barrier();
  int32_t *vrow = p.view_table + (int64_t)row * p.view_stride;
  if (((uintptr_t)vrow & 15) == 0) {
    for (int q = tid; 4 * q < tail_from; q += kThreads) {
      if (4 * q + 3 < tail_from) {
        *reinterpret_cast<int4 *>(vrow + 4 * q) =
            make_int4(s_out[4 * q], s_out[4 * q + 1], s_out[4 * q + 2], s_out[4 * q + 3]);
      } else {
        for (int b = 4 * q; b < tail_from; ++b) vrow[b] = s_out[b];
      }
    }
  } else {
    for (int b = tid; b < tail_from; b += kThreads) vrow[b] = s_out[b];
  }
  if (tid == 0) {  // block_view.py:53-55
    const int last = L - (int)(n64 - 1) * bs;
    const int view_len = n64 > 0 ? (total_kept - 1) * bs + last : 0;
    p.view_lens[row] = view_len;
    if (p.view_counts != nullptr) {
      // DecodeView._count for a live decoding row outside the audit (block_view.py:313-329)
      const long long read = view_len > 0 ? ((long long)view_len + bs - 1) / bs : 0;
      long long *c = p.view_counts + 5LL * row;
      c[0] += read;
      c[1] += n64;
      c[3] += view_len == L ? read : 0;
    }
  }
}

// The quota sums of the view build in one pass over the workgroup: v[0 .. NS) summed, then pairs of
// (largest as unsigned, largest as signed).
template <int N, int NS>
__device__ __forceinline__ void quota_reduce(int (&v)[N], int (*scratch)[kWaves]) {
  const int wave = threadIdx.x / kWave;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    if (j < NS) v[j] = wave_sum_int(v[j]);
    else if ((j - NS) % 2 == 0) v[j] = wave_max_int<false>(v[j]);
    else v[j] = wave_max_int<true>(v[j]);
  }
  if (lane_id() == 0) {
#pragma unroll
    for (int j = 0; j < N; ++j) scratch[j][wave] = v[j];
  }
  lds_barrier();
#pragma unroll
  for (int j = 0; j < N; ++j) {
    int r = j < NS ? 0 : ((j - NS) % 2 == 0 ? 0 : INT_MIN);
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const int x = scratch[j][w];
      if (j < NS) r += x;
      else if ((j - NS) % 2 == 0) r = (int)max((uint32_t)r, (uint32_t)x);
      else r = max(r, x);
    }
    v[j] = r;
  }
  lds_barrier();
}

// The uniform ranking and the view in one kernel, one row per workgroup (four per compute unit, 64
// registers a thread).  Every workgroup computes the budget from all rows' counts and its row's quota
// from all rows' open counts (the rows' floors and their order by remainder), then decides and
// compacts its row, the keys in LDS.  The decisions are those of rank_kernel<PER, true>.  (Two rows
// per workgroup, both rows' scores and table runs requested at entry so that the second row's data
// streams in while the first is decided, took 40.5 us against 33.6 us at 1024 rows x 8192 blocks:
// at two workgroups per compute unit the select's barriers and LDS atomics stall the CU.)
template <int PER>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(8, 8))) void rank_view_kernel(
    const Params p) {
  // the row's keys during the select, then the view row being assembled
  __shared__ uint32_t s_row[PER * kThreads];
  __shared__ int s_red[5][kWaves];
  // the select's digit counts: four copies of each bin side by side (bin * 4 + lane % 4), so that
  // the lanes of one instruction that share a digit add to four words, not one
  __shared__ __align__(16) int s_hist[256 * 4];
  __shared__ int s_scan[kWaves];
  __shared__ int s_sel[3];  // the select's digit, remaining count and whether the bucket ends it

  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  if (tid < 256) *reinterpret_cast<int4 *>(&s_hist[4 * tid]) = make_int4(0, 0, 0, 0);  // seen after the first barrier

  // ---- the row's counts and token length, every row's counts for the budget, then the row's
  // live scores ---------------------------------------------------------------------------------
  // Every load is unconditional (an absent array is read through the block counts, in range, and
  // ignored), so none waits inside a branch: the row's own four values, the counts of rows tid and
  // tid + kThreads, then (once the row's block count is in) the row's scores, all in flight at once.
  const uint8_t *measured = p.measured != nullptr ? p.measured : reinterpret_cast<const uint8_t *>(p.blocks);
  const int32_t *pin_from = p.pin_from != nullptr ? p.pin_from : p.blocks;
  const int my_blocks = p.blocks[row];
  const int my_measured = measured[row];
  const int my_pin_from = pin_from[row];
  const int L = p.seq_lens[row];
  const RowInfo me = row_info_of(p, my_blocks, p.measured == nullptr || my_measured != 0,
                                 p.pin_from != nullptr ? my_pin_from : INT_MAX);
  constexpr int kRegRows = 2;  // rows per thread whose open count stays in a register
  int nb[kRegRows], pf[kRegRows], ms[kRegRows];
#pragma unroll
  for (int i = 0; i < kRegRows; ++i) {
    const int r = min(tid + i * kThreads, p.rows - 1);
    nb[i] = p.blocks[r];
    ms[i] = measured[r];
    pf[i] = pin_from[r];
  }
  uint32_t key[PER];  // the raw score bits (past the row: whatever the row holds there)
  load_scores_run<PER>(p, row, __builtin_amdgcn_readfirstlane(me.n), key);
  int open_reg[kRegRows];
  int t5[5] = {0, 0, 0, 0, 0};  // total, floor_pins, sizes, open_total, requests
#pragma unroll
  for (int i = 0; i < kRegRows; ++i) {
    const bool in = tid + i * kThreads < p.rows;
    const RowInfo ri = row_info_of(p, in ? nb[i] : 0, p.measured == nullptr || ms[i] != 0,
                                   p.pin_from != nullptr ? pf[i] : INT_MAX);
    open_reg[i] = -1;  // not taking part
    if (ri.part) {
      t5[0] += ri.n;
      t5[1] += ri.pinned;
      t5[2] += ri.exist;
      t5[3] += ri.exist - ri.pinned;
      t5[4] += 1;
      open_reg[i] = ri.exist - ri.pinned;
    }
  }
  for (int r = tid + kRegRows * kThreads; r < p.rows; r += kThreads) {
    const RowInfo ri = row_info(p, r);
    if (!ri.part) continue;
    t5[0] += ri.n;
    t5[1] += ri.pinned;
    t5[2] += ri.exist;
    t5[3] += ri.exist - ri.pinned;
    t5[4] += 1;
  }
  block_sums_n<kThreads, 5, int, true>(t5, s_red);
  Budget bg;
  bg.total = t5[0];
  bg.floor_pins = t5[1];
  bg.sizes = t5[2];
  bg.open_total = t5[3];
  bg.nreq = t5[4];
  bg.budget = p.budget_in;
  if (bg.budget < 0) {  // controller.py:435-437
    const long long want = (long long)ceil(p.fraction * (double)bg.total);
    bg.budget = want > bg.floor_pins ? want : bg.floor_pins;
  }
  bg.error = bg.floor_pins > bg.budget && bg.budget < bg.sizes;  // allocation.py:64-65
  bg.keep_all = bg.budget >= bg.sizes;                            // allocation.py:66-67
  bg.free_blocks = bg.budget - bg.floor_pins;
  if (blockIdx.x == 0 && tid == 0 && p.summary != nullptr) {
    p.summary[0] = bg.budget;
    p.summary[1] = bg.total;
    p.summary[2] = bg.floor_pins;
    p.summary[3] = bg.error ? 1 : 0;
    p.summary[4] = bg.nreq;
    p.summary[5] = bg.free_blocks;
  }

  // ---- the row's quota and key mode ----------------------------------------------------------
  const bool decide = me.part && !bg.error;
  const Quota q = quota_of(bg, me);
  // [0] floors of every row, [1] rows ahead of this one in the leftover order (int sums: the floors
  // add up to at most the budget), [2] [3] the two maxima of the key mode
  int qs[4] = {0, 0, 0, 0};
  if (decide && !bg.keep_all) {
    auto visit = [&](int r, int open) {
      const double exact = bg.open_total > 0 ? (double)(bg.free_blocks * open) / (double)bg.open_total : 0.0;
      const int fl = (int)exact;
      const double frac = exact - (double)fl;
      qs[0] += fl;
      qs[1] += (frac > q.frac || (frac == q.frac && r < row)) ? 1 : 0;
    };
#pragma unroll
    for (int i = 0; i < kRegRows; ++i)
      if (open_reg[i] >= 0) visit(tid + i * kThreads, open_reg[i]);
    for (int r = tid + kRegRows * kThreads; r < p.rows; r += kThreads) {
      const RowInfo ri = row_info(p, r);
      if (ri.part) visit(r, ri.exist - ri.pinned);
    }
  }
  {
    uint32_t mag = 0;
    int sgn = 0;
    const int live = me.n - tid * PER;  // the thread's live slots
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const uint32_t k = i < live ? key[i] : 0u;
      mag = max(mag, k & 0x7fffffffu);
      sgn = max(sgn, (int)k);
    }
    qs[2] = (int)mag;
    qs[3] = sgn;
  }
  quota_reduce<4, 2>(qs, s_red);
  const long long leftover = bg.free_blocks - qs[0];
  const long long quota = bg.keep_all ? q.open : q.floor + (qs[1] < leftover ? 1 : 0);
  keep_and_view<PER>(p, row, me, L, key, decide, quota, key_mode((uint32_t)qs[2], qs[3]), s_row, s_hist,
                     s_scan, s_sel);
}

// ---------------------------------------------------------------------------------------
// Rows wider than a row in registers (width > kMaxWidth): one 1024-thread workgroup per row
// streams the row from memory in every pass instead -- the same budget, quota, key modes, radix
// select and ties by index as rank_kernel, the keys recomputed from the scores and masks each
// time they are needed.  The ties are ranked in index order, chunk by chunk, by a running scan.
// ---------------------------------------------------------------------------------------
constexpr int kWideThreads = 1024;
constexpr int kMaxWideWidth = 1 << 18;  // 262144 blocks: a float64 row's set bits and their prefix fit LDS

template <bool F64>
__global__ __launch_bounds__(kWideThreads) void rank_wide_kernel(const Params p) {
  constexpr int NT = kWideThreads, NW = NT / kWave;
  using Key = typename std::conditional<F64, unsigned long long, uint32_t>::type;
  constexpr Key kClosedKey = ~Key(0);
  constexpr int kPasses = F64 ? 8 : 4;
  __shared__ long long s_red[6][NW];
  __shared__ int s_hist[2][256];
  __shared__ int s_scan[NW];
  __shared__ int s_digit, s_krem, s_whole;
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const RowInfo me = row_info(p, row);
  uint8_t *keep_row = p.keep + (int64_t)row * p.keep_stride;

  long long t5[5] = {0, 0, 0, 0, 0};  // total, floor_pins, sizes, open_total, requests
  for (int r = tid; r < p.rows; r += NT) {
    const RowInfo ri = row_info(p, r);
    if (!ri.part) continue;
    t5[0] += ri.n;
    t5[1] += ri.pinned;
    t5[2] += ri.exist;
    t5[3] += ri.exist - ri.pinned;
    t5[4] += 1;
  }
  block_sums_n<NT>(t5, reinterpret_cast<long long (*)[NW]>(s_red));
  const long long total = t5[0], floor_pins = t5[1], sizes = t5[2], open_total = t5[3], nreq = t5[4];
  long long budget = p.budget_in;
  if (budget < 0) {  // controller.py:435-437
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
  if (!me.part || error) {  // rows without evidence read in full, controller.py:401
    for (int b = tid; b < p.width; b += NT) keep_row[b] = 1;
    return;
  }
  const int n = me.n;
  auto open_at = [&](int b) -> bool { return b < n && exists(p, row, b) && !is_pinned(p, me, row, b); };
  const double row_total = F64 ? p.totals[row] : 0.0;
  const double uniform = 1.0 / (double)(me.exist > 0 ? me.exist : 1);

  // ---- this row's quota (allocation.py:79-86) and its blocks' counts ----------------------------
  const long long my_open = me.exist - me.pinned;
  const double my_exact = open_total > 0 ? (double)(free_blocks * my_open) / (double)open_total : 0.0;
  const long long my_floor = (long long)my_exact;
  const double my_frac = my_exact - (double)my_floor;
  // floors, rows ahead in the leftover order, NaN / +inf / positive existing scores, open blocks
  long long q[6] = {0, 0, 0, 0, 0, 0};
  if (!keep_all) {
    for (int r = tid; r < p.rows; r += NT) {
      const RowInfo ri = row_info(p, r);
      if (!ri.part) continue;
      const long long open = ri.exist - ri.pinned;
      const double exact = open_total > 0 ? (double)(free_blocks * open) / (double)open_total : 0.0;
      const long long fl = (long long)exact;
      const double frac = exact - (double)fl;
      q[0] += fl;
      q[1] += (frac > my_frac || (frac == my_frac && r < row)) ? 1 : 0;
    }
  }
  for (int b = tid; b < n; b += NT) {
    if (!exists(p, row, b)) continue;
    if (!F64) {
      const float s = p.scores[(int64_t)row * p.scores_stride + b];
      q[2] += __builtin_isnan(s) ? 1 : 0;
      q[3] += (__builtin_isinf(s) && s > 0.0f) ? 1 : 0;
      q[4] += s > 0.0f ? 1 : 0;
    }
    q[5] += is_pinned(p, me, row, b) ? 0 : 1;
  }
  block_sums_n<NT>(q, s_red);
  long long quota;
  if (keep_all) {
    quota = my_open;
  } else {
    const long long leftover = free_blocks - q[0];
    quota = my_floor + (q[1] < leftover ? 1 : 0);
  }
  const long long open_count = q[5];
  const int mode = q[2] ? 0 : (q[3] ? 2 : (q[4] ? 1 : 0));  // 0 tie, 1 by value, 2 inf last

  // a block's key (order-preserving, larger first), kClosedKey unless open
  auto key_at = [&](int b) -> Key {
    if (!open_at(b)) return kClosedKey;
    if constexpr (F64) {
      double v = row_total <= 0.0 ? uniform : clamp0(p.scores64[(int64_t)row * p.scores_stride + b]) / row_total;
      if (v == 0.0) v = 0.0;
      return v != v ? 0ull : __builtin_bit_cast(unsigned long long, v) + 1ull;
    } else {
      const float s = p.scores[(int64_t)row * p.scores_stride + b];
      if (mode == 1) return s > 0.0f ? __builtin_bit_cast(uint32_t, s) : 0u;
      if (mode == 2) return (__builtin_isinf(s) && s > 0.0f) ? 0u : 1u;
      return 0u;
    }
  };

  bool keep_open = quota >= open_count, keep_none = quota <= 0;
  Key prefix = 0, mask = 0;
  int k_rem = (int)quota;
  bool whole = false;
  if (!keep_open && !keep_none) {
    if (tid < 256) s_hist[0][tid] = 0;
    __syncthreads();
    for (int pass = 0; pass < kPasses; ++pass) {
      const int shift = 8 * (kPasses - 1) - 8 * pass;
      int *hist = s_hist[pass & 1];
      for (int b = tid; b < n; b += NT) {
        const Key k = key_at(b);
        if (k != kClosedKey && (k & mask) == prefix) atomicAdd(&hist[(int)(k >> shift) & 255], 1);
      }
      if (tid < 256) s_hist[(pass & 1) ^ 1][tid] = 0;
      __syncthreads();
      if (wave == 0) {
        int c[4], s4 = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          c[j] = hist[255 - 4 * lane - j];
          s4 += c[j];
        }
        const int inc = wave_inclusive_scan(s4);
        int acc = inc - s4;
        if (acc < k_rem && inc >= k_rem) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (acc < k_rem && acc + c[j] >= k_rem) {
              s_digit = 255 - 4 * lane - j;
              s_krem = k_rem - acc;
              s_whole = acc + c[j] == k_rem ? 1 : 0;
            }
            acc += c[j];
          }
        }
      }
      __syncthreads();
      prefix |= (Key)s_digit << shift;
      mask |= (Key)255 << shift;
      k_rem = s_krem;
      whole = s_whole != 0;
      if (whole) break;
    }
  }
  // the keep, chunk by chunk in index order; the equal keys before a block counted by a running scan
  int eq_before = 0;
  for (int b0 = 0; b0 < p.width; b0 += NT) {
    const int b = b0 + tid;
    const Key k = b < n ? key_at(b) : kClosedKey;
    bool kept = false;
    int eq_chunk = 0;
    if (keep_open) {
      kept = k != kClosedKey;
    } else if (!keep_none) {
      if (whole) {
        kept = k != kClosedKey && (k & mask) >= prefix;
      } else {
        const bool eq = k != kClosedKey && k == prefix;
        const int before = eq_before + block_exclusive_scan<NT>(eq ? 1 : 0, s_scan, eq_chunk);
        kept = k != kClosedKey && (k > prefix || (eq && before < k_rem));
      }
    }
    eq_before += eq_chunk;
    if (b < p.width) {
      uint8_t v;
      if (b >= n) v = 1;
      else if (!exists(p, row, b)) v = 0;
      else if (is_pinned(p, me, row, b)) v = 1;
      else v = kept ? 1 : 0;
      keep_row[b] = v;
    }
  }
}

// Each float64 request's NumPy total over its existing blocks for rows wider than kMaxWidth with a
// released mask: the row's existing blocks as bits in LDS with each word's prefix count, so that
// NumPy's sum over the remaining blocks (taken by wave 0) finds the i-th one by a binary search.
__global__ __launch_bounds__(kWideThreads) void total64_wide_kernel(const Params p, double *totals) {
  constexpr int NT = kWideThreads, kWords = kMaxWideWidth / 32;
  __shared__ uint32_t s_bits[kWords];
  __shared__ int s_pref[kWords];
  __shared__ int s_scan[NT / kWave];
  __shared__ int s_start[kMaxLeaves], s_len[kMaxLeaves];
  __shared__ double s_leaf[kMaxLeaves];
  const int r = blockIdx.x;
  const int n = min(max(p.blocks[r], 0), p.width);
  const int words = (n + 31) / 32;
  constexpr int kPer = kWords / NT;  // words per thread, a contiguous run (the scan below is in word order)
  int cnt[kPer], mine = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int w = threadIdx.x * kPer + j;
    uint32_t bits = 0;
    if (w < words)
      for (int i = 0; i < 32; ++i) {
        const int b = 32 * w + i;
        bits |= (b < n && exists(p, r, b)) ? (1u << i) : 0u;
      }
    s_bits[w] = bits;
    cnt[j] = __popc(bits);
    mine += cnt[j];
  }
  int total_bits;
  int before = block_exclusive_scan<NT>(mine, s_scan, total_bits);
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    s_pref[threadIdx.x * kPer + j] = before;
    before += cnt[j];
  }
  __syncthreads();
  if (threadIdx.x >= kWave) return;
  const double *srow = p.scores64 + (int64_t)r * p.scores_stride;
  static_assert(kWords % NT == 0, "whole runs of words per thread");
  auto block_of = [&](int i) -> int {  // the i-th existing block
    int lo = 0, hi = words - 1;
    while (lo < hi) {  // the last word whose prefix count is at most i
      const int mid = (lo + hi + 1) >> 1;
      if (s_pref[mid] <= i) lo = mid; else hi = mid - 1;
    }
    uint32_t bits = s_bits[lo];
    for (int k = i - s_pref[lo]; k > 0; --k) bits &= bits - 1;  // drop the lower set bits
    return 32 * lo + __builtin_ctz(bits);
  };
  const double total = numpy_sum([&](int i) { return clamp0(srow[block_of(i)]); }, total_bits, s_start, s_len,
                                 s_leaf);
  if (lane_id() == 0) totals[r] = total;
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

extern "C" int ekv_rank_uniform_view(const float *scores, int64_t scores_stride, const int32_t *blocks,
                                     const uint8_t *measured, const int32_t *pin_from, int32_t recent_blocks,
                                     int32_t rows, int32_t width, double fraction, int64_t budget, uint8_t *keep,
                                     int64_t keep_stride, int64_t *summary, const int32_t *table,
                                     int64_t table_stride, const int32_t *seq_lens, int32_t block_size,
                                     int32_t *view_table, int64_t view_stride, int32_t *view_lens,
                                     int64_t *counts, void *stream) {
  if (scores == nullptr || blocks == nullptr || keep == nullptr || table == nullptr || seq_lens == nullptr ||
      view_table == nullptr || view_lens == nullptr)
    return fail(EKV_EINVAL, "ekv_rank_uniform_view: null pointer");
  if (rows < 0 || width < 1 || width > rank::kMaxWideWidth)
    return fail(EKV_EINVAL, "ekv_rank_uniform_view: rows %d, width %d (at most %d)", rows, width, rank::kMaxWideWidth);
  if (recent_blocks < 0) return fail(EKV_EINVAL, "ekv_rank_uniform_view: recent_blocks %d < 0", recent_blocks);
  if (budget < 0 && !(fraction > 0.0 && fraction <= 1.0))
    return fail(EKV_EINVAL, "ekv_rank_uniform_view: the budget fraction %g is not in (0, 1]", fraction);
  if (block_size < 1) return fail(EKV_EINVAL, "ekv_rank_uniform_view: block size %d", block_size);
  if (rows == 0) return EKV_OK;
  rank::Params p{};
  p.scores = scores;
  p.scores_stride = scores_stride;
  p.blocks = blocks;
  p.measured = measured;
  p.pin_from = pin_from;
  p.recent = recent_blocks;
  p.rows = rows;
  p.width = width;
  p.fraction = fraction;
  p.budget_in = budget;
  p.keep = keep;
  p.keep_stride = keep_stride;
  p.summary = summary;
  p.table = table;
  p.table_stride = table_stride;
  p.seq_lens = seq_lens;
  p.block_size = block_size;
  p.view_table = view_table;
  p.view_stride = view_stride;
  p.view_lens = view_lens;
  p.view_counts = (long long *)counts;
  hipStream_t s = (hipStream_t)stream;
  if (width > rank::kMaxWidth) {  // a row too wide for registers: the streaming ranking, then the view
    hipLaunchKernelGGL((rank::rank_wide_kernel<false>), dim3(rows), dim3(rank::kWideThreads), 0, s, p);
    const int rc = check_hip(hipGetLastError(), "ekv_rank_uniform_view launch");
    if (rc != EKV_OK) return rc;
    return ekv_build_view(table, table_stride, seq_lens, keep, keep_stride, nullptr, 0, nullptr, nullptr, 1, rows,
                          width, block_size, view_table, view_stride, view_lens, counts, stream);
  }
  const int per = (width + rank::kThreads - 1) / rank::kThreads;
  // the lean kernel counts blocks in 32 bits; larger batches (and the widest rows) take rank_kernel
  const bool lean = (int64_t)rows * width < ((int64_t)1 << 31);
  if (lean && per <= 4)
    hipLaunchKernelGGL((rank::rank_view_kernel<4>), dim3(rows), dim3(rank::kThreads), 0, s, p);
  else if (lean && per <= 8)
    hipLaunchKernelGGL((rank::rank_view_kernel<8>), dim3(rows), dim3(rank::kThreads), 0, s, p);
  else if (lean && per <= 16)
    hipLaunchKernelGGL((rank::rank_view_kernel<16>), dim3(rows), dim3(rank::kThreads), 0, s, p);
  else if (per <= 4)
    hipLaunchKernelGGL((rank::rank_kernel<4, true>), dim3(rows), dim3(rank::kThreads), 0, s, p);
  else if (per <= 8)
    hipLaunchKernelGGL((rank::rank_kernel<8, true>), dim3(rows), dim3(rank::kThreads), 0, s, p);
  else if (per <= 16)
    hipLaunchKernelGGL((rank::rank_kernel<16, true>), dim3(rows), dim3(rank::kThreads), 0, s, p);
  else
    hipLaunchKernelGGL((rank::rank_kernel<24, true>), dim3(rows), dim3(rank::kThreads), 0, s, p);
  return check_hip(hipGetLastError(), "ekv_rank_uniform_view launch");
}

extern "C" int ekv_rank_uniform_ws(const float *scores, int64_t scores_stride, const int32_t *blocks,
                                   const uint8_t *measured, const uint8_t *pinned, int64_t pinned_stride,
                                   const int32_t *pin_from, int32_t recent_blocks, const uint8_t *released,
                                   int64_t released_stride, int32_t rows, int32_t width, double fraction,
                                   int64_t budget, uint8_t *keep, int64_t keep_stride, int64_t *summary,
                                   int32_t *workspace, void *stream) {
  if (scores == nullptr || blocks == nullptr || keep == nullptr)
    return fail(EKV_EINVAL, "ekv_rank_uniform: null pointer");
  if (rows < 0 || width < 1 || width > rank::kMaxWideWidth)
    return fail(EKV_EINVAL, "ekv_rank_uniform: rows %d, width %d (at most %d)", rows, width, rank::kMaxWideWidth);
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
  if (width > rank::kMaxWidth) {  // a row too wide for registers: the streaming ranking
    hipLaunchKernelGGL((rank::rank_wide_kernel<false>), dim3(rows), dim3(rank::kWideThreads), 0, (hipStream_t)stream,
                       p);
    return check_hip(hipGetLastError(), "ekv_rank_uniform launch");
  }
  const int per = (width + rank::kThreads - 1) / rank::kThreads;
  if (per <= 4)
    hipLaunchKernelGGL(rank::rank_kernel<4>, dim3(rows), dim3(rank::kThreads), 0, (hipStream_t)stream, p);
  else if (per <= 8)
    hipLaunchKernelGGL(rank::rank_kernel<8>, dim3(rows), dim3(rank::kThreads), 0, (hipStream_t)stream, p);
  else if (per <= 16)
    hipLaunchKernelGGL(rank::rank_kernel<16>, dim3(rows), dim3(rank::kThreads), 0, (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL(rank::rank_kernel<24>, dim3(rows), dim3(rank::kThreads), 0, (hipStream_t)stream, p);
  return check_hip(hipGetLastError(), "ekv_rank_uniform launch");
}

namespace {
// workspace of ekv_rank_uniform64: the rows' float64 totals, then 2 * rows ints of mask counts
size_t uniform64_totals_bytes(int32_t rows) { return ((size_t)(rows > 0 ? rows : 1) * 8 + 255) / 256 * 256; }
}  // namespace

extern "C" size_t ekv_rank_uniform64_workspace(int32_t rows) {
  if (rows < 0) return 0;
  return uniform64_totals_bytes(rows) + (size_t)(rows > 0 ? rows : 1) * 2 * sizeof(int32_t);
}

extern "C" int ekv_rank_uniform64(const double *scores, int64_t scores_stride, const int32_t *blocks,
                                  const uint8_t *measured, const uint8_t *pinned, int64_t pinned_stride,
                                  const int32_t *pin_from, int32_t recent_blocks, const uint8_t *released,
                                  int64_t released_stride, int32_t rows, int32_t width, double fraction,
                                  int64_t budget, uint8_t *keep, int64_t keep_stride, int64_t *summary,
                                  void *workspace, size_t workspace_bytes, void *stream) {
  if (scores == nullptr || blocks == nullptr || keep == nullptr || workspace == nullptr)
    return fail(EKV_EINVAL, "ekv_rank_uniform64: null pointer");
  if (rows < 0 || width < 1 || width > rank::kMaxWideWidth)
    return fail(EKV_EINVAL, "ekv_rank_uniform64: rows %d, width %d (at most %d)", rows, width, rank::kMaxWideWidth);
  if (recent_blocks < 0) return fail(EKV_EINVAL, "ekv_rank_uniform64: recent_blocks %d < 0", recent_blocks);
  if (budget < 0 && !(fraction > 0.0 && fraction <= 1.0))
    return fail(EKV_EINVAL, "ekv_rank_uniform64: the budget fraction %g is not in (0, 1]", fraction);
  if (workspace_bytes < ekv_rank_uniform64_workspace(rows))
    return fail(EKV_EINVAL, "ekv_rank_uniform64: a workspace of %zu bytes, %zu needed", workspace_bytes,
                ekv_rank_uniform64_workspace(rows));
  if (rows == 0) return EKV_OK;
  rank::Params p{};
  p.scores64 = scores;
  p.scores_stride = scores_stride;
  p.blocks = blocks;
  p.measured = measured;
  p.pinned = pinned;
  p.pinned_stride = pinned_stride;
  p.pin_from = pin_from;
  p.recent = recent_blocks;
  p.released = released;
  p.released_stride = released_stride;
  p.rows = rows;
  p.width = width;
  p.fraction = fraction;
  p.budget_in = budget;
  p.keep = keep;
  p.keep_stride = keep_stride;
  p.summary = summary;
  double *totals = (double *)workspace;
  int32_t *counts = (int32_t *)((char *)workspace + uniform64_totals_bytes(rows));
  hipStream_t s = (hipStream_t)stream;
  if (width > rank::kMaxWidth && released != nullptr)  // the remaining blocks found through LDS bits
    hipLaunchKernelGGL(rank::total64_wide_kernel, dim3(rows), dim3(rank::kWideThreads), 0, s, p, totals);
  else
    hipLaunchKernelGGL(rank::total64_kernel, dim3(rows), dim3(kWave), 0, s, p, totals);
  int rc = check_hip(hipGetLastError(), "ekv_rank_uniform64 totals launch");
  if (rc != EKV_OK) return rc;
  p.totals = totals;
  if (pinned != nullptr || released != nullptr) {
    hipLaunchKernelGGL(rank::count_kernel, dim3(rows), dim3(256), 0, s, p, counts);
    rc = check_hip(hipGetLastError(), "ekv_rank_uniform64 count launch");
    if (rc != EKV_OK) return rc;
    p.counts = counts;
  }
  if (width > rank::kMaxWidth) {  // a row too wide for registers: the streaming ranking
    hipLaunchKernelGGL((rank::rank_wide_kernel<true>), dim3(rows), dim3(rank::kWideThreads), 0, s, p);
    return check_hip(hipGetLastError(), "ekv_rank_uniform64 launch");
  }
  const int per = (width + rank::kThreads - 1) / rank::kThreads;
  if (per <= 4)
    hipLaunchKernelGGL((rank::rank_kernel<4, false, true>), dim3(rows), dim3(rank::kThreads), 0, s, p);
  else if (per <= 8)
    hipLaunchKernelGGL((rank::rank_kernel<8, false, true>), dim3(rows), dim3(rank::kThreads), 0, s, p);
  else if (per <= 16)
    hipLaunchKernelGGL((rank::rank_kernel<16, false, true>), dim3(rows), dim3(rank::kThreads), 0, s, p);
  else
    hipLaunchKernelGGL((rank::rank_kernel<24, false, true>), dim3(rows), dim3(rank::kThreads), 0, s, p);
  return check_hip(hipGetLastError(), "ekv_rank_uniform64 launch");
}
