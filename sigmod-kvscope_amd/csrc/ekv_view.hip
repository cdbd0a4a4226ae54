// The block-table view: the stable partition of every row of the block table by its keep mask.
// Semantics: compact_block_table (runtime/block_view.py:36-56), and for ekv_build_view also
// DecodeView.build's keep composition (runtime/block_view.py:272-281) and read counters
// (runtime/block_view.py:297-329).
//
// One workgroup of 8 waves per row.  Rows of at most 12288 blocks: thread t takes a contiguous run
// of entries (16-byte loads), one block scan of the threads' kept counts gives every entry its
// number of kept entries before it, kb; a kept entry goes to kb, a dropped one to
// total_kept + (b - kb) -- kept first, then dropped, both in original order, the reference's
// stable argsort of ~keep including the tail -- assembled in LDS and written with 16-byte stores.
// Wider rows go by segments of 512 x 24 entries ranked with ballots, written in place.
#include "ekv_common.hpp"

namespace ekv {
namespace view {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxPer = 24;  // entries per thread per segment (12288 per segment)

struct Params {
  const int32_t *table;
  int64_t table_stride;
  const int32_t *seq_lens;
  const uint8_t *keep;  // committed mask (ekv_build_view) or keep mask (ekv_compact_view)
  int64_t keep_stride;
  const uint8_t *released;
  int64_t released_stride;
  const uint8_t *audited;
  const uint8_t *decoding;
  int32_t live, compose;
  int32_t rows, width, block_size;
  int32_t *view_table;
  int64_t view_stride;
  int32_t *view_lens;
  long long *counts;  // [rows][5] per-row counters, accumulated
};

// the row's blocks and whether it reads them all
struct RowPlan {
  int L;            // tokens
  long long n64;    // blocks, ceil(L / bs) (0 for L <= 0), block_view.py:49
  int n;            // the same, clipped: only b < W and b == n - 1 < W matter
  bool whole;       // every block of the row is read
  long long c[5];   // thread 0: the row's counters before this call
};

__device__ __forceinline__ RowPlan row_plan(const Params &p, int row) {
  RowPlan r;
  // the row's own counter slot: one workgroup per row adds to it, so no atomics are needed, and
  // its load goes out with the row's other loads
  if (threadIdx.x == 0 && p.counts != nullptr) {
#pragma unroll
    for (int k = 0; k < 5; ++k) r.c[k] = p.counts[5LL * row + k];
  }
  r.L = p.seq_lens[row];
  r.n64 = r.L > 0 ? ((long long)r.L + p.block_size - 1) / p.block_size : 0;
  r.n = r.n64 > p.width + 1LL ? p.width + 1 : (int)r.n64;
  r.whole = false;
  if (p.compose) {
    const bool audited = p.audited != nullptr && p.audited[row] != 0;
    const bool prefill = p.decoding != nullptr && p.decoding[row] == 0;
    r.whole = !p.live || audited || prefill;  // block_view.py:273-279
  }
  return r;
}

// counts only: the row reads its whole table (DecodeView.skip, block_view.py:352-361)
__device__ __forceinline__ void count_whole_row(const Params &p, const RowPlan &r, int row) {
  if (threadIdx.x != 0 || p.counts == nullptr) return;
  const bool decoding = p.decoding == nullptr || p.decoding[row] != 0;
  const long long read = decoding ? r.n64 : 0;
  long long *c = p.counts + 5LL * row;
  c[0] = r.c[0] + read;
  c[1] = r.c[1] + read;
  c[2] = r.c[2];
  c[3] = r.c[3] + (p.live ? read : 0);
  c[4] = r.c[4] + (p.live ? 0 : read);
}

// keep' of block b from its keep and released bytes, block_view.py:51 and :280-281
__device__ __forceinline__ bool keep_of(const RowPlan &r, bool has_keep, uint8_t keep, uint8_t released, int b) {
  bool k = r.whole || !has_keep || keep != 0;
  if (released != 0) k = false;  // released last
  return (k || b == 0 || b == r.n - 1) && b < r.n;
}

// the new length and DecodeView._count's counters, by thread 0 (block_view.py:53-55, :313-329)
__device__ __forceinline__ void finish_row(const Params &p, const RowPlan &r, int row, int total_kept) {
  if (threadIdx.x != 0) return;
  const int bs = p.block_size;
  const int last = r.L - (int)(r.n64 - 1) * bs;
  const int view_len = r.n64 > 0 ? (total_kept - 1) * bs + last : 0;
  if (p.view_lens != nullptr) p.view_lens[row] = view_len;
  if (p.counts != nullptr) {
    const long long read = view_len > 0 ? ((long long)view_len + bs - 1) / bs : 0;
    const long long full = r.n64;
    const bool decoding = p.decoding == nullptr || p.decoding[row] != 0;
    const bool in_audit = p.audited != nullptr && p.audited[row] != 0;
    const bool whole_read = view_len == r.L;
    const long long rd = decoding ? read : 0, f = decoding ? full : 0;
    const long long untrimmed = (whole_read && !in_audit && p.live) ? rd : 0;
    long long *c = p.counts + 5LL * row;
    c[0] = r.c[0] + rd;
    c[1] = r.c[1] + f;
    c[2] = r.c[2] + (in_audit ? rd : 0);
    c[3] = r.c[3] + untrimmed;
    c[4] = r.c[4] + (p.live ? 0 : rd);
  }
}

// Rows of at most kLdsWidth blocks: thread t takes the contiguous run of PER entries from t * PER
// (16-byte table loads and 4-byte keep loads when the rows are aligned), one block scan of the
// threads' kept counts places every entry, the row is assembled in LDS and written with 16-byte
// stores.
constexpr int kLdsWidth = 12288;

template <int PER>
__global__ __launch_bounds__(kThreads) void view_lds_kernel(const Params p) {
  static_assert(PER % 4 == 0, "runs of whole 16-byte groups");
  extern __shared__ int32_t s_out[];  // [width] the view row
  __shared__ int s_scan[kWaves];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int W = p.width;
  const RowPlan r = row_plan(p, row);
  if (p.table == nullptr) {
    count_whole_row(p, r, row);
    return;
  }
  const int32_t *trow = p.table + (int64_t)row * p.table_stride;
  const uint8_t *krow = p.keep != nullptr ? p.keep + (int64_t)row * p.keep_stride : nullptr;
  const uint8_t *rrow = p.released != nullptr ? p.released + (int64_t)row * p.released_stride : nullptr;
  const int b0 = tid * PER;
  const bool vec = b0 + PER <= W && ((uintptr_t)(trow + b0) & 15) == 0 &&
                   (krow == nullptr || ((uintptr_t)(krow + b0) & 3) == 0) &&
                   (rrow == nullptr || ((uintptr_t)(rrow + b0) & 3) == 0);
  int32_t entry[PER];
  uint32_t kb[PER / 4], rb[PER / 4];  // keep and released bytes, four per word
  if (vec) {
#pragma unroll
    for (int g = 0; g < PER / 4; ++g) {
      const int4 t4 = *reinterpret_cast<const int4 *>(trow + b0 + 4 * g);
      entry[4 * g] = t4.x;
      entry[4 * g + 1] = t4.y;
      entry[4 * g + 2] = t4.z;
      entry[4 * g + 3] = t4.w;
      kb[g] = krow != nullptr ? *reinterpret_cast<const uint32_t *>(krow + b0 + 4 * g) : 0u;
      rb[g] = rrow != nullptr ? *reinterpret_cast<const uint32_t *>(rrow + b0 + 4 * g) : 0u;
    }
  } else {
#pragma unroll
    for (int g = 0; g < PER / 4; ++g) {
      kb[g] = rb[g] = 0u;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int b = b0 + 4 * g + k;
        entry[4 * g + k] = b < W ? trow[b] : 0;
        if (b < W && krow != nullptr) kb[g] |= (uint32_t)krow[b] << (8 * k);
        if (b < W && rrow != nullptr) rb[g] |= (uint32_t)rrow[b] << (8 * k);
      }
    }
  }
  uint32_t kept_bits = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int b = b0 + i;
    const uint8_t k = (uint8_t)(kb[i / 4] >> (8 * (i % 4)));
    const uint8_t rel = (uint8_t)(rb[i / 4] >> (8 * (i % 4)));
    kept_bits |= (b < W && keep_of(r, krow != nullptr, k, rel, b)) ? (1u << i) : 0u;
  }
  int total_kept;
  int before = block_exclusive_scan<kThreads>(__popc(kept_bits), s_scan, total_kept);
  if (p.view_table != nullptr) {
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
  }
  finish_row(p, r, row, total_kept);
}

// Wider rows: segments of kThreads * PER entries, entry tid + kThreads i of a segment in slot i; the
// row is counted first, then each segment ranked by ballots and a scan over (load, wave) counts
// and written straight to its places.
template <int PER>
__global__ __launch_bounds__(kThreads) void view_kernel(const Params p) {
  constexpr int kPer = PER, kSegment = kThreads * PER;
  __shared__ int s_count[kPer * kWaves];  // kept entries per (load, wave), then their exclusive scan
  __shared__ int s_scan[kWaves];
  __shared__ long long s_red[kWaves];

  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const int W = p.width;
  const RowPlan r = row_plan(p, row);
  if (p.table == nullptr) {
    count_whole_row(p, r, row);
    return;
  }
  const int32_t *trow = p.table + (int64_t)row * p.table_stride;
  const uint8_t *krow = p.keep != nullptr ? p.keep + (int64_t)row * p.keep_stride : nullptr;
  const uint8_t *rrow = p.released != nullptr ? p.released + (int64_t)row * p.released_stride : nullptr;
  auto keep_at = [&](int b) -> bool {
    return keep_of(r, krow != nullptr, krow != nullptr ? krow[b] : 0, rrow != nullptr ? rrow[b] : 0, b);
  };

  long long c = 0;
  for (int b = tid; b < W; b += kThreads) c += keep_at(b) ? 1 : 0;
  const int total_kept = (int)block_sum<kThreads>(c, s_red);
  int32_t *vrow = p.view_table != nullptr ? p.view_table + (int64_t)row * p.view_stride : nullptr;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));  // lanes under this one
  int kept_before = 0;  // kept entries of the earlier segments
  for (int seg = 0; seg < W; seg += kSegment) {
    int32_t entry[kPer];
    uint32_t kept_bits = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int b = seg + i * kThreads + tid;
      entry[i] = b < W ? trow[b] : 0;
      kept_bits |= (b < W && keep_at(b)) ? (1u << i) : 0u;
    }
    int rank_in_wave[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const uint64_t mask = __ballot((kept_bits >> i) & 1u);
      rank_in_wave[i] = __popcll(mask & below);
      if (lane == 0) s_count[i * kWaves + wave] = __popcll(mask);
    }
    __syncthreads();
    const int v = tid < kPer * kWaves ? s_count[tid] : 0;
    int seg_kept;
    const int excl = block_exclusive_scan<kThreads>(v, s_scan, seg_kept);
    if (tid < kPer * kWaves) s_count[tid] = excl;
    __syncthreads();
    if (vrow != nullptr) {
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int b = seg + i * kThreads + tid;
        if (b >= W) continue;
        const int kb = kept_before + s_count[i * kWaves + wave] + rank_in_wave[i];
        vrow[(kept_bits >> i) & 1u ? kb : total_kept + (b - kb)] = entry[i];
      }
    }
    kept_before += seg_kept;
    __syncthreads();  // s_count is rewritten by the next segment
  }
  finish_row(p, r, row, total_kept);
}

int launch(const Params &p, void *stream) {
  if (p.seq_lens == nullptr) return fail(EKV_EINVAL, "block-table view: null lengths");
  if (p.table == nullptr && (p.view_table != nullptr || p.view_lens != nullptr))
    return fail(EKV_EINVAL, "block-table view: a view needs the block table");
  if (p.rows < 0 || p.width < 1 || p.block_size < 1)
    return fail(EKV_EINVAL, "block-table view: rows %d, width %d, block size %d", p.rows, p.width, p.block_size);
  if (p.rows == 0) return EKV_OK;
  hipStream_t s = (hipStream_t)stream;
  const int per = (p.width + kThreads - 1) / kThreads;
  const size_t lds = (size_t)p.width * sizeof(int32_t);
  if (p.width > kLdsWidth)
    hipLaunchKernelGGL(view_kernel<kMaxPer>, dim3(p.rows), dim3(kThreads), 0, s, p);
  else if (per <= 4)
    hipLaunchKernelGGL(view_lds_kernel<4>, dim3(p.rows), dim3(kThreads), lds, s, p);
  else if (per <= 8)
    hipLaunchKernelGGL(view_lds_kernel<8>, dim3(p.rows), dim3(kThreads), lds, s, p);
  else if (per <= 16)
    hipLaunchKernelGGL(view_lds_kernel<16>, dim3(p.rows), dim3(kThreads), lds, s, p);
  else
    hipLaunchKernelGGL(view_lds_kernel<kMaxPer>, dim3(p.rows), dim3(kThreads), lds, s, p);
  return check_hip(hipGetLastError(), "block-table view launch");
}

}  // namespace view
}  // namespace ekv

using namespace ekv;

extern "C" int ekv_compact_view(const int32_t *table, int64_t table_stride, const int32_t *seq_lens,
                                const uint8_t *keep, int64_t keep_stride, int32_t rows, int32_t width,
                                int32_t block_size, int32_t *view_table, int64_t view_stride,
                                int32_t *view_lens, void *stream) {
  if (keep == nullptr || view_table == nullptr || view_lens == nullptr)
    return fail(EKV_EINVAL, "ekv_compact_view: null pointer");
  view::Params p{};
  p.table = table;
  p.table_stride = table_stride;
  p.seq_lens = seq_lens;
  p.keep = keep;
  p.keep_stride = keep_stride;
  p.compose = 0;
  p.live = 1;
  p.rows = rows;
  p.width = width;
  p.block_size = block_size;
  p.view_table = view_table;
  p.view_stride = view_stride;
  p.view_lens = view_lens;
  return view::launch(p, stream);
}

extern "C" int ekv_build_view(const int32_t *table, int64_t table_stride, const int32_t *seq_lens,
                              const uint8_t *committed, int64_t committed_stride, const uint8_t *released,
                              int64_t released_stride, const uint8_t *audited, const uint8_t *decoding,
                              int32_t live, int32_t rows, int32_t width, int32_t block_size, int32_t *view_table,
                              int64_t view_stride, int32_t *view_lens, int64_t *counts, void *stream) {
  view::Params p{};
  p.table = table;
  p.table_stride = table_stride;
  p.seq_lens = seq_lens;
  p.keep = committed;
  p.keep_stride = committed_stride;
  p.released = released;
  p.released_stride = released_stride;
  p.audited = audited;
  p.decoding = decoding;
  p.live = live != 0;
  p.compose = 1;
  p.rows = rows;
  p.width = width;
  p.block_size = block_size;
  p.view_table = view_table;
  p.view_stride = view_stride;
  p.view_lens = view_lens;
  p.counts = (long long *)counts;
  return view::launch(p, stream);
}
