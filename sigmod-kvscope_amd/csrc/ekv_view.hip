// The block-table view: the stable partition of every row of the block table by its keep mask.
// Semantics: compact_block_table (runtime/block_view.py:36-56), and for ekv_build_view also
// DecodeView.build's keep composition (runtime/block_view.py:272-281) and read counters
// (runtime/block_view.py:297-329).
//
// One workgroup of 8 waves per row.  A row is taken in segments of 512 x PER entries (PER = 4,
// 8, 16 or 24, the least that holds the width, else 24): every thread loads its PER entries of
// the segment (coalesced: entry tid + 512 i) and their keep
// bytes at once, a ballot per wave and load gives each entry its rank among the kept entries of
// its wave, and one workgroup scan over the PER x 8 (load, wave) counts gives every entry its
// number of kept entries before it, kb.  A kept entry goes to kb, a dropped one to
// total_kept + (b - kb): kept first, then dropped, both in original order -- the reference's
// stable argsort of ~keep, including the tail.  A row of more than one segment first counts its
// kept entries.  No LDS holds the row, so any width fits.
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
  long long *counts;
};

// PER: entries per thread per segment of kThreads * PER entries
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
  const int bs = p.block_size;
  const int L = p.seq_lens[row];
  // blocks = ceil(L / bs) with floor division, block_view.py:49 (n <= 0 keeps nothing)
  const long long n64 = L > 0 ? ((long long)L + bs - 1) / bs : 0;
  const int n = n64 > W + 1LL ? W + 1 : (int)n64;  // only b < W and b == n - 1 < W matter

  // the keep of each block before the first / last rule
  bool whole = false;  // every block of the row is read
  if (p.compose) {
    const bool audited = p.audited != nullptr && p.audited[row] != 0;
    const bool prefill = p.decoding != nullptr && p.decoding[row] == 0;
    whole = !p.live || audited || prefill;  // block_view.py:273-279
  }
  if (p.table == nullptr) {
    // counts only: the row reads its whole table (DecodeView.skip, block_view.py:352-361)
    if (tid == 0 && p.counts != nullptr) {
      const bool decoding = p.decoding == nullptr || p.decoding[row] != 0;
      const long long r = decoding ? n64 : 0;
      if (r) {
        atomicAdd((unsigned long long *)&p.counts[0], (unsigned long long)r);
        atomicAdd((unsigned long long *)&p.counts[1], (unsigned long long)r);
        if (p.live) atomicAdd((unsigned long long *)&p.counts[3], (unsigned long long)r);
        else atomicAdd((unsigned long long *)&p.counts[4], (unsigned long long)r);
      }
    }
    return;
  }
  const int32_t *trow = p.table + (int64_t)row * p.table_stride;
  const uint8_t *krow = p.keep != nullptr ? p.keep + (int64_t)row * p.keep_stride : nullptr;
  const uint8_t *rrow = p.released != nullptr ? p.released + (int64_t)row * p.released_stride : nullptr;
  auto keep_at = [&](int b) -> bool {
    bool k = whole || krow == nullptr || krow[b] != 0;
    if (rrow != nullptr && rrow[b] != 0) k = false;  // released last, block_view.py:280-281
    return (k || b == 0 || b == n - 1) && b < n;     // block_view.py:51
  };

  int total_kept = 0;
  if (W > kSegment) {
    long long c = 0;
    for (int b = tid; b < W; b += kThreads) c += keep_at(b) ? 1 : 0;
    total_kept = (int)block_sum<kThreads>(c, s_red);
  }
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
    if (W <= kSegment) total_kept = seg_kept;
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

  if (tid == 0) {
    // block_view.py:53-55
    const int last = L - (int)(n64 - 1) * bs;
    const int view_len = n64 > 0 ? (total_kept - 1) * bs + last : 0;
    if (p.view_lens != nullptr) p.view_lens[row] = view_len;
    if (p.counts != nullptr) {
      // DecodeView._count, block_view.py:313-329
      const long long read = view_len > 0 ? ((long long)view_len + bs - 1) / bs : 0;
      const long long full = n64;
      const bool decoding = p.decoding == nullptr || p.decoding[row] != 0;
      const bool in_audit = p.audited != nullptr && p.audited[row] != 0;
      const bool whole_read = view_len == L;
      const long long r = decoding ? read : 0, f = decoding ? full : 0;
      const long long untrimmed = (whole_read && !in_audit && p.live) ? r : 0;
      if (r) atomicAdd((unsigned long long *)&p.counts[0], (unsigned long long)r);
      if (f) atomicAdd((unsigned long long *)&p.counts[1], (unsigned long long)f);
      if (in_audit && r) atomicAdd((unsigned long long *)&p.counts[2], (unsigned long long)r);
      if (untrimmed) atomicAdd((unsigned long long *)&p.counts[3], (unsigned long long)untrimmed);
      if (!p.live && r) atomicAdd((unsigned long long *)&p.counts[4], (unsigned long long)r);
    }
  }
}

int launch(const Params &p, void *stream) {
  if (p.seq_lens == nullptr) return fail(EKV_EINVAL, "block-table view: null lengths");
  if (p.table == nullptr && (p.view_table != nullptr || p.view_lens != nullptr))
    return fail(EKV_EINVAL, "block-table view: a view needs the block table");
  if (p.rows < 0 || p.width < 1 || p.block_size < 1)
    return fail(EKV_EINVAL, "block-table view: rows %d, width %d, block size %d", p.rows, p.width, p.block_size);
  if (p.rows == 0) return EKV_OK;
  const int per = (p.width + kThreads - 1) / kThreads;  // a row in one segment when it fits
  if (per <= 4)
    hipLaunchKernelGGL(view_kernel<4>, dim3(p.rows), dim3(kThreads), 0, (hipStream_t)stream, p);
  else if (per <= 8)
    hipLaunchKernelGGL(view_kernel<8>, dim3(p.rows), dim3(kThreads), 0, (hipStream_t)stream, p);
  else if (per <= 16)
    hipLaunchKernelGGL(view_kernel<16>, dim3(p.rows), dim3(kThreads), 0, (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL(view_kernel<kMaxPer>, dim3(p.rows), dim3(kThreads), 0, (hipStream_t)stream, p);
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
