// The block-table view: the stable partition of every row of the block table by its keep mask.
// Semantics: compact_block_table (runtime/block_view.py:36-56), and for ekv_build_view also
// DecodeView.build's keep composition (runtime/block_view.py:272-281) and read counters
// (runtime/block_view.py:297-329).
//
// One workgroup per row.  The row's keep bytes are composed into LDS with coalesced loads; each
// thread then takes a contiguous run of blocks, a block scan over the runs gives every kept
// block its place among the kept ones and every dropped block its place after them (both in
// original order), the permuted row is assembled in LDS (5 bytes per block, so a 12288-block
// row fits the 64 KB a workgroup may hold) and written out with coalesced stores.  The result is the reference's stable argsort of ~keep, including the
// tail of dropped blocks.
#include "ekv_common.hpp"

namespace ekv {
namespace view {

constexpr int kThreads = 256;
constexpr int kMaxWidth = 12288;

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

__global__ __launch_bounds__(kThreads) void view_kernel(const Params p) {
  extern __shared__ int32_t s_buf[];  // [width] view out, then [width] keep bytes
  __shared__ int s_scan[kThreads / kWave];
  int32_t *s_out = s_buf;
  uint8_t *s_keep = (uint8_t *)(s_buf + p.width);

  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int W = p.width;
  const int bs = p.block_size;
  const int L = p.seq_lens[row];
  // blocks = ceil(L / bs) with floor division, block_view.py:49 (n <= 0 keeps nothing)
  const long long n64 = L > 0 ? ((long long)L + bs - 1) / bs : 0;
  const int n = n64 > W + 1 ? W + 1 : (int)n64;  // only b < W and b == n - 1 < W matter

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
      const long long read = L > 0 ? ((long long)L + bs - 1) / bs : 0;
      const bool decoding = p.decoding == nullptr || p.decoding[row] != 0;
      const long long r = decoding ? read : 0;
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
  for (int b = tid; b < W; b += kThreads) {
    bool k = whole || krow == nullptr || krow[b] != 0;
    if (rrow != nullptr && rrow[b] != 0) k = false;  // released last, block_view.py:280-281
    k = (k || b == 0 || b == n - 1) && b < n;        // block_view.py:51
    s_keep[b] = k ? 1 : 0;
  }
  __syncthreads();

  const int chunk = (W + kThreads - 1) / kThreads;
  const int b0 = min(tid * chunk, W), b1 = min(b0 + chunk, W);
  int kept = 0;
  for (int b = b0; b < b1; ++b) kept += s_keep[b];
  int total_kept;
  int before = block_exclusive_scan<kThreads>(kept, s_scan, total_kept);
  for (int b = b0; b < b1; ++b) {
    const int dst = s_keep[b] ? before : total_kept + (b - before);
    before += s_keep[b];
    s_out[dst] = trow[b];
  }
  __syncthreads();
  if (p.view_table != nullptr) {
    int32_t *vrow = p.view_table + (int64_t)row * p.view_stride;
    for (int b = tid; b < W; b += kThreads) vrow[b] = s_out[b];
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
  if (p.rows < 0 || p.width < 1 || p.width > kMaxWidth || p.block_size < 1)
    return fail(EKV_EINVAL, "block-table view: rows %d, width %d (at most %d), block size %d", p.rows, p.width,
                kMaxWidth, p.block_size);
  if (p.rows == 0) return EKV_OK;
  const size_t lds = (size_t)p.width * (sizeof(int32_t) + 1);
  hipLaunchKernelGGL(view_kernel, dim3(p.rows), dim3(kThreads), lds, (hipStream_t)stream, p);
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
