// The compaction of SGLang's key-value index list: the token-granular form of the view.
// Semantics: runtime/sglang_compact.py:22-167 (plan_kernel, gather_kernel, SlotCompactor.compact).
//
// Request r reads slots[indptr[r] .. indptr[r + 1]), one token slot per entry.  BLOCK_TOKENS
// consecutive entries form a block; the view keeps some blocks of each row.  A row keeps its
// first and its last block always, and all its blocks when the policy is not live (active 0), when
// it is audited in this step, or when it is a row a CUDA graph adds to fill its batch (rows from
// n_real on).  The row's new length is its kept blocks times BLOCK_TOKENS less the unfilled part
// of its last block, and the five read counters grow by the row's blocks.
//
// Three kernels and no host synchronisation:
//  * plan: one workgroup per row.  The row's chosen blocks are ranked with a ballot per wave and
//    a scan over the waves (512 blocks per pass); the rank-th kept block goes to table[row][rank].
//    The counters take one 64-bit atomic add each per row (integer sums, so the order of the
//    rows does not matter).
//  * gather: every workgroup rebuilds the new offsets (an exclusive scan of the new lengths) and
//    the old ones in LDS, finds each output position's row by binary search and copies the slot
//    it comes from; workgroup 0 writes new_indptr.  Past kMaxRows rows (more than LDS holds) one
//    workgroup writes new_indptr and the counters first, and the gather searches new_indptr and
//    indptr in memory instead.
//  * write back (optional): new_indptr into indptr and the new list into slots, in place.
#include "ekv_common.hpp"

namespace ekv {
namespace slots {

constexpr int kPlanThreads = 512;
constexpr int kPlanWaves = kPlanThreads / kWave;
constexpr int kGatherThreads = 256;
constexpr int kPerThread = 4;  // output positions per gather thread
constexpr int kMaxRows = 6000;  // the gather keeps two offsets per row in LDS up to this many rows
constexpr int kOffsetThreads = 1024;  // offsets_kernel, for more rows

struct Params {
  const int32_t *indptr;
  const char *slots;
  int32_t slot_bytes;
  const uint8_t *keep;
  int64_t keep_stride;
  const uint8_t *audit;
  int32_t active, n_real, n_rows, width, block_tokens;
  int32_t *new_indptr;
  int32_t *lens;
  int32_t *table;
  int64_t table_stride;
  char *out;
  long long *counts;
  char *slots_rw;  // write back target (slots itself), or null
  int32_t *indptr_rw;
};

__global__ __launch_bounds__(kPlanThreads) void plan_kernel(const Params p) {
  __shared__ int s_wave[kPlanWaves];
  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  const int length = p.indptr[row + 1] - p.indptr[row];
  const int bt = p.block_tokens;
  const int blocks = length > 0 ? (length + bt - 1) / bt : 0;
  const bool real = row < p.n_real;
  const bool audited = p.audit != nullptr && real && p.audit[row] != 0;
  const bool whole = p.active == 0 || audited || !real;
  const uint8_t *krow = p.keep + (int64_t)row * p.keep_stride;
  int32_t *trow = p.table + (int64_t)row * p.table_stride;
  const int n = min(blocks, p.width);  // a row holds at most width blocks
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));

  int kept = 0;  // chosen blocks before this pass
  for (int base = 0; base < n; base += kPlanThreads) {
    const int b = base + tid;
    bool chosen = false;
    if (b < n) chosen = whole || b == 0 || b == blocks - 1 || (real && krow[b] != 0);
    const uint64_t mask = __ballot(chosen);
    if (lane == 0) s_wave[wave] = __popcll(mask);
    __syncthreads();
    int before = kept;
    for (int w = 0; w < wave; ++w) before += s_wave[w];
    if (chosen) trow[before + __popcll(mask & below)] = b;
    for (int w = 0; w < kPlanWaves; ++w) kept += s_wave[w];
    __syncthreads();
  }
  if (tid == 0) p.lens[row] = blocks > 0 ? (kept - 1) * bt + length - (blocks - 1) * bt : 0;
}

// The counters, runtime/sglang_compact.py:62-73, by one workgroup from every row's old and new
// offsets: a row of `blocks` blocks whose length went from `length` to `new_length` kept
// blocks + (new_length - length) / block_tokens of them.  One uncontended add per counter (the
// rows' workgroups of plan_kernel would otherwise contend on the same five addresses).
template <int NT>
__device__ __forceinline__ void add_counts(const Params &p, const int *s_new, const int *s_old) {
  __shared__ long long s_red[5][NT / kWave];
  const int bt = p.block_tokens;
  long long v[5] = {0, 0, 0, 0, 0};  // read, full, audit, untrimmed, expired
  for (int r = threadIdx.x; r < p.n_real && r < p.n_rows; r += NT) {
    const int length = s_old[r + 1] - s_old[r];
    const int new_length = s_new[r + 1] - s_new[r];
    const int blocks = length > 0 ? (length + bt - 1) / bt : 0;
    const long long kept = blocks > 0 ? blocks + (new_length - length) / bt : 0;
    const bool audited = p.audit != nullptr && p.audit[r] != 0;
    v[0] += kept;
    v[1] += blocks;
    v[2] += audited ? kept : 0;
    v[3] += (new_length == length && !audited && p.active != 0) ? kept : 0;
    v[4] += p.active == 0 ? kept : 0;
  }
  const int wave = threadIdx.x / kWave;
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    v[k] = wave_sum_i64(v[k]);
    if (lane_id() == 0) s_red[k][wave] = v[k];
  }
  __syncthreads();
  if (threadIdx.x < 5) {
    long long t = 0;
    for (int w = 0; w < NT / kWave; ++w) t += s_red[threadIdx.x][w];
    if (t != 0) atomicAdd((unsigned long long *)&p.counts[threadIdx.x], (unsigned long long)t);
  }
}

// new offsets (exclusive scan of lens, total at [n_rows]) and old offsets of every row, in LDS
__device__ __forceinline__ void offsets_in_lds(const Params &p, int *s_new, int *s_old, int *s_scan) {
  const int rows = p.n_rows;
  for (int r = threadIdx.x; r <= rows; r += kGatherThreads) s_old[r] = p.indptr[r];
  const int per = (rows + kGatherThreads - 1) / kGatherThreads;
  const int r0 = threadIdx.x * per, r1 = min(r0 + per, rows);
  int local = 0;
  for (int r = r0; r < r1; ++r) local += p.lens[r];
  int total;
  int base = block_exclusive_scan<kGatherThreads>(local, s_scan, total);
  for (int r = r0; r < r1; ++r) {
    s_new[r] = base;
    base += p.lens[r];
  }
  if (threadIdx.x == 0) s_new[rows] = total;
  __syncthreads();
}

__device__ __forceinline__ void copy_slot(char *dst, const char *src, int bytes) {
  if (bytes == 8) *(uint64_t *)dst = *(const uint64_t *)src;
  else *(uint32_t *)dst = *(const uint32_t *)src;
}

// More rows than LDS holds: the new offsets (new_indptr) and the counters, by one workgroup, before
// the gather reads them from memory.
__global__ __launch_bounds__(kOffsetThreads) void offsets_kernel(const Params p) {
  __shared__ int s_scan[kOffsetThreads / kWave];
  const int rows = p.n_rows;
  const int per = (rows + kOffsetThreads - 1) / kOffsetThreads;
  const int r0 = min((int)threadIdx.x * per, rows), r1 = min(r0 + per, rows);
  int local = 0;
  for (int r = r0; r < r1; ++r) local += p.lens[r];
  int total;
  int base = block_exclusive_scan<kOffsetThreads>(local, s_scan, total);
  for (int r = r0; r < r1; ++r) {
    p.new_indptr[r] = base;
    base += p.lens[r];
  }
  if (threadIdx.x == 0) p.new_indptr[rows] = total;
  if (p.counts == nullptr) return;
  __syncthreads();  // the workgroup's writes of new_indptr are seen by its reads below
  add_counts<kOffsetThreads>(p, p.new_indptr, p.indptr);
}

// OFFSETS_IN_MEMORY: the new offsets in new_indptr (offsets_kernel) and the old ones in indptr.
template <bool OFFSETS_IN_MEMORY>
__global__ __launch_bounds__(kGatherThreads) void gather_kernel(const Params p) {
  extern __shared__ int s_mem[];  // [n_rows + 1] new offsets, [n_rows + 1] old offsets
  __shared__ int s_scan[kGatherThreads / kWave];
  const int *s_new, *s_old;
  if constexpr (OFFSETS_IN_MEMORY) {
    s_new = p.new_indptr;
    s_old = p.indptr;
  } else {
    offsets_in_lds(p, s_mem, s_mem + p.n_rows + 1, s_scan);
    s_new = s_mem;
    s_old = s_mem + p.n_rows + 1;
  }
  const int rows = p.n_rows;
  const int total = s_new[rows];
  if (!OFFSETS_IN_MEMORY && blockIdx.x == 0) {
    for (int r = threadIdx.x; r <= rows; r += kGatherThreads) p.new_indptr[r] = s_new[r];
    if (p.counts != nullptr) add_counts<kGatherThreads>(p, s_new, s_old);
  }
  const int bt = p.block_tokens;
  const int sb = p.slot_bytes;
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int pos = (blockIdx.x * kPerThread + k) * kGatherThreads + threadIdx.x;
    if (pos >= total) continue;
    // the row: the last one whose new offset is <= pos (rows of no entries share an offset)
    int lo = 0, hi = rows;  // s_new[lo] <= pos < s_new[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (s_new[mid] <= pos) lo = mid; else hi = mid;
    }
    const int offset = pos - s_new[lo];
    const int block = p.table[(int64_t)lo * p.table_stride + offset / bt];
    const int64_t source = (int64_t)s_old[lo] + (int64_t)block * bt + offset % bt;
    copy_slot(p.out + (int64_t)pos * sb, p.slots + source * sb, sb);
  }
}

__global__ __launch_bounds__(kGatherThreads) void write_back_kernel(const Params p) {
  const int rows = p.n_rows;
  const int total = p.new_indptr[rows];
  const int sb = p.slot_bytes;
  if (blockIdx.x == 0)
    for (int r = threadIdx.x; r <= rows; r += kGatherThreads) p.indptr_rw[r] = p.new_indptr[r];
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int pos = (blockIdx.x * kPerThread + k) * kGatherThreads + threadIdx.x;
    if (pos < total) copy_slot(p.slots_rw + (int64_t)pos * sb, p.out + (int64_t)pos * sb, sb);
  }
}

}  // namespace slots
}  // namespace ekv

using namespace ekv;

extern "C" int ekv_compact_slots(int32_t *indptr, void *slots_buf, int32_t slot_bytes, const uint8_t *keep,
                                 int64_t keep_stride, const uint8_t *audit, int32_t active, int32_t n_real,
                                 int32_t n_rows, int32_t width, int32_t block_tokens, int64_t entries,
                                 int32_t *new_indptr, int32_t *lens, int32_t *table, int64_t table_stride,
                                 void *out, int64_t *counts, int32_t write_back, void *stream) {
  if (indptr == nullptr || slots_buf == nullptr || (keep == nullptr && n_rows > 0) || new_indptr == nullptr ||
      lens == nullptr || table == nullptr || out == nullptr)
    return fail(EKV_EINVAL, "ekv_compact_slots: null pointer");
  if (slot_bytes != 4 && slot_bytes != 8)
    return fail(EKV_EUNSUPPORTED, "ekv_compact_slots: slots of %d bytes (4 or 8)", slot_bytes);
  if (n_rows < 0 || n_rows >= INT32_MAX || width < 1 || block_tokens < 1 || entries < 0 || entries > INT32_MAX ||
      table_stride < width)
    return fail(EKV_EINVAL, "ekv_compact_slots: rows %d, width %d, block tokens %d, entries %lld", n_rows, width,
                block_tokens, (long long)entries);
  if (n_real < 0) n_real = 0;
  slots::Params p{};
  p.indptr = indptr;
  p.slots = (const char *)slots_buf;
  p.slot_bytes = slot_bytes;
  p.keep = keep;
  p.keep_stride = keep_stride;
  p.audit = audit;
  p.active = active != 0;
  p.n_real = n_real;
  p.n_rows = n_rows;
  p.width = width;
  p.block_tokens = block_tokens;
  p.new_indptr = new_indptr;
  p.lens = lens;
  p.table = table;
  p.table_stride = table_stride;
  p.out = (char *)out;
  p.counts = (long long *)counts;
  p.slots_rw = write_back ? (char *)slots_buf : nullptr;
  p.indptr_rw = write_back ? indptr : nullptr;
  hipStream_t s = (hipStream_t)stream;
  int rc = EKV_OK;
  if (n_rows > 0) {  // no rows: the gather alone writes new_indptr = [0]
    hipLaunchKernelGGL(slots::plan_kernel, dim3(n_rows), dim3(slots::kPlanThreads), 0, s, p);
    rc = check_hip(hipGetLastError(), "ekv_compact_slots plan launch");
    if (rc != EKV_OK) return rc;
  }
  // the new list is never longer than the old one
  const int64_t per_block = (int64_t)slots::kGatherThreads * slots::kPerThread;
  const int64_t grid = entries > 0 ? (entries + per_block - 1) / per_block : 1;
  if (n_rows <= slots::kMaxRows) {
    const size_t lds = (size_t)2 * (n_rows + 1) * sizeof(int);
    hipLaunchKernelGGL(slots::gather_kernel<false>, dim3((unsigned)grid), dim3(slots::kGatherThreads), lds, s, p);
  } else {  // more rows than LDS holds: the offsets go through memory
    hipLaunchKernelGGL(slots::offsets_kernel, dim3(1), dim3(slots::kOffsetThreads), 0, s, p);
    hipLaunchKernelGGL(slots::gather_kernel<true>, dim3((unsigned)grid), dim3(slots::kGatherThreads), 0, s, p);
  }
  rc = check_hip(hipGetLastError(), "ekv_compact_slots gather launch");
  if (rc != EKV_OK || !write_back) return rc;
  hipLaunchKernelGGL(slots::write_back_kernel, dim3((unsigned)grid), dim3(slots::kGatherThreads), 0, s, p);
  return check_hip(hipGetLastError(), "ekv_compact_slots write back launch");
}
