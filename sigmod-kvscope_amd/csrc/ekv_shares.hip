// Exact per-block attention shares from the tile records, on the device.
// Semantics: read_tile_rows (observe/tile_shares.py:129-173) forms u = m + log(l) - log(T) from
// the two planes; normalize_tile_lse (observe/tile_shares.py:58-103) gives a partial last tile's
// blocks back log(T / valid_in_tail), drops cells past the row, turns every (layer, query row)
// with a finite value into a softmax over the row's blocks, and averages them (or takes the
// renormalised per-block max).  The reference copies the planes to the host and does this in
// float64 NumPy; here it runs in float32 on the planes where the audit kernel wrote them.
//
// Algebra.  exp(u - c) = l * t * exp(m - c) / T, with t = T / valid on a partial last tile and 1
// elsewhere.  The 1/T cancels in every softmax, so with the weight w = l * t the softmax of a
// (layer, query row) record over its blocks is w_b exp(m_b - M) / sum w exp(m - M) for any M,
// and no logarithm is taken.  M = the largest m of the record keeps every term at most w (l is
// a sum of at most T * block_size exponentials no larger than 1).  u is finite -- the block
// carries weight -- iff m is finite and 0 < l < inf.  With u planes (ekv_normalize_tile_lse),
// m = u and l = 1.
//
// A workgroup takes one output row and a range of its layers.  Phase 1: the layers are spread over
// the waves; for each the row's [width][cells] records are streamed (coalesced; when the cells
// come in 16-byte quads, as for a group of 4 query rows, a lane loads a block's quad at once; 8
// loads of each plane in flight per lane) with a running (max m, sum w exp(m - max)) per cell,
// which a butterfly over the lanes holding the same cells turns into the record's peak and total,
// kept in LDS.  Phase 2: the row's blocks x layer groups are spread over the workgroup; each
// thread sums (or maxes) its block's shares over its layers and query rows in a fixed order, and
// the group partials are combined in LDS in a fixed order.
//
// Three forms.  Without a workspace one 1024-thread workgroup takes a whole row, so the longest row
// sets the time (its records are read twice by one CU).  With a workspace (ekv_tile_shares_ws)
// the layers are split into K groups whose workgroups write per-block partial sums (or maxes) and
// their contributor counts: for 4 query rows and rows of at most 512 blocks (shares_wave_kernel)
// the last of a row's workgroups to finish adds them and writes the row, otherwise a second kernel
// (combine_kernel) adds each row's K partials in group order.  Every form adds in a fixed order,
// so the results are the same on every call (the wave form's arrival counter only picks which
// workgroup adds the partials).
#include <limits.h>
#include <math.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "ekv_common.hpp"

// The scratch of ekv_tile_shares_noalloc: the split form's partials and contributor counts, held
// by the library on every device it runs on until the process ends.  Host code never passes this
// name to a kernel (on the host it is only a stand-in for the symbol): it uses the device address
// that hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) unsigned char scratch[EKV_TILE_SHARES_SCRATCH_BYTES];

namespace ekv {
namespace shares {

constexpr int kThreads = 1024;      // a whole row per workgroup
constexpr int kSplitThreads = 256;  // a (row, layer group) per workgroup
constexpr int kBatch = 8;  // quads (or cells) of each plane in flight per lane
constexpr int kMaxCells = 64;
constexpr int kMaxStats = 8000;  // layers * padded cells: 2 floats each in LDS (64 KB)
constexpr int kWaveLayers = 8;   // the wave form: one layer per wave, 8 or 16 waves per workgroup
constexpr int kMaxArrivalRows = 65536;  // rows whose arrival counters the workspace holds
constexpr size_t kHeaderBytes = 256;    // the workspace's status word, then padding
constexpr size_t kArrivalBytes = (size_t)kMaxArrivalRows * sizeof(int32_t);

struct Params {
  const float *m;  // plane 0 (or u when from_u)
  const float *l;  // plane 1 (unused when from_u)
  int64_t layer_stride, row_stride;
  int32_t layers, cells, cells_pow2, width;
  const int32_t *row_ids, *row_blocks;
  int32_t tile_blocks, aggregate, from_u;
  int32_t lanes_per_layer;  // the peak pass's lanes per layer (quads path)
  float *shares;
  int64_t shares_stride;
  int32_t groups;      // layer groups per row (the split form), 1 otherwise
  float *part;         // split form: [rows][groups][width] partial sums (or maxes)
  int32_t *part_count; // split form: [rows][groups] contributing (layer, query row) pairs
  int32_t *arrivals;   // wave form: [rows] workgroups of the row done so far (0 between calls)
  int32_t *status;     // wave form: the workspace's sticky status word (non-zero after a lost slot)
  int32_t spin_limit;  // wave form: reloads of a slot before its value is taken as lost
  int32_t lose;        // wave form, for tests of the failure path: no slot is ever seen as landed
};

typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bool finite(float x) { return __builtin_isfinite(x); }

// The row's weight rule.  n is the row's length in blocks, which may exceed the width: the tail
// rule uses it unclipped (tile_shares.py:84-87).
struct RowWeight {
  int tail_start;   // first block of a partial last tile (INT_MAX when the last tile is whole)
  float tail_mult;  // T / blocks in that tile
  bool from_u;

  __device__ RowWeight(const Params &p, int n) {
    const int T = p.tile_blocks;
    const int whole = (n / T) * T;
    tail_start = n != whole ? whole : INT_MAX;
    tail_mult = n != whole ? (float)T / (float)(n - whole) : 1.0f;
    from_u = p.from_u != 0;
  }
  // w of block b's record from its two plane values; 0 when the record carries no weight
  __device__ __forceinline__ float operator()(float m, float l, int b) const {
    const float lw = from_u ? 1.0f : l;
    const bool carries = finite(m) && lw > 0.0f && lw < INFINITY;
    return carries ? (b >= tail_start ? lw * tail_mult : lw) : 0.0f;
  }
};

// merge two (max, sum w exp(m - max)) pairs
__device__ __forceinline__ void merge(float &m, float &s, float m2, float s2) {
  const float M = fmaxf(m, m2);
  if (M == -INFINITY) return;
  const float a = m == -INFINITY ? 0.0f : s * __expf(m - M);
  const float b = m2 == -INFINITY ? 0.0f : s2 * __expf(m2 - M);
  m = M;
  s = a + b;
}

// running (max, sum) after a batch of N (m, w) pairs (w = 0: no weight)
template <int N>
__device__ __forceinline__ void absorb(float &mx, float &sum, const float (&m)[N], const float (&w)[N]) {
  float bm = -INFINITY;
#pragma unroll
  for (int k = 0; k < N; ++k) bm = w[k] > 0.0f ? fmaxf(bm, m[k]) : bm;
  if (bm > mx) {
    sum *= __expf(mx - bm);  // mx = -inf: sum is 0 and stays 0
    mx = bm;
  }
#pragma unroll
  for (int k = 0; k < N; ++k) sum += w[k] > 0.0f ? w[k] * __expf(m[k] - mx) : 0.0f;
}

// VEC: the cells of a block come in 16-byte quads (cells a multiple of 4, cells / 4 a power of
// two, 16-byte aligned planes and strides), so one lane loads a quad with one instruction and
// quad e of a (layer, row) record is at 4 e.  Otherwise every cell is loaded on its own.
template <bool VEC, int NT, bool SPLIT>
__global__ __launch_bounds__(NT) void shares_kernel(const Params p) {
  constexpr int kWaves = NT / kWave;
  extern __shared__ float s_stats[];  // [layers][cells_pow2] peak, then [layers][cells_pow2] 1/total
  __shared__ float s_part[NT];        // per (layer group, block) partial shares
  __shared__ float s_red[kWaves];
  __shared__ int s_contrib;

  const int out_row = SPLIT ? blockIdx.x / p.groups : blockIdx.x;
  const int group = SPLIT ? blockIdx.x - out_row * p.groups : 0;
  // this workgroup's layers [l_first, l_first + nl); stats are indexed from l_first
  const int l_first = SPLIT ? group * p.layers / p.groups : 0;
  const int nl = SPLIT ? (group + 1) * p.layers / p.groups - l_first : p.layers;
  const int src_row = p.row_ids != nullptr ? p.row_ids[out_row] : out_row;
  const int n_row = p.row_blocks != nullptr ? max(p.row_blocks[out_row], 0) : p.width;
  const int n = min(n_row, p.width);  // blocks with records
  const int CP = p.cells_pow2, cp_log2 = __builtin_ctz(CP);
  const int cells = p.cells;
  const RowWeight weight(p, n_row);
  const int64_t row_base = (int64_t)src_row * p.row_stride;
  // the l plane; for u input the m plane again (loaded unconditionally, so that no load waits for
  // another; the weight ignores it)
  const float *lplane = weight.from_u ? p.m : p.l;
  float *peak = s_stats;
  float *inv_total = s_stats + nl * CP;
  if (threadIdx.x == 0) s_contrib = 0;
  __syncthreads();

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;

  // ---- phase 1: peak and total of every (layer, query row) ------------------------------
  int contrib = 0;
  if constexpr (VEC) {
    // LPL lanes take one layer (several layers per wave when there are few blocks per lane), each
    // lane a running (max, sum) per cell of its quads; the lanes of a layer then reduce the max,
    // rescale their sums once and reduce the sums
    const int QP = cells >> 2, qp_log2 = __builtin_ctz(QP);  // quads per block, dividing 64
    const int LPL = p.lanes_per_layer;                       // a power of two, QP <= LPL <= 64
    const int sub = lane & (LPL - 1);
    const int slot = sub & (QP - 1);  // the quad of the block every element of this lane is in
    const int slots = NT / LPL;  // layers reduced at once by the workgroup
    const int quads = n * QP;
    for (int layer = (tid / LPL); layer - (tid / LPL) < nl; layer += slots) {
      const bool live = layer < nl;
      const int64_t base = (int64_t)(l_first + (live ? layer : 0)) * p.layer_stride + row_base;
      const f32x4_t *mq = reinterpret_cast<const f32x4_t *>(p.m + base);
      const f32x4_t *lq = reinterpret_cast<const f32x4_t *>(lplane + base);
      float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY}, sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int e0 = sub; live && e0 < quads; e0 += LPL * kBatch) {
        f32x4_t mv[kBatch], lv[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          const int at = e0 + k * LPL < quads ? e0 + k * LPL : 0;
          mv[k] = mq[at];
          lv[k] = lq[at];  // the m plane again for u input (its weight ignores it)
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float m[kBatch], w[kBatch];
#pragma unroll
          for (int k = 0; k < kBatch; ++k) {
            const int e = e0 + k * LPL;
            m[k] = mv[k][j];
            w[k] = e < quads ? weight(mv[k][j], lv[k][j], e >> qp_log2) : 0.0f;
          }
          absorb(mx[j], sum[j], m, w);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float M = mx[j];
        for (int msk = QP; msk < LPL; msk <<= 1) M = fmaxf(M, shfl_xor(M, msk));
        float t = (mx[j] == -INFINITY) ? 0.0f : sum[j] * __expf(mx[j] - M);
        for (int msk = QP; msk < LPL; msk <<= 1) t += shfl_xor(t, msk);
        mx[j] = M;
        sum[j] = t;
      }
      if (live && sub < QP) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int c = 4 * slot + j;
          const bool has = mx[j] != -INFINITY;
          peak[layer * CP + c] = has ? mx[j] : NAN;
          inv_total[layer * CP + c] = has ? 1.0f / sum[j] : 0.0f;
          contrib += has ? 1 : 0;
        }
      }
    }
  } else {
    const int q = lane & (CP - 1);  // every element a lane visits has this query row (CP divides 64)
    const int span = n * CP;
    for (int layer = wave; layer < nl; layer += kWaves) {
      const float *mrow = p.m + (int64_t)(l_first + layer) * p.layer_stride + row_base;
      const float *lrow = lplane + (int64_t)(l_first + layer) * p.layer_stride + row_base;
      float mx = -INFINITY, sum = 0.0f;
      if (q < cells) {
        for (int e0 = lane; e0 < span; e0 += kWave * kBatch) {
          float m[kBatch], w[kBatch];
#pragma unroll
          for (int k = 0; k < kBatch; ++k) {
            const int e = e0 + k * kWave;
            const int idx = e < span ? (e >> cp_log2) * cells + q : 0;
            m[k] = mrow[idx];
            w[k] = lrow[idx];
          }
#pragma unroll
          for (int k = 0; k < kBatch; ++k) {
            const int e = e0 + k * kWave;
            w[k] = e < span ? weight(m[k], w[k], e >> cp_log2) : 0.0f;
          }
          absorb(mx, sum, m, w);
        }
      }
      for (int msk = CP; msk < kWave; msk <<= 1) {
        const float m2 = shfl_xor(mx, msk);
        const float s2 = shfl_xor(sum, msk);
        merge(mx, sum, m2, s2);
      }
      if (lane < CP) {
        const bool has = lane < cells && mx != -INFINITY;
        peak[layer * CP + lane] = has ? mx : NAN;
        inv_total[layer * CP + lane] = has ? 1.0f / sum : 0.0f;
        contrib += has ? 1 : 0;
      }
    }
  }
  contrib = wave_sum_int(contrib);
  if (lane == 0 && contrib) atomicAdd(&s_contrib, contrib);
  __syncthreads();
  const int contributors = s_contrib;

  float *out = p.shares + (int64_t)out_row * p.shares_stride;
  if constexpr (SPLIT) {
    if (tid == 0) p.part_count[(int64_t)out_row * p.groups + group] = contributors;
    if (contributors == 0) {  // nothing from these layers: zero partials
      float *part = p.part + ((int64_t)out_row * p.groups + group) * p.width;
      for (int b = tid; b < p.width; b += NT) part[b] = 0.0f;
      return;
    }
  } else if (contributors == 0) {  // no evidence about the row, tile_shares.py:103
    for (int b = tid; b < p.width; b += NT) out[b] = NAN;
    return;
  }

  // ---- phase 2: per-block shares, summed (or maxed) over (layer, query row) in a fixed order
  const bool use_max = p.aggregate == EKV_AGG_MAX;
  // block b's shares over layers [l0, l1) of this workgroup's range (stats index)
  auto shares_of = [&](int b, int l0, int l1) -> float {
    float acc = 0.0f;
    const int64_t block_base = row_base + (int64_t)b * cells;
    if constexpr (VEC) {
      const int QP = cells >> 2, qp_log2 = __builtin_ctz(QP);
      const int r_end = l1 * QP;  // quad rq = (layer rq / QP, cells 4 (rq % QP) ..)
      for (int r0 = l0 * QP; r0 < r_end; r0 += kBatch) {
        f32x4_t mv[kBatch], lv[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          const int rq = r0 + k < r_end ? r0 + k : r0;
          const int64_t at = (int64_t)(l_first + (rq >> qp_log2)) * p.layer_stride + block_base + 4 * (rq & (QP - 1));
          mv[k] = *reinterpret_cast<const f32x4_t *>(p.m + at);
          lv[k] = *reinterpret_cast<const f32x4_t *>(lplane + at);
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          const int rq = r0 + k;
          if (rq >= r_end) break;
          const int stat = (rq >> qp_log2) * CP + 4 * (rq & (QP - 1));
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float w = weight(mv[k][j], lv[k][j], b);  // > 0 only where phase 1 found a peak
            const float share = w > 0.0f ? w * __expf(mv[k][j] - peak[stat + j]) * inv_total[stat + j] : 0.0f;
            acc = use_max ? fmaxf(acc, share) : acc + share;
          }
        }
      }
    } else {
      const int r_end = l1 * cells;  // record r = (layer r / cells, cell r % cells)
      for (int r0 = l0 * cells; r0 < r_end; r0 += kBatch) {
        float mv[kBatch], lv[kBatch];
        int stat[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          const int rec = r0 + k < r_end ? r0 + k : r0;
          const int layer = rec / cells, c = rec - layer * cells;
          const int64_t at = (int64_t)(l_first + layer) * p.layer_stride + block_base + c;
          stat[k] = layer * CP + c;
          mv[k] = p.m[at];
          lv[k] = lplane[at];
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          if (r0 + k >= r_end) break;
          const float w = weight(mv[k], lv[k], b);
          const float share = w > 0.0f ? w * __expf(mv[k] - peak[stat[k]]) * inv_total[stat[k]] : 0.0f;
          acc = use_max ? fmaxf(acc, share) : acc + share;
        }
      }
    }
    return acc;
  };

  // the row's n blocks (rounded up to whole waves) times LG layer groups fill the workgroup;
  // the split form writes its sums (or maxes) over its layers, the whole-row form the shares
  float *part = SPLIT ? p.part + ((int64_t)out_row * p.groups + group) * p.width : nullptr;
  const int NC = ((n + kWave - 1) / kWave) * kWave;
  const int LG = NC >= NT ? 1 : min(NT / NC, nl);
  float local_total = 0.0f;
  if (LG > 1) {
    const int g = tid / NC, col = tid - g * NC;
    float acc = 0.0f;
    if (g < LG && col < n) acc = shares_of(col, g * nl / LG, (g + 1) * nl / LG);
    s_part[tid] = acc;  // = s_part[g * NC + col]
    __syncthreads();
    for (int b = tid; b < p.width; b += NT) {
      float v = 0.0f;
      if (b < n) {
        for (int h = 0; h < LG; ++h) v = use_max ? fmaxf(v, s_part[h * NC + b]) : v + s_part[h * NC + b];
      }
      local_total += v;
      if constexpr (SPLIT) part[b] = v;
      else out[b] = use_max ? v : v / (float)contributors;
    }
  } else {
    for (int b = tid; b < p.width; b += NT) {
      const float v = b < n ? shares_of(b, 0, nl) : 0.0f;
      local_total += v;
      if constexpr (SPLIT) part[b] = v;
      else out[b] = use_max ? v : v / (float)contributors;
    }
  }
  if (!SPLIT && use_max) {  // renormalise the per-block max, tile_shares.py:97-100
    const float total = block_sum<NT>(local_total, s_red);
    for (int b = tid; b < p.width; b += NT) out[b] = total > 0.0f ? out[b] / total : 0.0f;
  }
}

// Transpose reduction of a[0 .. CUR) over the lanes: each step halves the values a lane carries
// (the lane with the mask bit keeps the upper half and receives its partner's), so CUR values take
// CUR - 1 shuffles and then sit one per lane; the remaining masks finish the reduction.
template <int CUR, int MASK, int N, bool MAX>
__device__ __forceinline__ void transpose_reduce(float (&a)[N], int lane) {
  if constexpr (MASK >= 1) {
    if constexpr (CUR > 1) {
      constexpr int kHalf = CUR / 2;
      const bool upper = (lane & MASK) != 0;
#pragma unroll
      for (int k = 0; k < kHalf; ++k) {
        const float send = upper ? a[k] : a[k + kHalf];
        const float keep = upper ? a[k + kHalf] : a[k];
        const float got = shfl_xor(send, MASK);
        a[k] = MAX ? fmaxf(keep, got) : keep + got;
      }
      transpose_reduce<kHalf, MASK / 2, N, MAX>(a, lane);
    } else {
      const float got = shfl_xor(a[0], MASK);
      a[0] = MAX ? fmaxf(a[0], got) : a[0] + got;
      transpose_reduce<1, MASK / 2, N, MAX>(a, lane);
    }
  }
}

// The split form for quads of 4 cells and rows of at most 256 J blocks: one pass over memory.
// Thread t keeps blocks t + 256 j (j < J) of each of the group's NL layers in registers, the peak
// and total of each (layer, query row) are workgroup reductions over them (butterflies, then the
// waves' results in LDS in wave order), and the block's partial is formed from the same registers.
template <int J, int NL>
__global__ __launch_bounds__(kSplitThreads) void shares_reg_kernel(const Params p) {
  constexpr int NT = kSplitThreads, NW = NT / kWave, V = NL * 4;  // V: the group's (layer, cell) pairs
  static_assert(V <= kWave && (V & (V - 1)) == 0, "a power of two of pairs, at most a wave");
  __shared__ float s_red[NW][V];
  const int out_row = blockIdx.x / p.groups;
  const int group = blockIdx.x - out_row * p.groups;
  const int l_first = group * p.layers / p.groups;
  const int nl = (group + 1) * p.layers / p.groups - l_first;  // <= NL
  const int src_row = p.row_ids != nullptr ? p.row_ids[out_row] : out_row;
  const int n_row = p.row_blocks != nullptr ? max(p.row_blocks[out_row], 0) : p.width;
  const int n = min(n_row, p.width);
  const RowWeight weight(p, n_row);
  const int64_t row_base = (int64_t)src_row * p.row_stride;
  const float *lplane = weight.from_u ? p.m : p.l;
  const int t = threadIdx.x, lane = lane_id(), wave = t / kWave;

  // the thread's records: m and the weight w (0: the record carries none).  Every load is issued
  // before any is used, so all are in flight at once; an absent record (past the row or the
  // group) reads the row's first record, which costs no memory traffic, and is masked afterwards.
  f32x4_t mv[J][NL], wv[J][NL];
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int li = 0; li < NL; ++li) {
      const int b = t + NT * j;
      const bool live = b < n && li < nl;
      const int64_t at = live ? (int64_t)(l_first + li) * p.layer_stride + row_base + 4 * (int64_t)b
                              : (int64_t)l_first * p.layer_stride + row_base;
      mv[j][li] = *reinterpret_cast<const f32x4_t *>(p.m + at);
      wv[j][li] = *reinterpret_cast<const f32x4_t *>(lplane + at);
    }
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int li = 0; li < NL; ++li) {
      const bool live = t + NT * j < n && li < nl;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        wv[j][li][c] = live ? weight(mv[j][li][c], wv[j][li][c], t + NT * j) : 0.0f;
        mv[j][li][c] = live ? mv[j][li][c] : -INFINITY;
      }
    }

  // a workgroup-wide max or sum of v[0 .. V); every thread gets the results: a transpose
  // reduction in each wave (value lane / (64 / V) ends in that lane), then the waves' results
  // meet in LDS in wave order
  auto reduce = [&](float (&v)[V], auto max_tag) {
    constexpr bool is_max = decltype(max_tag)::value;
    transpose_reduce<V, kWave / 2, V, is_max>(v, lane);
    constexpr int kLanesPerValue = kWave / V;
    if ((lane & (kLanesPerValue - 1)) == 0) s_red[wave][lane / kLanesPerValue] = v[0];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < V; ++k) {
      float r = s_red[0][k];
#pragma unroll
      for (int w = 1; w < NW; ++w) r = is_max ? fmaxf(r, s_red[w][k]) : r + s_red[w][k];
      v[k] = r;
    }
    __syncthreads();
  };

  // ---- phase 1: peak M and total T of each (layer, query row) ----------------------------
  float peak[V], total[V];
#pragma unroll
  for (int li = 0; li < NL; ++li)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < J; ++j) mx = wv[j][li][c] > 0.0f ? fmaxf(mx, mv[j][li][c]) : mx;
      peak[li * 4 + c] = mx;
    }
  reduce(peak, std::true_type{});
  // each record's term w exp(m - M) replaces its weight (m is not needed again), which keeps the
  // kernel within the registers of four workgroups per compute unit
#pragma unroll
  for (int li = 0; li < NL; ++li)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float sum = 0.0f;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const float term = wv[j][li][c] > 0.0f ? wv[j][li][c] * __expf(mv[j][li][c] - peak[li * 4 + c]) : 0.0f;
        wv[j][li][c] = term;
        sum += term;
      }
      total[li * 4 + c] = sum;
    }
  reduce(total, std::false_type{});
  int contributors = 0;
#pragma unroll
  for (int k = 0; k < V; ++k) {
    contributors += peak[k] != -INFINITY ? 1 : 0;
    total[k] = 1.0f / total[k];  // now 1 / T (used only where T > 0)
  }

  // ---- phase 2: the block's partial over the group's pairs --------------------------------
  const bool use_max = p.aggregate == EKV_AGG_MAX;
  float *part = p.part + ((int64_t)out_row * p.groups + group) * p.width;
  if (t == 0) p.part_count[(int64_t)out_row * p.groups + group] = contributors;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int b = t + NT * j;
    if (b >= p.width) continue;
    float acc = 0.0f;
#pragma unroll
    for (int li = 0; li < NL; ++li)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float term = wv[j][li][c];  // > 0 only where phase 1 found a peak
        const float share = term > 0.0f ? term * total[li * 4 + c] : 0.0f;
        acc = use_max ? fmaxf(acc, share) : acc + share;
      }
    part[b] = acc;
  }
}

// Four values per lane reduced over the wave: afterwards lane 16 r holds value r's reduction (and
// so does every lane of 16-lane row r).  Values 0 and 2, then 1 and 3, trade wave halves
// (v_permlane32_swap), the two results trade 16-lane rows (v_permlane16_swap), and each row
// finishes with rotations by 8, 4, 2 and 1 lanes (DPP row_ror), so no value goes through LDS.  The
// lanes of a row may hold differently rounded sums; callers read lane 16 r.
template <bool MAX>
__device__ __forceinline__ float wave_reduce4(const float (&v)[4]) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  auto swap = [](float x, float y, auto rows16) {
    uint32_t xi = __builtin_bit_cast(uint32_t, x), yi = __builtin_bit_cast(uint32_t, y);
    asm volatile("" : "+v"(xi), "+v"(yi));
    uint32_t r0, r1;
    if constexpr (decltype(rows16)::value) {
      const auto r = __builtin_amdgcn_permlane16_swap(xi, yi, false, false);
      r0 = r[0];
      r1 = r[1];
    } else {
      const auto r = __builtin_amdgcn_permlane32_swap(xi, yi, false, false);
      r0 = r[0];
      r1 = r[1];
    }
    asm volatile("" : "+v"(r0), "+v"(r1));
    return MAX ? fmaxf(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1))
               : __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
  };
  // lanes 0-31: value 0 (resp. 1), lanes 32-63: value 2 (resp. 3)
  const float x = swap(v[0], v[2], std::false_type{});
  const float y = swap(v[1], v[3], std::false_type{});
  // row r: value r, over lanes l, l + 16, l + 32, l + 48
  float z = swap(x, y, std::true_type{});
  auto ror = [](float a, auto ctrl) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, a),
                                                                 decltype(ctrl)::value, 0xf, 0xf, false));
  };
  z = op(z, ror(z, std::integral_constant<int, 0x128>{}));
  z = op(z, ror(z, std::integral_constant<int, 0x124>{}));
  z = op(z, ror(z, std::integral_constant<int, 0x122>{}));
  z = op(z, ror(z, std::integral_constant<int, 0x121>{}));
  return z;
}

__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// The wave form's workspace slots hold a value plus one, so that a slot reads 0 until its value
// has landed: a partial's bits plus one (a NaN with every bit set is stored as the quiet NaN), a
// count plus one.  The workgroup that adds a row's partials waits on each slot it reads until it is
// non-zero, then sets it back to 0; combine_kernel clears the slots it reads too, so that between
// calls every slot of the workspace is 0.
constexpr int kSpinLimit = 1 << 20;  // reloads of a slot before the value is taken as lost

__device__ __forceinline__ uint32_t slot_of(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  return (u == 0xFFFFFFFFu ? 0x7FC00000u : u) + 1u;
}

__device__ __forceinline__ uint32_t load_slot(const uint32_t *at) {
  return __hip_atomic_load(at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void store_slot(uint32_t *at, uint32_t v) {
  __hip_atomic_store(at, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// the slot's value once it has landed (0 when it was first read), or 0 after `limit` reloads (with
// `lose`, a test of the failure path, no value is taken: every wait runs to its limit)
__device__ __forceinline__ uint32_t landed(const uint32_t *at, uint32_t first, int limit, bool lose) {
  uint32_t v = lose ? 0u : first;
  for (int k = 0; v == 0u && k < limit; ++k) {
    __builtin_amdgcn_s_sleep(1);
    v = lose ? 0u : load_slot(at);
  }
  return v;
}

// The wave form for quads of 4 cells and rows of at most 64 S blocks: one pass over memory, and a
// (layer, query row)'s softmax never leaves its wave.  Wave w of a workgroup takes layer
// 8 g + w of layer group g of the row; lane i keeps blocks i + 64 s (s < S) of that layer in
// registers, so the peak and total of each query row are wave reductions (wave_reduce4) and the
// slots past the row's blocks are skipped by the whole wave.  The layers' per-block shares meet in
// LDS and are added in layer order.  A row of several groups writes each group's partial to the
// workspace; the last of the row's workgroups to finish (counted in arrivals[row], which it
// resets) adds them in group order and writes the row, so no second kernel runs.
template <int S, int NW>
__global__ __launch_bounds__(NW *kWave) __attribute__((amdgpu_waves_per_eu(4)))
void shares_wave_kernel(const Params p) {
  constexpr int NT = NW * kWave, kSlots = S * kWave;
  static_assert(kSlots <= NT, "a thread per block in the layer sums");
  __shared__ float s_part[NW][kSlots];
  __shared__ int s_count[NW];
  __shared__ float s_red[NW];
  __shared__ int s_last;
  __shared__ int s_status;
  const int out_row = blockIdx.x / p.groups;
  const int group = blockIdx.x - out_row * p.groups;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = lane_id();
  const int nl = min(NW, p.layers - group * NW);  // the group's layers
  const bool mine = wave < nl;                     // this wave has a layer
  const int src_row = p.row_ids != nullptr ? p.row_ids[out_row] : out_row;
  const int n_row = p.row_blocks != nullptr ? max(p.row_blocks[out_row], 0) : p.width;
  const int n = min(n_row, p.width);
  const RowWeight weight(p, n_row);  // planes of m and l (never u values: those take no workspace)
  const int64_t base = (int64_t)(group * NW + (mine ? wave : 0)) * p.layer_stride + (int64_t)src_row * p.row_stride;

  // the lane's records; a slot the whole wave has past the row is neither loaded nor used
  float mv[S][4], wv[S][4];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    if (mine && s * kWave < n) {
      const int b = s * kWave + lane;
      const int64_t at = base + 4 * (int64_t)(b < n ? b : 0);
      const f32x4_t mq = *reinterpret_cast<const f32x4_t *>(p.m + at);
      const f32x4_t lq = *reinterpret_cast<const f32x4_t *>(p.l + at);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        mv[s][c] = mq[c];
        wv[s][c] = lq[c];
      }
    }
  }
  // weights (0: the record carries none, its m then -inf) and the lane's peak per query row
  float red[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
  for (int s = 0; s < S; ++s) {
    if (mine && s * kWave < n) {
      const int b = s * kWave + lane;
      const bool live = b < n;
      const float tail = b >= weight.tail_start ? weight.tail_mult : 1.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float m = mv[s][c], l = wv[s][c];
        const bool carries = live && finite(m) && l > 0.0f && l < INFINITY;
        wv[s][c] = carries ? l * tail : 0.0f;
        mv[s][c] = carries ? m : -INFINITY;
        red[c] = mv[s][c] > red[c] ? mv[s][c] : red[c];  // no NaN here: a plain compare
      }
    }
  }
  float peak[4];
  int contributors = 0;
  {
    float z = wave_reduce4<true>(red);
    const bool found = z != -INFINITY;
    z = found ? z : 0.0f;  // a query row with no weight: its terms are w * exp(-inf) = 0
    const uint64_t rows_found = __ballot(found);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      peak[c] = lane_value(z, 16 * c);
      contributors += mine ? (int)((rows_found >> (16 * c)) & 1) : 0;
    }
  }
  // each record's term w exp(m - M) replaces its weight; the lane's totals per query row
#pragma unroll
  for (int c = 0; c < 4; ++c) red[c] = 0.0f;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    if (mine && s * kWave < n) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float term = wv[s][c] * __expf(mv[s][c] - peak[c]);
        wv[s][c] = term;
        red[c] += term;
      }
    }
  }
  float inv_total[4];
  {
    const float z = wave_reduce4<false>(red);
    const float inv = z > 0.0f ? 1.0f / z : 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) inv_total[c] = lane_value(inv, 16 * c);
  }
  // the layer's share of each block, summed (or maxed) over its query rows
  const bool use_max = p.aggregate == EKV_AGG_MAX;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    if (mine && s * kWave < n) {
      float sh;
      if (use_max) {
        sh = fmaxf(fmaxf(wv[s][0] * inv_total[0], wv[s][1] * inv_total[1]),
                   fmaxf(wv[s][2] * inv_total[2], wv[s][3] * inv_total[3]));
      } else {
        sh = wv[s][0] * inv_total[0];
        sh = fmaf(wv[s][1], inv_total[1], sh);
        sh = fmaf(wv[s][2], inv_total[2], sh);
        sh = fmaf(wv[s][3], inv_total[3], sh);
      }
      s_part[wave][s * kWave + lane] = sh;
    }
  }
  if (lane == 0) s_count[wave] = contributors;
  if (threadIdx.x == 0)
    s_status = p.groups > 1 ? __hip_atomic_load(p.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
  __syncthreads();

  // the group's partial of block b = threadIdx.x, over its layers in order
  const int b = threadIdx.x;
  float v = 0.0f;
  if (b < n) {
    for (int w = 0; w < nl; ++w) v = use_max ? fmaxf(v, s_part[w][b]) : v + s_part[w][b];
  }
  int count = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) count += s_count[w];

  if (p.groups > 1 && s_status != 0) {
    // A slot of an earlier call was lost and may still be written: until the workspace is reset,
    // no slot is used and the row comes out without evidence (NaN).
    if (group == 0 && b < p.width) p.shares[(int64_t)out_row * p.shares_stride + b] = NAN;
    return;
  }
  if (p.groups > 1) {
    // The partials and counts cross workgroups (and XCDs) through device-coherent stores and
    // loads, which pass the per-XCD L2 caches; a fence would instead write back and invalidate
    // the whole L2 of the XCD.  A workgroup counts its arrival without waiting for its stores to
    // complete: the last workgroup of the row, which adds the partials, waits on each slot until
    // its value has landed (slots read 0 until then) and sets it back to 0.
    uint32_t *part = reinterpret_cast<uint32_t *>(p.part) + (int64_t)out_row * p.groups * p.width;
    uint32_t *counts = reinterpret_cast<uint32_t *>(p.part_count) + (int64_t)out_row * p.groups;
    if (b < n) store_slot(&part[(int64_t)group * p.width + b], slot_of(v));
    if (threadIdx.x == 0) {
      store_slot(&counts[group], (uint32_t)count + 1u);
      s_last = __hip_atomic_fetch_add(&p.arrivals[out_row], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               p.groups - 1;
    }
    __syncthreads();
    if (!s_last) return;
    // this group's own slots, written before it knew it was last, are cleared as well
    if (b < n) store_slot(&part[(int64_t)group * p.width + b], 0u);
    if (threadIdx.x == 0) {
      store_slot(&counts[group], 0u);
      __hip_atomic_store(&p.arrivals[out_row], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // every group's partial of block b, in group order (this group's from registers), and, by
    // thread 0 in the same batches, their contributor counts (a count slot is read by one thread
    // only, so that it is cleared after its last read)
    float acc = 0.0f;
    int total = count;
    bool lost = false, lost_count = false;
    const bool counter = threadIdx.x == 0;
    for (int g0 = 0; g0 < p.groups; g0 += kBatch) {
      uint32_t x[kBatch], c[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int g = g0 + k;
        const bool other = g < p.groups && g != group;
        x[k] = other && b < n ? load_slot(&part[(int64_t)g * p.width + b]) : 1u;
        c[k] = other && counter ? load_slot(&counts[g]) : 1u;
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int g = g0 + k;
        float xv = 0.0f;
        if (g == group) {
          xv = v;
        } else if (g < p.groups) {
          if (b < n) {
            x[k] = landed(&part[(int64_t)g * p.width + b], x[k], p.spin_limit, p.lose != 0);
            lost |= x[k] == 0u;
            xv = __builtin_bit_cast(float, x[k] - 1u);
            store_slot(&part[(int64_t)g * p.width + b], 0u);
          }
          if (counter) {
            c[k] = landed(&counts[g], c[k], p.spin_limit, p.lose != 0);
            lost_count |= c[k] == 0u;
            total += (int)c[k] - 1;
            store_slot(&counts[g], 0u);
          }
        }
        acc = use_max ? fmaxf(acc, xv) : acc + xv;
      }
    }
    if (counter) s_count[0] = lost_count ? -1 : total;
    // a lost slot's value may land after this call: the sticky status keeps later calls off the
    // workspace until ekv_tile_shares_reset clears it
    if (lost || (counter && lost_count))
      __hip_atomic_store(p.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    count = s_count[0];
    v = lost ? NAN : acc;
    if (count < 0) {  // a count never landed: the row is left without evidence
      if (b < p.width) p.shares[(int64_t)out_row * p.shares_stride + b] = NAN;
      return;
    }
  }
  // the whole-row rules: NaN without evidence, the mean over contributing pairs, or the max
  // renormalised over the row
  float *out = p.shares + (int64_t)out_row * p.shares_stride;
  if (count == 0) {
    if (b < p.width) out[b] = NAN;
    return;
  }
  if (use_max) {
    const float total = block_sum<NT>(v, s_red);
    if (b < p.width) out[b] = total > 0.0f ? v / total : 0.0f;
  } else if (b < p.width) {
    out[b] = v / (float)count;
  }
}

// The split form's second kernel: one workgroup per row combines the row's K partials in group
// order, then applies the whole-row rules (NaN without evidence, the mean over contributing
// pairs, or the max renormalised over the row).
__global__ __launch_bounds__(kSplitThreads) void combine_kernel(const Params p) {
  constexpr int NT = kSplitThreads;
  __shared__ float s_red[NT / kWave];
  const int row = blockIdx.x;
  const int K = p.groups;
  float *part = p.part + (int64_t)row * K * p.width;
  float *out = p.shares + (int64_t)row * p.shares_stride;
  int contributors = 0;
  for (int g0 = 0; g0 < K; g0 += kBatch) {  // kBatch counts in flight
    int c[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) c[k] = g0 + k < K ? p.part_count[(int64_t)row * K + g0 + k] : 0;
#pragma unroll
    for (int k = 0; k < kBatch; ++k) contributors += c[k];
  }
  __syncthreads();  // every thread has read the counts: they are cleared for the next call
  for (int g = threadIdx.x; g < K; g += NT) p.part_count[(int64_t)row * K + g] = 0;
  if (contributors == 0) {  // no evidence about the row, tile_shares.py:103
    for (int b = threadIdx.x; b < p.width; b += NT) {
      out[b] = NAN;
      for (int g = 0; g < K; ++g) part[(int64_t)g * p.width + b] = 0.0f;
    }
    return;
  }
  const bool use_max = p.aggregate == EKV_AGG_MAX;
  float local_total = 0.0f;
  for (int b = threadIdx.x; b < p.width; b += NT) {
    float v = 0.0f;
    for (int g0 = 0; g0 < K; g0 += kBatch) {  // kBatch partials in flight, added in group order
      float x[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) x[k] = g0 + k < K ? part[(int64_t)(g0 + k) * p.width + b] : 0.0f;
#pragma unroll
      for (int k = 0; k < kBatch; ++k) v = use_max ? fmaxf(v, x[k]) : v + x[k];
#pragma unroll
      for (int k = 0; k < kBatch; ++k)
        if (g0 + k < K) part[(int64_t)(g0 + k) * p.width + b] = 0.0f;  // cleared for the next call
    }
    local_total += v;
    out[b] = use_max ? v : v / (float)contributors;
  }
  if (use_max) {  // renormalise the per-block max, tile_shares.py:97-100
    const float total = block_sum<NT>(local_total, s_red);
    for (int b = threadIdx.x; b < p.width; b += NT) out[b] = total > 0.0f ? out[b] / total : 0.0f;
  }
}

// The split form's groups per row: enough (row, group) workgroups to cover the GPU about twice,
// at most one per layer.
int split_groups(int nrows, int layers) {
  if (nrows < 1) return 1;
  const int want = (2 * cu_count() + nrows - 1) / nrows;
  return std::max(1, std::min(want, layers));
}

// The workspace: the wave form's arrival counters for up to kMaxArrivalRows rows (zero before the
// first call, and every call leaves them zero), then the partials and their counts, sized for one
// group per layer, the most any split form takes.  The counters sit at the same place whatever the
// call's shape, and no call writes partials over them.
size_t split_workspace(int nrows, int width, int layers) {
  const size_t parts = (size_t)nrows * layers * width * sizeof(float);
  return kHeaderBytes + kArrivalBytes + ((parts + 255) / 256) * 256 + (size_t)nrows * layers * sizeof(int32_t);
}

// The wave form's wait for a slot, for every call in the process: the reloads before a slot is
// taken as lost, and (tests of the failure path only) whether every wait is made to run to it.
int g_spin_limit = kSpinLimit;
int g_lose = 0;

// the register form's layers per group for J blocks per thread (at most 12 quads of each plane)
constexpr int reg_layers(int J) { return J == 1 ? 8 : (J == 4 ? 2 : 4); }

// workspace null: one workgroup per row; otherwise the split form (workspace_bytes at least
// split_workspace(nrows, width, layers))
int launch(Params p, int nrows, void *workspace, size_t workspace_bytes, void *stream) {
  if (p.cells < 1 || p.cells > kMaxCells)
    return fail(EKV_EUNSUPPORTED, "tile shares: %d cells per block (at most %d)", p.cells, kMaxCells);
  if (p.layers < 1 || p.width < 1 || p.tile_blocks < 1 || nrows < 0)
    return fail(EKV_EINVAL, "tile shares: layers %d, width %d, tile_blocks %d, rows %d", p.layers, p.width,
                p.tile_blocks, nrows);
  if (p.aggregate != EKV_AGG_MEAN && p.aggregate != EKV_AGG_MAX)
    return fail(EKV_EINVAL, "tile shares: unknown aggregate %d", p.aggregate);
  if ((int64_t)p.width * kMaxCells > INT_MAX)
    return fail(EKV_EUNSUPPORTED, "tile shares: width %d too large", p.width);
  int cp = 1;
  while (cp < p.cells) cp <<= 1;
  p.cells_pow2 = cp;
  if ((int64_t)p.layers * cp > kMaxStats)
    return fail(EKV_EUNSUPPORTED, "tile shares: %d layers x %d cells exceed the %d statistics kept per row",
                p.layers, cp, kMaxStats);
  if (workspace != nullptr && workspace_bytes < split_workspace(nrows, p.width, p.layers))
    return fail(EKV_EINVAL, "tile shares: workspace of %zu bytes, %zu needed", workspace_bytes,
                split_workspace(nrows, p.width, p.layers));
  if (nrows == 0) return EKV_OK;
  const bool split = workspace != nullptr;
  const int NT = split ? kSplitThreads : kThreads;
  p.groups = split ? split_groups(nrows, p.layers) : 1;
  const int group_layers = (p.layers + p.groups - 1) / p.groups;  // the largest group
  if (split) {
    const size_t parts = (size_t)nrows * p.groups * p.width * sizeof(float);
    p.status = (int32_t *)workspace;
    p.spin_limit = g_spin_limit;
    p.lose = g_lose;
    p.arrivals = (int32_t *)((char *)workspace + kHeaderBytes);
    p.part = (float *)((char *)workspace + kHeaderBytes + kArrivalBytes);
    p.part_count = (int32_t *)((char *)p.part + ((parts + 255) / 256) * 256);
  }
  const size_t lds = (size_t)2 * group_layers * cp * sizeof(float);
  const bool aligned = ((uintptr_t)p.m % 16) == 0 && (p.from_u || ((uintptr_t)p.l % 16) == 0) &&
                       p.layer_stride % 4 == 0 && p.row_stride % 4 == 0;
  const bool vec = aligned && p.cells % 4 == 0 && cp == p.cells;  // cells / 4 a power of two
  // the peak pass: as many lanes per layer as the workgroup has per layer, a power of two from the
  // quads per block to a wave
  int lpl = kWave;
  while (lpl > 1 && lpl * group_layers > NT) lpl >>= 1;
  p.lanes_per_layer = std::max(lpl, std::max(cp / 4, 1));
  hipStream_t s = (hipStream_t)stream;
  if (split && vec && !p.from_u && p.cells == 4 && p.width <= kWaveLayers * kWave && nrows <= kMaxArrivalRows) {
    // the wave form: one layer per wave, 8 waves a workgroup up to 8 layers, else 16 (fewer layer
    // groups to combine: none up to 16 layers); the row's last workgroup combines
    const int nw = p.layers <= kWaveLayers ? kWaveLayers : 2 * kWaveLayers;
    p.groups = (p.layers + nw - 1) / nw;
    const size_t parts = (size_t)nrows * p.groups * p.width * sizeof(float);
    p.part_count = (int32_t *)((char *)p.part + ((parts + 255) / 256) * 256);
    const unsigned grid = (unsigned)nrows * (unsigned)p.groups;
    const dim3 block(nw * kWave);
    auto launch = [&](auto nw_tag) {
      constexpr int NW = decltype(nw_tag)::value;
      if (p.width <= kWave) hipLaunchKernelGGL((shares_wave_kernel<1, NW>), dim3(grid), block, 0, s, p);
      else if (p.width <= 2 * kWave) hipLaunchKernelGGL((shares_wave_kernel<2, NW>), dim3(grid), block, 0, s, p);
      else if (p.width <= 4 * kWave) hipLaunchKernelGGL((shares_wave_kernel<4, NW>), dim3(grid), block, 0, s, p);
      else hipLaunchKernelGGL((shares_wave_kernel<8, NW>), dim3(grid), block, 0, s, p);
    };
    if (nw == kWaveLayers) launch(std::integral_constant<int, kWaveLayers>());
    else launch(std::integral_constant<int, 2 * kWaveLayers>());
    return check_hip(hipGetLastError(), "tile shares launch");
  }
  if (split && vec && p.cells == 4 && p.width <= 4 * kSplitThreads) {
    // the register form: one pass, J blocks per thread, reg_layers(J) layers per group
    const int J = (p.width + kSplitThreads - 1) / kSplitThreads;
    const int NLg = reg_layers(J);
    p.groups = (p.layers + NLg - 1) / NLg;
    const size_t parts = (size_t)nrows * p.groups * p.width * sizeof(float);
    p.part_count = (int32_t *)((char *)p.part + ((parts + 255) / 256) * 256);
    const unsigned grid = (unsigned)nrows * (unsigned)p.groups;
    switch (J) {
      case 1: hipLaunchKernelGGL((shares_reg_kernel<1, reg_layers(1)>), dim3(grid), dim3(kSplitThreads), 0, s, p); break;
      case 2: hipLaunchKernelGGL((shares_reg_kernel<2, reg_layers(2)>), dim3(grid), dim3(kSplitThreads), 0, s, p); break;
      case 3: hipLaunchKernelGGL((shares_reg_kernel<3, reg_layers(3)>), dim3(grid), dim3(kSplitThreads), 0, s, p); break;
      default: hipLaunchKernelGGL((shares_reg_kernel<4, reg_layers(4)>), dim3(grid), dim3(kSplitThreads), 0, s, p); break;
    }
    const int rc = check_hip(hipGetLastError(), "tile shares launch");
    if (rc != EKV_OK) return rc;
    hipLaunchKernelGGL(combine_kernel, dim3(nrows), dim3(kSplitThreads), 0, s, p);
    return check_hip(hipGetLastError(), "tile shares combine launch");
  }
  if (!split) {
    if (vec) hipLaunchKernelGGL((shares_kernel<true, kThreads, false>), dim3(nrows), dim3(NT), lds, s, p);
    else hipLaunchKernelGGL((shares_kernel<false, kThreads, false>), dim3(nrows), dim3(NT), lds, s, p);
    return check_hip(hipGetLastError(), "tile shares launch");
  }
  const unsigned grid = (unsigned)nrows * (unsigned)p.groups;
  if (vec) hipLaunchKernelGGL((shares_kernel<true, kSplitThreads, true>), dim3(grid), dim3(NT), lds, s, p);
  else hipLaunchKernelGGL((shares_kernel<false, kSplitThreads, true>), dim3(grid), dim3(NT), lds, s, p);
  const int rc = check_hip(hipGetLastError(), "tile shares launch");
  if (rc != EKV_OK) return rc;
  hipLaunchKernelGGL(combine_kernel, dim3(nrows), dim3(kSplitThreads), 0, s, p);
  return check_hip(hipGetLastError(), "tile shares combine launch");
}

}  // namespace shares
}  // namespace ekv

using namespace ekv;

extern "C" int ekv_tile_shares(const float *lse, int64_t lse_plane_stride, int64_t lse_layer_stride,
                               int64_t lse_row_stride, int32_t layers, int32_t cells, int32_t width,
                               const int32_t *row_ids, const int32_t *row_blocks, int32_t nrows,
                               int32_t tile_blocks, int32_t aggregate, float *shares, int64_t shares_stride,
                               void *stream) {
  if (lse == nullptr || shares == nullptr) return fail(EKV_EINVAL, "ekv_tile_shares: null pointer");
  shares::Params p{};
  p.m = lse;
  p.l = lse + lse_plane_stride;
  p.layer_stride = lse_layer_stride;
  p.row_stride = lse_row_stride;
  p.layers = layers;
  p.cells = cells;
  p.width = width;
  p.row_ids = row_ids;
  p.row_blocks = row_blocks;
  p.tile_blocks = tile_blocks;
  p.aggregate = aggregate;
  p.from_u = 0;
  p.shares = shares;
  p.shares_stride = shares_stride;
  return shares::launch(p, nrows, nullptr, 0, stream);
}

extern "C" size_t ekv_tile_shares_workspace(int32_t nrows, int32_t width, int32_t layers) {
  if (nrows < 0 || width < 1 || layers < 1) return 0;
  return shares::split_workspace(nrows, width, layers);
}

extern "C" int ekv_tile_shares_ws(const float *lse, int64_t lse_plane_stride, int64_t lse_layer_stride,
                                  int64_t lse_row_stride, int32_t layers, int32_t cells, int32_t width,
                                  const int32_t *row_ids, const int32_t *row_blocks, int32_t nrows,
                                  int32_t tile_blocks, int32_t aggregate, float *shares, int64_t shares_stride,
                                  void *workspace, size_t workspace_bytes, void *stream) {
  if (lse == nullptr || shares == nullptr || workspace == nullptr)
    return fail(EKV_EINVAL, "ekv_tile_shares_ws: null pointer");
  shares::Params p{};
  p.m = lse;
  p.l = lse + lse_plane_stride;
  p.layer_stride = lse_layer_stride;
  p.row_stride = lse_row_stride;
  p.layers = layers;
  p.cells = cells;
  p.width = width;
  p.row_ids = row_ids;
  p.row_blocks = row_blocks;
  p.tile_blocks = tile_blocks;
  p.aggregate = aggregate;
  p.from_u = 0;
  p.shares = shares;
  p.shares_stride = shares_stride;
  return shares::launch(p, nrows, workspace, workspace_bytes, stream);
}

namespace {

constexpr int kMaxScratchDevices = 64;
void *g_scratch_ptr[kMaxScratchDevices] = {nullptr};
std::mutex g_scratch_lock;

// The current device's copy of `scratch`, looked up once per device with that device current.
int device_scratch(void **out) {
  int device = -1;
  int rc = check_hip(hipGetDevice(&device), "hipGetDevice");
  if (rc != EKV_OK) return rc;
  if (device < 0 || device >= kMaxScratchDevices)
    return fail(EKV_EUNSUPPORTED, "ekv_tile_shares_noalloc: device %d (at most %d devices)", device,
                kMaxScratchDevices);
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch_ptr[device] == nullptr) {
    void *ptr = nullptr;
    rc = check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (rc != EKV_OK) return rc;
    if (ptr == nullptr) return fail(EKV_ELAUNCH, "ekv_tile_shares_noalloc: no device address for the scratch");
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return EKV_OK;
}

}  // namespace

extern "C" int ekv_tile_shares_noalloc(const float *lse, int64_t lse_plane_stride, int64_t lse_layer_stride,
                                       int64_t lse_row_stride, int32_t layers, int32_t cells, int32_t width,
                                       const int32_t *row_ids, const int32_t *row_blocks, int32_t nrows,
                                       int32_t tile_blocks, int32_t aggregate, float *shares,
                                       int64_t shares_stride, void *stream) {
  if (lse == nullptr || shares == nullptr) return fail(EKV_EINVAL, "ekv_tile_shares_noalloc: null pointer");
  if (nrows < 0 || width < 1 || layers < 1)
    return fail(EKV_EINVAL, "ekv_tile_shares_noalloc: rows %d, width %d, layers %d", nrows, width, layers);
  const size_t need = shares::split_workspace(nrows, width, layers);
  if (need > (size_t)EKV_TILE_SHARES_SCRATCH_BYTES)
    return fail(EKV_EINVAL,
                "ekv_tile_shares_noalloc: %d rows x %d blocks x %d layers need %zu bytes of scratch, the "
                "library holds %zu per device (use ekv_tile_shares_ws with a workspace)",
                nrows, width, layers, need, (size_t)EKV_TILE_SHARES_SCRATCH_BYTES);
  void *ws = nullptr;
  const int rc = device_scratch(&ws);
  if (rc != EKV_OK) return rc;
  shares::Params p{};
  p.m = lse;
  p.l = lse + lse_plane_stride;
  p.layer_stride = lse_layer_stride;
  p.row_stride = lse_row_stride;
  p.layers = layers;
  p.cells = cells;
  p.width = width;
  p.row_ids = row_ids;
  p.row_blocks = row_blocks;
  p.tile_blocks = tile_blocks;
  p.aggregate = aggregate;
  p.from_u = 0;
  p.shares = shares;
  p.shares_stride = shares_stride;
  return shares::launch(p, nrows, ws, (size_t)EKV_TILE_SHARES_SCRATCH_BYTES, stream);
}

namespace ekv {
namespace shares {

// Zeroes a workspace (a kernel, not a memset, so that a captured graph can hold it).
__global__ __launch_bounds__(256) void clear_kernel(uint4 *ws, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
    ws[i] = make_uint4(0u, 0u, 0u, 0u);
}

}  // namespace shares
}  // namespace ekv

extern "C" int ekv_tile_shares_status(const void *workspace, int32_t *status) {
  if (status == nullptr) return fail(EKV_EINVAL, "ekv_tile_shares_status: null status");
  void *ws = const_cast<void *>(workspace);
  if (ws == nullptr) {
    const int rc = device_scratch(&ws);
    if (rc != EKV_OK) return rc;
  }
  int rc = check_hip(hipDeviceSynchronize(), "ekv_tile_shares_status synchronize");
  if (rc != EKV_OK) return rc;
  return check_hip(hipMemcpy(status, ws, sizeof(int32_t), hipMemcpyDeviceToHost), "ekv_tile_shares_status copy");
}

extern "C" int ekv_tile_shares_reset(void *workspace, size_t workspace_bytes, void *stream) {
  void *ws = workspace;
  size_t bytes = workspace_bytes;
  if (ws == nullptr) {
    const int rc = device_scratch(&ws);
    if (rc != EKV_OK) return rc;
    bytes = (size_t)EKV_TILE_SHARES_SCRATCH_BYTES;
  }
  if (((uintptr_t)ws & 15) != 0 || bytes % 16 != 0)
    return fail(EKV_EINVAL, "ekv_tile_shares_reset: the workspace must be 16-byte aligned and sized");
  const size_t n16 = bytes / 16;
  if (n16 == 0) return EKV_OK;
  const unsigned blocks = (unsigned)std::min<size_t>((n16 + 255) / 256, 4096);
  hipLaunchKernelGGL(shares::clear_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (uint4 *)ws, n16);
  return check_hip(hipGetLastError(), "ekv_tile_shares_reset launch");
}

extern "C" int ekv_tile_shares_test_wait(int32_t spin_limit, int32_t lose) {
  shares::g_spin_limit = spin_limit > 0 ? spin_limit : shares::kSpinLimit;
  shares::g_lose = lose != 0;
  return EKV_OK;
}

extern "C" int ekv_normalize_tile_lse(const float *u, int64_t u_layer_stride, int64_t u_row_stride,
                                      int32_t layers, int32_t cells, int32_t width, const int32_t *row_blocks,
                                      int32_t nrows, int32_t tile_blocks, int32_t aggregate, float *shares,
                                      int64_t shares_stride, void *stream) {
  if (u == nullptr || shares == nullptr) return fail(EKV_EINVAL, "ekv_normalize_tile_lse: null pointer");
  shares::Params p{};
  p.m = u;
  p.l = nullptr;
  p.layer_stride = u_layer_stride;
  p.row_stride = u_row_stride;
  p.layers = layers;
  p.cells = cells;
  p.width = width;
  p.row_ids = nullptr;
  p.row_blocks = row_blocks;
  p.tile_blocks = tile_blocks;
  p.aggregate = aggregate;
  p.from_u = 1;
  p.shares = shares;
  p.shares_stride = shares_stride;
  return shares::launch(p, nrows, nullptr, 0, stream);
}
