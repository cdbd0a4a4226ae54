// Exact per-block attention shares from the tile records, on the device.
// Semantics: read_tile_rows (observe/tile_shares.py:129-173) forms u = m + log(l) - log(T) from
// the two planes; normalize_tile_lse (observe/tile_shares.py:58-103) gives a partial last tile's
// blocks back log(T / valid_in_tail), drops cells past the row, turns every (layer, query row)
// with a finite value into a softmax over the row's blocks, and averages them (or takes the
// renormalised per-block max).  The reference copies the planes to the host and does this in
// float64 NumPy; here it runs in float32 on the planes where the audit kernel wrote them.
//
// One workgroup of 16 waves per output row.  Phase 1: wave w takes layers w, w + 16, ...; for
// each it streams the row's [width][cells] records (coalesced: consecutive lanes read
// consecutive cells, 8 elements' loads in flight per lane before any is used) and keeps an
// online (max, sum of exp) per lane, which a butterfly over the lanes of the same query row
// turns into the (layer, query row) peak and total, kept in LDS.  Phase 2: each thread owns
// blocks and sums their shares over layers and query rows in a fixed order (8 records loaded
// ahead), so the result is deterministic (no atomics).
#include <math.h>

#include "ekv_common.hpp"

namespace ekv {
namespace shares {

constexpr int kThreads = 1024;
constexpr int kBatch = 8;  // loads in flight per lane
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxCells = 64;
constexpr int kMaxStats = 8000;  // layers * padded cells: 2 floats each in LDS (64 KB)

struct Params {
  const float *m;  // plane 0 (or u when from_u)
  const float *l;  // plane 1 (unused when from_u)
  int64_t layer_stride, row_stride;
  int32_t layers, cells, cells_pow2, width;
  const int32_t *row_ids, *row_blocks;
  float log_tile;  // log(tile_blocks)
  int32_t tile_blocks, aggregate, from_u;
  float *shares;
  int64_t shares_stride;
};

__device__ __forceinline__ bool finite(float x) { return __builtin_isfinite(x); }

// log weight of block b of one record (m and l as loaded, or u itself when from_u), NaN when the
// record carries none.  n is the row's length in blocks, which may exceed the width: the tail
// rule uses it unclipped.
__device__ __forceinline__ float weight_of(const Params &p, float m, float l, int b, int n) {
  float u = p.from_u ? m : m + __logf(l) - p.log_tile;
  // a partial last tile gives its weight back to the blocks that exist, tile_shares.py:84-87
  const int T = p.tile_blocks;
  const int tail_start = (n / T) * T;
  if ((n % T) != 0 && b >= tail_start) u += __logf((float)T / (float)max(n - tail_start, 1));
  return u;
}

// merge two (max, sum exp(x - max)) pairs
__device__ __forceinline__ void merge(float &m, float &s, float m2, float s2) {
  const float M = fmaxf(m, m2);
  if (M == -INFINITY) return;
  const float a = m == -INFINITY ? 0.0f : s * __expf(m - M);
  const float b = m2 == -INFINITY ? 0.0f : s2 * __expf(m2 - M);
  m = M;
  s = a + b;
}

__global__ __launch_bounds__(kThreads) void shares_kernel(const Params p) {
  extern __shared__ float s_stats[];  // [layers][cells_pow2] peak, then [layers][cells_pow2] 1/total
  __shared__ float s_red[kWaves];
  __shared__ int s_contrib;

  const int out_row = blockIdx.x;
  const int src_row = p.row_ids != nullptr ? p.row_ids[out_row] : out_row;
  const int n_row = p.row_blocks != nullptr ? max(p.row_blocks[out_row], 0) : p.width;
  const int n = min(n_row, p.width);  // blocks with records
  const int CP = p.cells_pow2;
  const int cells = p.cells;
  float *peak = s_stats;
  float *inv_total = s_stats + p.layers * CP;
  if (threadIdx.x == 0) s_contrib = 0;
  __syncthreads();

  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int q = lane & (CP - 1);  // every element a lane visits has this query row (CP divides 64)
  const int64_t span = (int64_t)n * CP;

  // ---- phase 1: peak and total of every (layer, query row) ------------------------------
  int contrib = 0;
  for (int layer = wave; layer < p.layers; layer += kWaves) {
    const float *mrow = p.m + layer * p.layer_stride + (int64_t)src_row * p.row_stride;
    const float *lrow = p.from_u ? nullptr : p.l + layer * p.layer_stride + (int64_t)src_row * p.row_stride;
    float mx = -INFINITY, sum = 0.0f;
    if (q < cells) {
      for (int64_t e0 = lane; e0 < span; e0 += (int64_t)kWave * kBatch) {
        float mv[kBatch], lv[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          const int64_t e = e0 + (int64_t)k * kWave;
          const int64_t idx = e < span ? (e / CP) * cells + q : 0;
          mv[k] = mrow[idx];
          lv[k] = p.from_u ? 0.0f : lrow[idx];
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          const int64_t e = e0 + (int64_t)k * kWave;
          if (e >= span) break;
          const int b = (int)(e / CP);
          const float u = weight_of(p, mv[k], lv[k], b, n_row);
          if (finite(u)) {
            if (u > mx) {
              sum = sum * __expf(mx - u) + 1.0f;
              mx = u;
            } else {
              sum += __expf(u - mx);
            }
          }
        }
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
  contrib = wave_sum_int(contrib);
  if (lane == 0 && contrib) atomicAdd(&s_contrib, contrib);
  __syncthreads();
  const int contributors = s_contrib;

  float *out = p.shares + (int64_t)out_row * p.shares_stride;
  if (contributors == 0) {  // no evidence about the row, tile_shares.py:103
    for (int b = threadIdx.x; b < p.width; b += kThreads) out[b] = NAN;
    return;
  }

  // ---- phase 2: per-block shares, summed (or maxed) in a fixed order -----------------------
  const bool use_max = p.aggregate == EKV_AGG_MAX;
  float local_total = 0.0f;
  const int records = p.layers * cells;  // (layer, query row) pairs, in a fixed order
  for (int b = threadIdx.x; b < p.width; b += kThreads) {
    float acc = 0.0f;
    if (b < n) {
      for (int r0 = 0; r0 < records; r0 += kBatch) {
        float mv[kBatch], lv[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          const int rec = r0 + k < records ? r0 + k : 0;
          const int layer = rec / cells, c = rec - layer * cells;
          const int64_t at = layer * p.layer_stride + (int64_t)src_row * p.row_stride + (int64_t)b * cells + c;
          mv[k] = p.m[at];
          lv[k] = p.from_u ? 0.0f : p.l[at];
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          const int rec = r0 + k;
          if (rec >= records) break;
          const int layer = rec / cells, c = rec - layer * cells;
          const float pk = peak[layer * CP + c];
          if (!finite(pk)) continue;
          const float u = weight_of(p, mv[k], lv[k], b, n_row);
          const float share = finite(u) ? __expf(u - pk) * inv_total[layer * CP + c] : 0.0f;
          acc = use_max ? fmaxf(acc, share) : acc + share;
        }
      }
    }
    if (use_max) {
      local_total += acc;
      out[b] = acc;
    } else {
      out[b] = acc / (float)contributors;
    }
  }
  if (use_max) {
    const float total = block_sum<kThreads>(local_total, s_red);
    for (int b = threadIdx.x; b < p.width; b += kThreads) out[b] = total > 0.0f ? out[b] / total : 0.0f;
  }
}

int launch(Params p, int nrows, void *stream) {
  if (p.cells < 1 || p.cells > kMaxCells)
    return fail(EKV_EUNSUPPORTED, "tile shares: %d cells per block (at most %d)", p.cells, kMaxCells);
  if (p.layers < 1 || p.width < 1 || p.tile_blocks < 1 || nrows < 0)
    return fail(EKV_EINVAL, "tile shares: layers %d, width %d, tile_blocks %d, rows %d", p.layers, p.width,
                p.tile_blocks, nrows);
  if (p.aggregate != EKV_AGG_MEAN && p.aggregate != EKV_AGG_MAX)
    return fail(EKV_EINVAL, "tile shares: unknown aggregate %d", p.aggregate);
  int cp = 1;
  while (cp < p.cells) cp <<= 1;
  p.cells_pow2 = cp;
  if ((int64_t)p.layers * cp > kMaxStats)
    return fail(EKV_EUNSUPPORTED, "tile shares: %d layers x %d cells exceed the %d statistics kept per row",
                p.layers, cp, kMaxStats);
  p.log_tile = logf((float)p.tile_blocks);
  if (nrows == 0) return EKV_OK;
  const size_t lds = (size_t)2 * p.layers * cp * sizeof(float);
  hipLaunchKernelGGL(shares_kernel, dim3(nrows), dim3(kThreads), lds, (hipStream_t)stream, p);
  return check_hip(hipGetLastError(), "tile shares launch");
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
  return shares::launch(p, nrows, stream);
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
  return shares::launch(p, nrows, stream);
}
