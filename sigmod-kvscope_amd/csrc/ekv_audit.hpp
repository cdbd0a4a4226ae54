// Definitions the audit's translation units share: the kernel parameters, the step plan's tile
// descriptors and the layers of a launch, and the VALU dot-product helpers.
#pragma once

#include <math.h>

#include "ekv_common.hpp"

namespace ekv {
namespace audit {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kCuThreads = 768;  // tile_lse_cu_kernel: 12 waves, one workgroup per compute unit
constexpr int kTileBlocks = 2;  // TILE_BLOCKS, runtime/audit_kernel.py:31
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kMaxRows = 6000;  // LDS holds two ints per row beside the kernels' staging buffers
constexpr int kCycleSlots = 64;  // per-row cycle accumulators of a round in tile_lse_cu_kernel

enum Mode : int { kModeF32 = 0, kModeF16 = 1, kModeBF16 = 2, kModeFp8Bf16 = 3 };

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

struct Params {
  const char *q;
  int64_t q_stride_token, q_stride_head;  // bytes
  const char *keys;
  int64_t k_stride_block, k_stride_pos, k_stride_head;  // bytes
  const int32_t *table;
  int64_t table_stride;
  const int32_t *lens;
  const int32_t *qrow;
  const uint8_t *select;
  const uint32_t *flag;
  float *lse;  // already offset to the layer
  int64_t plane_stride, row_stride;
  int32_t cells;
  uint64_t *cycles;
  int32_t cycles_rows;
  float scale;  // scale * k_scale
  int32_t group_first, groups, group_rows, rows, width, block_size, chunk_tiles, nsub, nsub_log2;
};

template <int MODE, int HEAD_DIM, int NL, int GP>
struct Shape {
  static constexpr int kKBytes = MODE == kModeF32 ? 4 : (MODE == kModeFp8Bf16 ? 1 : 2);
  static constexpr int kQBytes = MODE == kModeF32 ? 4 : 2;
  static constexpr int kRowBytes = HEAD_DIM * kKBytes;
  static constexpr int kLPT = kRowBytes / 16;          // lanes per key row
  static constexpr int kTPI = kWave / kLPT;            // tokens per load instruction
  static constexpr int kEPL = 16 / kKBytes;            // key elements per lane per load
  static constexpr int kQW = kEPL * kQBytes / 4;       // query words per head per lane
  static constexpr int kOW = MODE == kModeFp8Bf16 ? 8 : 4;  // operand words per load
  static constexpr int kV = NL * GP;                   // partial dots per lane
  static constexpr int kVF = kV / kLPT;                // scores per lane after the reduction
  static constexpr int kCT = NL * kTPI;                // tokens per chunk
  // the shape is compiled only when a row is 16..1024 bytes and the transpose reduction
  // leaves at least one score per lane
  static constexpr bool kValid = kLPT >= 1 && kLPT <= kWave && (kLPT & (kLPT - 1)) == 0 && kV >= kLPT &&
                                 kQW == kOW;
  static constexpr int kLPH = !kValid ? 1 : (kVF <= NL ? NL / kVF : 1);  // lanes of a slot per head
  static constexpr int kHPL = !kValid ? 1 : (kVF <= NL ? 1 : kVF / NL);  // heads per lane
};

__device__ __forceinline__ float as_float(uint32_t w) { return __builtin_bit_cast(float, w); }

// Operand words of one 16-byte key load: the raw words, or fp8 pairs widened to bf16 pairs.
template <int MODE>
__device__ __forceinline__ void key_operand(const u32x4 k, uint32_t (&op)[MODE == kModeFp8Bf16 ? 8 : 4]) {
  if constexpr (MODE == kModeFp8Bf16) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int w = (int)k[e];
      op[2 * e] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
      op[2 * e + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) op[e] = k[e];
  }
}

template <int MODE, int OW>
__device__ __forceinline__ float dot_words(const uint32_t (&qw)[OW], const uint32_t (&kw)[OW]) {
  float acc = 0.0f;
  if constexpr (MODE == kModeF32) {
#pragma unroll
    for (int e = 0; e < OW; ++e) acc = fmaf(as_float(qw[e]), as_float(kw[e]), acc);
  } else if constexpr (MODE == kModeF16) {
#pragma unroll
    for (int e = 0; e < OW; ++e)
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, qw[e]), __builtin_bit_cast(f16x2_t, kw[e]),
                                   acc, false);
  } else {
#pragma unroll
    for (int e = 0; e < OW; ++e)
      acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, qw[e]),
                                            __builtin_bit_cast(bf16x2_t, kw[e]), acc, false);
  }
  return acc;
}

// Transpose reduction over the LPT lanes of a token slot: on entry lane j of a slot holds N
// partial sums a[0..N); on exit a[0..N/LPT) holds the complete sums of entries
// j*N/LPT .. j*N/LPT + N/LPT - 1.  Each step halves the live entries: the lane with the mask
// bit set keeps the upper half, its partner the lower half, and they swap the other halves.
template <int CUR, int MASK, int N>
__device__ __forceinline__ void transpose_reduce_step(float (&a)[N], int lane) {
  if constexpr (MASK >= 1) {
    constexpr int kHalf = CUR / 2;
    const bool upper = (lane & MASK) != 0;
#pragma unroll
    for (int k = 0; k < kHalf; ++k) {
      const float send = upper ? a[k] : a[k + kHalf];
      const float keep = upper ? a[k + kHalf] : a[k];
      a[k] = keep + shfl_xor(send, MASK);
    }
    transpose_reduce_step<kHalf, MASK / 2, N>(a, lane);
  }
}
template <int N, int LPT>
__device__ __forceinline__ void transpose_reduce(float (&a)[N], int lane) {
  transpose_reduce_step<N, LPT / 2, N>(a, lane);
}

// Max / sum over the lanes that hold the same head: the low bits of the slot lane within a
// head (LPH lanes) and every token slot (xor LPT .. 32).
template <int LPH, int LPT>
__device__ __forceinline__ float head_max(float v) {
#pragma unroll
  for (int m = 1; m < LPH; m <<= 1) v = fmaxf(v, shfl_xor(v, m));
#pragma unroll
  for (int m = LPT; m < kWave; m <<= 1) v = fmaxf(v, shfl_xor(v, m));
  return v;
}
template <int LPH, int LPT>
__device__ __forceinline__ float head_sum(float v) {
#pragma unroll
  for (int m = 1; m < LPH; m <<= 1) v += shfl_xor(v, m);
#pragma unroll
  for (int m = LPT; m < kWave; m <<= 1) v += shfl_xor(v, m);
  return v;
}

constexpr int kMaxGrid = 1024;  // the largest grid a plan splits its tiles over

struct TileDesc {
  int32_t row, k, valid, qtok, id0, id1, pad0, pad1;  // valid: tokens of the tile the row reaches
};
static_assert(sizeof(TileDesc) == 32, "a descriptor is 32 bytes, 16-byte aligned");

struct PlanView {
  const int4 *wg;  // per split: (tiles, first row, whole runs listed first, 0)
  const TileDesc *desc;
  int32_t cap;
};

// A descriptor into VGPRs with a vector load (the offset register keeps it one: a scalar load
// would be waited for with the wave's LDS traffic, both being counted by lgkmcnt).
// The descriptor's first 24 bytes (the padding is not read: a load into registers the kernel
// does not use still writes them, and the next write to such a register would wait for it)
__device__ __forceinline__ void load_desc(const TileDesc *d, u32x4 &lo, u32x2 &hi) {
  uint32_t o = 0;
  asm volatile("" : "+v"(o));
  const char *src = reinterpret_cast<const char *>(d) + o;
  lo = *as_global(reinterpret_cast<const u32x4 *>(src));
  hi = *as_global(reinterpret_cast<const u32x2 *>(src + 16));
}

// The tiles whose records share 128-byte lines: a tile records 2 blocks x `cells` floats in each
// plane, so 16 / cells consecutive tiles of a row fill a line.  A planned launch hands its waves runs
// of that many tiles times the audited heads (at most 8 items; a power of two of tiles, at most
// kPlanRun, since a plan's rows and splits fall on multiples of kPlanRun), so that one wave writes
// each line whole, at once.
constexpr int kPlanRun = 4;
__host__ __device__ inline int record_run_tiles(int cells, int groups) {
  int tiles = 1;
  while (tiles < kPlanRun && 2 * tiles * cells <= 16 && 2 * tiles * groups <= 8) tiles *= 2;
  return tiles;
}

// A plan pads each row's tiles to a multiple of kPlanRun (padding tiles have no tokens), so that the
// padded list's multiples of kPlanRun start runs of one row.  A split of `cnt` tiles from padded tile
// f lists its whole runs first, then the `head` tiles before its first multiple of kPlanRun, then the
// tail, so that a launch can hand out the runs as runs and the rest one tile at a time.
__host__ __device__ inline int plan_split_head(int f, int cnt) {
  const int h = (kPlanRun - f % kPlanRun) % kPlanRun;
  return h < cnt ? h : cnt;
}
__host__ __device__ inline int plan_split_runs(int f, int cnt) { return (cnt - plan_split_head(f, cnt)) / kPlanRun; }
// the place of the split's tile t (counted from f) in its list
__host__ __device__ inline int plan_split_pos(int t, int head, int runs) {
  const int whole = runs * kPlanRun;
  return t < head ? whole + t : (t < head + whole ? t - head : t);
}

// The records of a wave's current run (one row's consecutive tiles of one layer, record_run_tiles),
// held in registers until the run ends.  Records are ~1% of a launch's bytes but cost far more:
// under the streaming key reads, every record cache line that reaches memory costs about as much as
// several lines read, and a line stored in pieces by ordinary stores is no cheaper than one stored
// whole.  A whole, aligned line written with a non-temporal store costs least (at the Llama-3-8B
// decode shape the records took ~14% of the launch with a store per tile, ~10% as whole lines).
//
// Slot s holds the run's s-th item: in lane c * 16 + n, the tile max and sum of query n for the
// tile's block c, and the cell's offset in floats from the row's record base (-1 where the lane has
// no record).  When the run ends its records go out as whole lines if they are: the F records per
// plane (F a multiple of 32, at most 128) fill the F floats from the first one's cell, which is
// 128-byte aligned.  They then pass through the wave's LDS staging buffer into float order, and one
// non-temporal store per plane and 64 floats writes them, unless `hold` keeps them (the caller's
// store for lines written when the launch's reads are over).  Otherwise (a row's last run, which
// reaches past the row; a plane with more cells than the audited heads) each record is stored on its
// own.
template <int K>
struct RunRecords {
  float m[K], l[K];
  int off[K];
  int n;
  float *row;  // the record base of the run's row in its layer's max plane
  __device__ __forceinline__ void init() {
#pragma unroll
    for (int i = 0; i < K; ++i) off[i] = -1;
    n = 0;
  }
  // `stage`: 256 floats of the wave's LDS (its chunk staging buffer, free between the chunk's dots
  // and the next chunk's arrival)
  // hold(F, line, stage): true if it keeps the F floats per plane from `line` (stage[f] the max plane's
  // float f, stage[128 + f] the sum plane's)
  template <class Hold>
  __device__ __forceinline__ void flush(int64_t plane, float *stage, Hold &&hold) {
    const int lane = lane_id();
    const int off0 = __builtin_amdgcn_readlane(off[0], 0);  // slot 0, block 0, query 0
    int F = 0;  // the records held (their cells are distinct: each is one block, head and query)
#pragma unroll
    for (int i = 0; i < K; ++i) F += __builtin_popcountll(__builtin_amdgcn_ballot_w64(off[i] >= 0));
    // F distinct cells inside [off0, off0 + F) fill it
    bool inside = true;
#pragma unroll
    for (int i = 0; i < K; ++i)
      if (off[i] >= 0 && (off[i] < off0 || off[i] - off0 >= F)) inside = false;
    const bool lines = off0 >= 0 && F % 32 == 0 && F <= 128 && ((uintptr_t)(row + off0) & 127) == 0 &&
                       __builtin_amdgcn_ballot_w64(!inside) == 0;
    if (lines) {
#pragma unroll
      for (int i = 0; i < K; ++i)
        if (off[i] >= 0) {
          stage[off[i] - off0] = m[i];
          stage[128 + off[i] - off0] = l[i];
        }
      if (!hold(F, row + off0, stage)) {
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int f = lane + 64 * half;
          if (f < F) {
            __builtin_nontemporal_store(stage[f], as_global(row + off0 + f));
            __builtin_nontemporal_store(stage[128 + f], as_global(row + plane + off0 + f));
          }
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < K; ++i)
        if (off[i] >= 0) {
          as_global(row)[off[i]] = m[i];
          as_global(row)[off[i] + plane] = l[i];
        }
    }
    init();
  }
  // the item's records; the batch is stored first if it holds another row's (a run taken where the
  // plan has no whole runs can cross rows and layers), and after it when it holds K items (a run of
  // more than K items: more than 8 audited heads)
  template <class Hold>
  __device__ __forceinline__ void push(float *row_base, int cell_off, float mv, float lv, int64_t plane,
                                       float *stage, Hold &&hold) {
    if (n > 0 && row_base != row) flush(plane, stage, hold);
    row = row_base;
#pragma unroll
    for (int i = 0; i < K; ++i)
      if (i == n) {
        m[i] = mv;
        l[i] = lv;
        off[i] = cell_off;
      }
    if (++n == K) flush(plane, stage, hold);
  }
};

// The layers of one planned launch.  A decode step's audit launches differ only in the layer:
// its queries, its key cache, its records and its scale.  One launch can take up to
// kMaxLaunchLayers of them, so the launch's fixed costs (the first key requests, the spread of the
// workgroups' ends) are paid once for all of them.
constexpr int kMaxLaunchLayers = 32;

struct LayerArgs {
  const char *q;         // the layer's queries
  const char *keys;      // the layer's key cache
  float *lse;            // the statistic planes, offset to the layer
  float scale2;          // scale * k_scale * log2(e): scores in log2 units
  int32_t group_first;   // the first audited KV head
  int32_t q_head0;       // the query head that q's head 0 holds (a staged copy starts at the group)
  float scale;           // scale * k_scale (the VALU form scores in natural units)
};
static_assert(sizeof(LayerArgs) == 40, "packed layer arguments");

struct LayerSet {
  LayerArgs l[kMaxLaunchLayers];
  int32_t n;         // layers in the launch
  int32_t q_by_row;  // queries indexed by row (a staged copy), not by the row's query token
};

// The grid of a planned launch and of the plan it reads: one workgroup per compute unit.
int plan_grid();

// The VALU form of the planned launch (ekv_audit_valu.hip): whether it has a kernel for the shape,
// its chunks per tile, and one launch of the layers `ls` on the plan's grid.
bool valu_planned_shape(int mode, int head_dim, int block_size);
int valu_planned_nsub(int mode, int head_dim, int block_size, int group_rows);
int launch_valu_layers(int mode, int head_dim, int block_size, int group_rows, const Params &p, const PlanView &plan,
                       const LayerSet &ls, int grid, hipStream_t stream, const char *what);

}  // namespace audit
}  // namespace ekv
