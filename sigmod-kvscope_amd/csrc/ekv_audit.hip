// The audit statistic: per (row, tile of 2 blocks, query row) the tile max m and the tile sum
// l = sum exp(s - m) of the scaled scores s = scale * <q, k> over the tile's keys.
// Semantics follow tile_lse_kernel, runtime/audit_kernel.py:34-109; the launch it replaces is
// RecordingPlane.launch, runtime/audit_kernel.py:224-265.
//
// Design (gfx950, wave64):
//  * Work list.  A unit is (row, run of `chunk_tiles` tiles, audited KV head).  Every workgroup
//    builds the per-row unit offsets in LDS from lens/select (a block scan over the rows), so
//    the launch needs no host-side knowledge of the lengths, no scratch memory and no second
//    kernel; it is identical on every step and can be captured in a graph.  Waves walk the
//    units grid-stride, so only live tiles are visited (the reference's grid is rows x width
//    tiles with early exits).
//  * Loads.  One token's key row of one head is `row_bytes` contiguous bytes; LPT lanes load
//    it with 16-byte loads, TPI = 64 / LPT tokens per wave instruction.  A chunk is NL such
//    instructions; chunks are double-buffered so one chunk's loads are in flight while the
//    previous one is reduced.
//  * Dots.  Each lane multiplies its 16-byte slice with the matching slice of the (padded)
//    query group kept in registers (v_dot2 for 16-bit / fp8->bf16 keys, FMA for fp32), then a
//    transpose reduction over the LPT lanes of a token leaves VF complete scores per lane,
//    head-major, so the per-head max / sum need log2(64/GP) butterfly steps.
//  * Timer.  With a cycles buffer each unit adds its s_memtime duration to cycles[row] with a
//    vector 64-bit atomic (the pass's per-row timer, mlir_pass/lib/eKVTimer.cpp:1348-1387).
#include <math.h>

#include "ekv_common.hpp"

namespace ekv {
namespace audit {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kTileBlocks = 2;  // TILE_BLOCKS, runtime/audit_kernel.py:31
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxRows = 16000;  // LDS holds one int per row (64 KB per workgroup)

enum Mode : int { kModeF32 = 0, kModeF16 = 1, kModeBF16 = 2, kModeFp8Bf16 = 3 };

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
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
  int32_t group_first, groups, group_rows, rows, width, block_size, chunk_tiles, nsub;
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

template <int MODE, int HEAD_DIM, int NL, int GP>
__global__ __launch_bounds__(kThreads) void tile_lse_kernel(const Params p) {
  using S = Shape<MODE, HEAD_DIM, NL, GP>;
  static_assert(S::kValid, "invalid audit shape");
  constexpr int LPT = S::kLPT, TPI = S::kTPI, VF = S::kVF, OW = S::kOW, CT = S::kCT;
  constexpr int LPH = S::kLPH, HPL = S::kHPL;

  extern __shared__ int s_off[];  // [rows + 1] unit offsets per row
  __shared__ int s_scan[kWaves];

  if (*p.flag == 0u) return;  // the audit flag, runtime/audit_kernel.py:64

  const int rows = p.rows;
  const int bs = p.block_size;
  const int tile_tokens = kTileBlocks * bs;
  const int chunk = p.chunk_tiles;

  // ---- per-row unit counts and their exclusive scan (every workgroup) -------------------
  const int per = (rows + kThreads - 1) / kThreads;
  const int r0 = threadIdx.x * per;
  const int r1 = min(r0 + per, rows);
  auto units_of = [&](int r) -> int {
    if (p.select[r] == 0) return 0;  // runtime/audit_kernel.py:65
    const int len = min(max(p.lens[r], 0), p.width * bs);
    const int tiles = (len + tile_tokens - 1) / tile_tokens;
    return (tiles + chunk - 1) / chunk;
  };
  int local = 0;
  for (int r = r0; r < r1; ++r) local += units_of(r);
  int total_units = 0;
  int base = block_exclusive_scan<kThreads>(local, s_scan, total_units);
  for (int r = r0; r < r1; ++r) {
    s_off[r] = base;
    base += units_of(r);
  }
  if (threadIdx.x == 0) s_off[rows] = total_units;
  __syncthreads();

  const int lane = lane_id();
  const int slot = lane / LPT;  // token slot of the load instruction
  const int j = lane % LPT;     // 16-byte column of the key row
  const int nwaves = gridDim.x * kWaves;
  const int nsub = p.nsub;
  const int G = p.group_rows;
  const int all_units = total_units * p.groups;

  // the wave index is uniform across the wave; say so, so that the unit, row and chunk
  // arithmetic and the block-table reads stay scalar
  const int wave_id = __builtin_amdgcn_readfirstlane(blockIdx.x * kWaves + threadIdx.x / kWave);
  for (int u = wave_id; u < all_units; u += nwaves) {
    const int h = u % p.groups;
    const int bu = u / p.groups;
    int lo = 0, hi = rows;  // largest row with s_off[row] <= bu
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (s_off[mid] <= bu) lo = mid; else hi = mid;
    }
    const int row = lo;
    const int unit_in_row = bu - s_off[row];
    const uint64_t t_start = __builtin_amdgcn_s_memtime();

    const int len = min(max(p.lens[row], 0), p.width * bs);
    const int nblocks = (len + bs - 1) / bs;
    const int tiles = (len + tile_tokens - 1) / tile_tokens;
    const int tile_begin = unit_in_row * chunk;
    const int tile_end = min(tile_begin + chunk, tiles);
    const int g = p.group_first + h;  // KV head
    const int32_t *trow = p.table + (int64_t)row * p.table_stride;

    // ---- the query group of this KV head: GP rows, zero past group_rows -----------------
    uint32_t qw[GP][OW];
    {
      const char *qbase = p.q + (int64_t)p.qrow[row] * p.q_stride_token +
                          (int64_t)g * G * p.q_stride_head + (int64_t)j * (OW * 4);
#pragma unroll
      for (int gg = 0; gg < GP; ++gg) {
#pragma unroll
        for (int v = 0; v < OW / 4; ++v) {
          u32x4 w = {0u, 0u, 0u, 0u};
          if (gg < G) w = *(const u32x4 *)(qbase + (int64_t)gg * p.q_stride_head + v * 16);
#pragma unroll
          for (int e = 0; e < 4; ++e) qw[gg][4 * v + e] = w[e];
        }
      }
    }

    // per-lane part of a key address; the per-chunk part below is uniform across the wave
    const int64_t lane_off = (int64_t)slot * p.k_stride_pos + (int64_t)g * p.k_stride_head + j * 16;
    float *cell_row = p.lse + (int64_t)row * p.row_stride + h * G;

    // running (m, l) of the tile for the heads this lane holds
    float m_run[HPL], l_run[HPL];
#pragma unroll
    for (int e = 0; e < HPL; ++e) { m_run[e] = -INFINITY; l_run[e] = 0.0f; }

    // Loads are not predicated: a token past the row's end still lies in a block the row owns
    // (or in its first block when the tile's second block does not exist), so every address is
    // inside the key cache; its score is masked to -inf in reduce_chunk.
    auto load_chunk = [&](u32x4 (&D)[NL], int z) {
      const int tile = z / nsub;
      const int c = z - tile * nsub;
      const int b0 = tile * kTileBlocks;
      const int id0 = trow[b0];
      const int id1 = (b0 + 1 < nblocks) ? trow[b0 + 1] : id0;
      const char *base0 = p.keys + (int64_t)id0 * p.k_stride_block + lane_off;
      const char *base1 = p.keys + (int64_t)id1 * p.k_stride_block + lane_off;
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        const bool second = (2 * (c * NL + i)) >= nsub * NL;
        const int upos = c * CT + i * TPI - (second ? bs : 0);  // position of slot 0 in its block
        D[i] = *(const u32x4 *)((second ? base1 : base0) + (int64_t)upos * p.k_stride_pos);
      }
    };

    auto reduce_chunk = [&](const u32x4 (&D)[NL], int z) {
      const int tile = z / nsub;
      const int c = z - tile * nsub;
      const int tok0 = tile * tile_tokens + c * CT;
      float acc[GP * NL];
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        uint32_t kw[OW];
        key_operand<MODE>(D[i], kw);
#pragma unroll
        for (int gg = 0; gg < GP; ++gg) acc[gg * NL + i] = dot_words<MODE, OW>(qw[gg], kw);
      }
      transpose_reduce<GP * NL, LPT>(acc, lane);
      // acc[k] is the score of head (j*VF + k) / NL, load (j*VF + k) % NL
      float s[VF];
#pragma unroll
      for (int k = 0; k < VF; ++k) {
        const int i = (j * VF + k) % NL;
        const int tok = tok0 + i * TPI + slot;
        s[k] = tok < len ? acc[k] * p.scale : -INFINITY;
      }
#pragma unroll
      for (int e = 0; e < HPL; ++e) {
        constexpr int kPer = VF / HPL;  // scores of one head in this lane
        float mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < kPer; ++k) mx = fmaxf(mx, s[e * kPer + k]);
        mx = head_max<LPH, LPT>(mx);
        float sum = 0.0f;
        if (mx != -INFINITY) {
#pragma unroll
          for (int k = 0; k < kPer; ++k) sum += exp2f((s[e * kPer + k] - mx) * kLog2e);
        }
        sum = head_sum<LPH, LPT>(sum);
        // merge the chunk into the tile's running value
        const float M = fmaxf(m_run[e], mx);
        if (M != -INFINITY) {
          const float a = m_run[e] == -INFINITY ? 0.0f : l_run[e] * exp2f((m_run[e] - M) * kLog2e);
          const float b = mx == -INFINITY ? 0.0f : sum * exp2f((mx - M) * kLog2e);
          l_run[e] = a + b;
          m_run[e] = M;
        }
      }
      if (c == nsub - 1) {
        // store the tile into each of its blocks that the row reaches, runtime/audit_kernel.py:97-109
        if (slot == 0 && (j % LPH) == 0) {
#pragma unroll
          for (int e = 0; e < HPL; ++e) {
            const int head = (j / LPH) * HPL + e;
            if (head < G) {
#pragma unroll
              for (int b = 0; b < kTileBlocks; ++b) {
                const int blk = tile * kTileBlocks + b;
                if (blk < nblocks) {
                  float *cell = cell_row + (int64_t)blk * p.cells + head;
                  cell[0] = m_run[e];
                  cell[p.plane_stride] = l_run[e];
                }
              }
            }
          }
        }
#pragma unroll
        for (int e = 0; e < HPL; ++e) { m_run[e] = -INFINITY; l_run[e] = 0.0f; }
      }
    };

    const int z_end = tile_end * nsub;
    int z = tile_begin * nsub;
    u32x4 A[NL], B[NL];
    load_chunk(A, z);
    while (true) {
      if (z + 1 < z_end) load_chunk(B, z + 1);
      reduce_chunk(A, z);
      if (++z >= z_end) break;
      if (z + 1 < z_end) load_chunk(A, z + 1);
      reduce_chunk(B, z);
      if (++z >= z_end) break;
    }

    if (p.cycles != nullptr && h == 0 && row < p.cycles_rows && lane == 0) {
      const uint64_t t_end = __builtin_amdgcn_s_memtime();
      atomicAdd((unsigned long long *)(p.cycles + row), (unsigned long long)(t_end - t_start));
    }
  }
}

using KernelFn = void (*)(const Params);

template <int MODE, int HD, int NL, int GP>
KernelFn kernel_if_valid() {
  if constexpr (Shape<MODE, HD, NL, GP>::kValid) return tile_lse_kernel<MODE, HD, NL, GP>;
  else return nullptr;
}

template <int MODE, int HD, int NL>
KernelFn pick_gp(int gp) {
  switch (gp) {
    case 4: return kernel_if_valid<MODE, HD, NL, 4>();
    case 8: return kernel_if_valid<MODE, HD, NL, 8>();
    case 16: return kernel_if_valid<MODE, HD, NL, 16>();
  }
  return nullptr;
}

template <int MODE, int HD>
KernelFn pick_nl(int nl, int gp) {
  switch (nl) {
    case 4: return pick_gp<MODE, HD, 4>(gp);
    case 8: return pick_gp<MODE, HD, 8>(gp);
  }
  return nullptr;
}

template <int MODE>
KernelFn pick_hd(int hd, int nl, int gp) {
  switch (hd) {
    case 64: return pick_nl<MODE, 64>(nl, gp);
    case 128: return pick_nl<MODE, 128>(nl, gp);
  }
  return nullptr;
}

KernelFn pick(int mode, int hd, int nl, int gp) {
  switch (mode) {
    case kModeF32: return pick_hd<kModeF32>(hd, nl, gp);
    case kModeF16: return pick_hd<kModeF16>(hd, nl, gp);
    case kModeBF16: return pick_hd<kModeBF16>(hd, nl, gp);
    case kModeFp8Bf16: return pick_hd<kModeFp8Bf16>(hd, nl, gp);
  }
  return nullptr;
}

int dtype_bytes(int dtype) {
  switch (dtype) {
    case EKV_F32: return 4;
    case EKV_F16: return 2;
    case EKV_BF16: return 2;
    case EKV_FP8_E4M3: return 1;
  }
  return 0;
}

}  // namespace audit
}  // namespace ekv

using namespace ekv;
using namespace ekv::audit;

extern "C" int ekv_audit_tile_lse(
    const void *q, int q_dtype, int64_t q_stride_token, int64_t q_stride_head, const void *keys,
    int kv_dtype, int64_t k_stride_block, int64_t k_stride_pos, int64_t k_stride_head, float k_scale,
    const int32_t *table, int64_t table_stride, const int32_t *lens, const int32_t *qrow,
    const uint8_t *select, const uint32_t *flag, float *lse, int64_t lse_plane_stride,
    int64_t lse_layer_stride, int64_t lse_row_stride, int32_t cells, uint64_t *cycles,
    int32_t cycles_rows, float scale, int32_t layer, int32_t group_first, int32_t groups,
    int32_t group_rows, int32_t rows, int32_t width, int32_t block_size, int32_t tile_blocks,
    int32_t head_dim, int32_t chunk_tiles, void *stream) {
  if (q == nullptr || keys == nullptr || table == nullptr || lens == nullptr || qrow == nullptr ||
      select == nullptr || flag == nullptr || lse == nullptr)
    return fail(EKV_EINVAL, "ekv_audit_tile_lse: null pointer argument");
  if (tile_blocks != kTileBlocks)
    return fail(EKV_EUNSUPPORTED, "ekv_audit_tile_lse: tiles of %d blocks; the kernel records tiles of %d",
                tile_blocks, kTileBlocks);
  if (rows < 0 || rows > kMaxRows || width <= 0 || block_size <= 0 || layer < 0)
    return fail(EKV_EINVAL, "ekv_audit_tile_lse: rows %d (max %d), width %d, block %d, layer %d out of range",
                rows, kMaxRows, width, block_size, layer);
  if (group_rows < 1 || group_rows > 16)
    return fail(EKV_EINVAL, "ekv_audit_tile_lse: %d query rows per KV head; at most 16 are recorded", group_rows);
  if (groups < 1 || group_first < 0 || cells < groups * group_rows)
    return fail(EKV_EINVAL, "ekv_audit_tile_lse: %d groups from %d need %d cells per block, the plane has %d",
                groups, group_first, groups * group_rows, cells);
  if (((kTileBlocks * block_size) & (kTileBlocks * block_size - 1)) != 0)
    return fail(EKV_EINVAL, "ekv_audit_tile_lse: a tile must hold a power of two of tokens");
  if (rows == 0) return EKV_OK;

  int mode;
  if (kv_dtype == EKV_F32 && q_dtype == EKV_F32) mode = kModeF32;
  else if (kv_dtype == EKV_F16 && q_dtype == EKV_F16) mode = kModeF16;
  else if (kv_dtype == EKV_BF16 && q_dtype == EKV_BF16) mode = kModeBF16;
  else if (kv_dtype == EKV_FP8_E4M3 && q_dtype == EKV_BF16) mode = kModeFp8Bf16;
  else
    return fail(EKV_EUNSUPPORTED, "ekv_audit_tile_lse: query dtype %d with key dtype %d is not supported",
                q_dtype, kv_dtype);
  const int kbytes = dtype_bytes(kv_dtype);
  const int qbytes = dtype_bytes(q_dtype);
  const int row_bytes = head_dim * kbytes;
  if (row_bytes < 16 || row_bytes > 1024 || (row_bytes & (row_bytes - 1)) != 0)
    return fail(EKV_EUNSUPPORTED, "ekv_audit_tile_lse: head_dim %d of dtype %d", head_dim, kv_dtype);
  const int lpt = row_bytes / 16;
  const int tpi = kWave / lpt;
  const int tile_tokens = kTileBlocks * block_size;
  // A chunk is NL load instructions of TPI tokens (8 KB of keys at NL = 8).  A load
  // instruction must sit inside one block, and a chunk inside one tile.
  if (block_size % tpi != 0)
    return fail(EKV_EUNSUPPORTED, "ekv_audit_tile_lse: block size %d is below the %d tokens of one load",
                block_size, tpi);
  const int nl = tile_tokens / tpi >= 8 ? 8 : tile_tokens / tpi;
  const int gp = group_rows <= 4 ? 4 : (group_rows <= 8 ? 8 : 16);
  KernelFn fn = pick(mode, head_dim, nl, gp);
  if (fn == nullptr)
    return fail(EKV_EUNSUPPORTED, "ekv_audit_tile_lse: no kernel for dtype %d, head_dim %d, %d loads, group %d",
                kv_dtype, head_dim, nl, gp);
  // 16-byte loads of key rows and query slices
  const uint64_t kaddr = (uint64_t)keys | (uint64_t)(k_stride_block * kbytes) |
                         (uint64_t)(k_stride_pos * kbytes) | (uint64_t)(k_stride_head * kbytes);
  const uint64_t qaddr = (uint64_t)q | (uint64_t)(q_stride_token * qbytes) | (uint64_t)(q_stride_head * qbytes);
  if ((kaddr & 15) != 0 || (qaddr & 15) != 0)
    return fail(EKV_EINVAL, "ekv_audit_tile_lse: key and query rows must be 16-byte aligned");

  Params p;
  p.q = (const char *)q;
  p.q_stride_token = q_stride_token * qbytes;
  p.q_stride_head = q_stride_head * qbytes;
  p.keys = (const char *)keys;
  p.k_stride_block = k_stride_block * kbytes;
  p.k_stride_pos = k_stride_pos * kbytes;
  p.k_stride_head = k_stride_head * kbytes;
  p.table = table;
  p.table_stride = table_stride;
  p.lens = lens;
  p.qrow = qrow;
  p.select = select;
  p.flag = flag;
  p.lse = lse + (int64_t)layer * lse_layer_stride;
  p.plane_stride = lse_plane_stride;
  p.row_stride = lse_row_stride;
  p.cells = cells;
  p.cycles = cycles;
  p.cycles_rows = cycles == nullptr ? 0 : cycles_rows;
  p.scale = scale * k_scale;
  p.group_first = group_first;
  p.groups = groups;
  p.group_rows = group_rows;
  p.rows = rows;
  p.width = width;
  p.block_size = block_size;
  p.chunk_tiles = chunk_tiles > 0 ? chunk_tiles : 4;
  p.nsub = tile_tokens / (nl * tpi);

  const int64_t max_tiles = (width + kTileBlocks - 1) / kTileBlocks;
  const int64_t max_units = (int64_t)rows * ((max_tiles + p.chunk_tiles - 1) / p.chunk_tiles) * groups;
  int64_t blocks = (max_units + kWaves - 1) / kWaves;
  const int64_t cap = (int64_t)cu_count() * 4;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  const size_t lds = (size_t)(rows + 1) * sizeof(int);
  hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(kThreads), lds, (hipStream_t)stream, p);
  return check_hip(hipGetLastError(), "ekv_audit_tile_lse launch");
}
