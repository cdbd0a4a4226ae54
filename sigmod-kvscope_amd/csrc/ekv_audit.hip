// The audit statistic: per (row, tile of 2 blocks, query row) the tile max m and the tile sum
// l = sum exp(s - m) of the scaled scores s = scale * <q, k> over the tile's keys.
// Semantics follow tile_lse_kernel, runtime/audit_kernel.py:34-109; the launch it replaces is
// RecordingPlane.launch, runtime/audit_kernel.py:224-265.
//
// Design (gfx950, wave64):
//  * Work list.  The live tiles of the selected rows, times the audited KV heads, form one
//    flat list.  A self-contained launch has every workgroup build the per-row tile offsets in
//    LDS from lens/select with a block scan, so it needs no host-side knowledge of the lengths,
//    no scratch memory and no second kernel; a planned launch reads the list from a step plan
//    built once per decode step (below).  Both are identical on every step and can be captured
//    in a graph.
//  * Two kernels.  16-bit and fp8 keys (d = 64, 128, 256) in blocks of at least 16 tokens take
//    tile_lse_cu_kernel: one 12-wave workgroup per compute unit, an equal slice of the list
//    per CU, and the CU's waves share the slice through an LDS counter (a CU serves its loads
//    about in issue order, so equal per-wave slices leave the last-issued waves finishing last).
//    fp32 keys and blocks under 16 tokens take tile_lse_kernel on the VALU.
//  * Loads.  A load instruction reads whole key rows (16-byte lanes), the coalesced form that
//    DRAM serves at the streaming rate whatever the head's offset in the token.
//  * Dots.  The MFMA kernel computes S^T = K Q^T on v_mfma_f32_16x16x32_{bf16,f16} after an LDS
//    pass that turns whole-row loads into token-per-lane operands; the VALU kernel multiplies
//    each lane's slice with the query slice (v_dot2 / FMA) and reduces over the lanes of a row.
//  * Timer.  With a cycles buffer each wave adds its s_memtime durations to cycles[row] with a
//    vector 64-bit atomic (the pass's per-row timer, mlir_pass/lib/eKVTimer.cpp:1348-1387).
#include <math.h>

#include <algorithm>
#include <mutex>

#include "ekv_audit.hpp"

namespace ekv {
namespace audit {


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

  // ---- per-row live tile counts and their exclusive scan (every workgroup) -------------
  const int per = (rows + kThreads - 1) / kThreads;
  const int r0 = threadIdx.x * per;
  const int r1 = min(r0 + per, rows);
  auto tiles_of = [&](int r) -> int {
    if (p.select[r] == 0) return 0;  // runtime/audit_kernel.py:65
    const int len = min(max(p.lens[r], 0), p.width * bs);
    return (len + tile_tokens - 1) / tile_tokens;
  };
  int local = 0;
  for (int r = r0; r < r1; ++r) local += tiles_of(r);
  int total_tiles = 0;
  int base = block_exclusive_scan<kThreads>(local, s_scan, total_tiles);
  for (int r = r0; r < r1; ++r) {
    s_off[r] = base;
    base += tiles_of(r);
  }
  if (threadIdx.x == 0) s_off[rows] = total_tiles;
  __syncthreads();

  const int lane = lane_id();
  const int slot = lane / LPT;  // token slot of the load instruction
  const int j = lane % LPT;     // 16-byte column of the key row
  const int nwaves = gridDim.x * kWaves;
  const int nsub = p.nsub;
  const int G = p.group_rows;
  // the wave index is uniform across the wave; say so, so that the slice, row and tile
  // arithmetic and the block-table reads stay scalar
  const int wave_id = __builtin_amdgcn_readfirstlane(blockIdx.x * kWaves + threadIdx.x / kWave);
  const long long all = (long long)total_tiles * p.groups;
  long long u = all * wave_id / nwaves;
  const long long u_end = all * (wave_id + 1) / nwaves;

  while (u < u_end) {
    const int h = (int)(u / total_tiles);
    const int t = (int)(u - (long long)h * total_tiles);
    int lo = 0, hi = rows;  // the row holding flat tile t: largest row with s_off[row] <= t
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (s_off[mid] <= t) lo = mid; else hi = mid;
    }
    const int row = lo;
    const long long seg_end = min(u_end, (long long)(h + 1) * total_tiles);  // this head's part
    const int t_stop = (int)min((long long)s_off[row + 1], seg_end - (long long)h * total_tiles);
    const int tile_begin = t - s_off[row];
    const int tile_end = t_stop - s_off[row];
    u += t_stop - t;
    const uint64_t t_start = __builtin_amdgcn_s_memtime();

    const int len = min(max(p.lens[row], 0), p.width * bs);
    const int nblocks = (len + bs - 1) / bs;
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

    // Block ids come from a register holding one id per lane for a window of 64 blocks (read
    // with readlane), so the pipelined loop issues no table load whose wait would drain the key
    // loads in flight.  Loads are not predicated: a token past the row's end still lies in a
    // block the row owns (or in its first block when the tile's second block does not exist),
    // so every address is inside the key cache; its score is masked to -inf in reduce_chunk.
    int ids = 0, ids_base = 0;
    auto load_chunk = [&](u32x4 (&D)[NL], int z) {
      const int tile = z / nsub;
      const int c = z - tile * nsub;
      const int b0 = tile * kTileBlocks;
      const int id0 = __builtin_amdgcn_readlane(ids, b0 - ids_base);
      const int id1 = (b0 + 1 < nblocks) ? __builtin_amdgcn_readlane(ids, b0 + 1 - ids_base) : id0;
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

    // Windows of 32 tiles (the 64 block ids one register holds); inside a window two chunks are
    // in flight: the loop always prefetches and the tail drains.
    constexpr int kWindowTiles = kWave / kTileBlocks;
    for (int w0 = tile_begin; w0 < tile_end; w0 += kWindowTiles) {
      const int w1 = min(w0 + kWindowTiles, tile_end);
      ids_base = w0 * kTileBlocks;
      ids = ids_base + lane < nblocks ? trow[ids_base + lane] : 0;
      const int z_end = w1 * nsub;
      int z = w0 * nsub;
      u32x4 A[NL], B[NL];
      load_chunk(A, z);
      while (z + 2 < z_end) {
        load_chunk(B, z + 1);
        reduce_chunk(A, z);
        load_chunk(A, z + 2);
        reduce_chunk(B, z + 1);
        z += 2;
      }
      if (z + 1 < z_end) {
        load_chunk(B, z + 1);
        reduce_chunk(A, z);
        reduce_chunk(B, z + 1);
      } else {
        reduce_chunk(A, z);
      }
    }

    if (p.cycles != nullptr && h == 0 && row < p.cycles_rows && lane == 0) {
      const uint64_t t_end = __builtin_amdgcn_s_memtime();
      atomicAdd((unsigned long long *)(p.cycles + row), (unsigned long long)(t_end - t_start));
    }
  }
}

// ---------------------------------------------------------------------------------------
// MFMA form for 16-bit keys (and fp8 keys widened to bf16): S^T = K * Q^T on
// v_mfma_f32_16x16x32_{bf16,f16}.  A = keys (M = 16 tokens of one block, K = 32 dims),
// B = the query group (N = 16 query rows, zero past group_rows), C = scores.  Lane l holds
// A[token l % 16][dims of piece l / 16] and B[dims of piece l / 16][query row l % 16]; the 16-byte
// dim pieces are permuted identically in A and B (piece 4s + l / 16 feeds k-step s), and the
// keys reach that token-per-lane layout through LDS from whole-row loads.  C gives lane l the
// scores of tokens 4 (l / 16) + i of query row l % 16, so a query row's max / sum over a chunk
// is a local reduction of 4 values per M-tile and two swaps across the wave's 16-lane rows.
// ---------------------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <int MODE, int HEAD_DIM>
struct MfmaShape {
  static constexpr bool kFp8 = MODE == kModeFp8Bf16;
  static constexpr int kKBytes = kFp8 ? 1 : 2;
  static constexpr int kSteps = HEAD_DIM / 32;                   // k-steps of 32 dims
  static constexpr int kLoads = kFp8 ? kSteps / 2 : kSteps;      // 16-byte key loads per M-tile
  static constexpr int kRowBytes = HEAD_DIM * kKBytes;           // one token's key row of one head
  static constexpr int kPieces = kRowBytes / 16;                 // 16-byte pieces of a row
  static constexpr int kTPI = kWave / kPieces;                   // whole rows per load instruction
  static constexpr int kSwzDiv = kPieces >= 16 ? 1 : 16 / kPieces;
  static constexpr int kSwzMask = (kPieces >= 16 ? 16 : kPieces) - 1;
  static_assert(kTPI * kLoads == 16, "an M-tile is kLoads instructions of whole rows");
};

// LDS slot of piece pc of M-tile row t: the pieces of a row are permuted so that the 16 rows
// an MFMA operand read takes at one piece index fall in 16 different 16-byte bank columns
template <class S>
__device__ __forceinline__ int tr_slot(int t, int pc) {
  return t * S::kPieces + (pc ^ ((t / S::kSwzDiv) & S::kSwzMask));
}

template <int MODE>
__device__ __forceinline__ f32x4_t mfma_step(const u32x4 a, const u32x4 b, f32x4_t c) {
  if constexpr (MODE == kModeF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}

// 16 fp8 values (one 16-byte load) -> two bf16x8 operands (dims 0..7 and 8..15 of the piece)
__device__ __forceinline__ void widen_fp8(const u32x4 k, u32x4 &lo, u32x4 &hi) {
  uint32_t w[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    w[2 * e] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)k[e], 1.0f, false));
    w[2 * e + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)k[e], 1.0f, true));
  }
  lo = (u32x4){w[0], w[1], w[2], w[3]};
  hi = (u32x4){w[4], w[5], w[6], w[7]};
}

// ---------------------------------------------------------------------------------------
// The MFMA kernel: one workgroup per compute unit.
//
// A compute unit serves its waves' loads roughly in the order they were issued, so with equal
// static slices the waves that issued last receive their data last and finish last: at the
// Llama-3-8B shape the third workgroup on a CU gets its first chunk ~12 us after the first one
// and the launch ends on those waves alone.  Here the CU's waves share its slice instead: the
// slice is cut into rounds of one tile per thread, every thread describes one tile of the round
// in LDS (row, head, position in the row, the two block ids, the query token), and the waves take
// tiles from an LDS counter, one tile ahead of the one they load.  A wave that is served early
// simply takes more tiles, and all waves run out of work together.
//
// Per wave one chunk of MT 16-token M-tiles is in flight (8 KB of keys: one M-tile of 512-byte
// rows, two of 256-byte rows, four of rows up to 128 bytes when a tile holds 64 tokens): when it
// arrives it is written to the wave's LDS buffer (load order in, MFMA operand order out,
// conflict-free by tr_slot), the next chunk's loads go into the same registers, and the MFMAs and
// the softmax run from LDS while they are in flight.  Each finished tile's record is stored at
// once, into both of its blocks.
// ---------------------------------------------------------------------------------------
template <int MODE, int HEAD_DIM, int MT>
struct CuShape {
  using S = MfmaShape<MODE, HEAD_DIM>;
  static_assert(S::kRowBytes <= 512, "key rows of up to 512 bytes");
  static_assert(MT >= 1 && MT * 16 * S::kRowBytes <= 8192, "at most 8 KB of keys per chunk");
  static constexpr int kThreads = kCuThreads;  // 3 waves per SIMD: the shape's VGPR budget
  static constexpr int kWaves = kThreads / kWave;
  static constexpr int kRound = kThreads;  // tiles described per round, one per thread
  static constexpr int kMT = MT;           // M-tiles of 16 tokens per chunk
  static constexpr int kChunk = 16 * kMT;  // tokens per chunk
  static constexpr int kStash = kMT * 16 * S::kPieces;  // u32x4 per wave: the chunk's M-tiles
  static constexpr size_t kStaticLds = sizeof(u32x4) * kWaves * kStash + sizeof(int4) * kRound +
                                       sizeof(int) * (kRound + kWaves + 1) + sizeof(unsigned long long) * kCycleSlots;
};

template <int MODE, int HEAD_DIM, int MT>
__global__ __launch_bounds__(kCuThreads) void tile_lse_cu_kernel(const Params p) {
  using S = MfmaShape<MODE, HEAD_DIM>;
  using C = CuShape<MODE, HEAD_DIM, MT>;
  constexpr int KS = S::kSteps, NLD = S::kLoads, CH = C::kChunk;
  constexpr int NW = C::kWaves, NT = C::kThreads;
  static_assert(C::kStaticLds + sizeof(int) * (2 * kMaxRows + 1) <= 160 * 1024,
                "the staging buffers and the largest row count's offsets fit a compute unit's LDS");

  extern __shared__ int s_mem[];       // [rows + 1] tile offsets, [rows] clipped lengths
  __shared__ int s_scan[NW];
  __shared__ int s_next;               // the round's next untaken tile
  __shared__ int4 s_desc[C::kRound];   // (row | head << 16, tile in row, id0, id1)
  __shared__ int s_qtok[C::kRound];    // the row's query token
  __shared__ u32x4 s_tr[NW][C::kStash];
  // timer: the round's cycles per row, rows row0 .. row0 + kCycleSlots - 1 of the round (its rows
  // are contiguous from its first tile's), flushed once per round instead of once per wave
  __shared__ unsigned long long s_cycles[kCycleSlots];
  int *s_off = s_mem;
  int *s_len = s_mem + p.rows + 1;

  const int rows = p.rows;
  const int bs = p.block_size;
  const int tile_tokens = kTileBlocks * bs;

  // ---- per-row live tiles (runtime/audit_kernel.py:65-69) and their exclusive scan ---------
  // (the flag is a vector load issued with the lengths: a scalar one would be waited for first)
  const bool on = *(volatile const uint32_t *)p.flag != 0u;
  if (rows <= NT) {
    // a row per thread: its tile count stays in a register through the scan
    int tiles = 0;
    if (threadIdx.x < rows) {
      const int len = min(max(p.lens[threadIdx.x], 0), p.width * bs);
      s_len[threadIdx.x] = len;
      tiles = p.select[threadIdx.x] != 0 ? (len + tile_tokens - 1) / tile_tokens : 0;  // :65-69
    }
    if (!on) return;  // runtime/audit_kernel.py:64
    int total = 0;
    const int base = block_exclusive_scan<NT>(tiles, s_scan, total);
    if (threadIdx.x < rows) s_off[threadIdx.x] = base;
    if (threadIdx.x == 0) s_off[rows] = total;
  } else {
#pragma unroll 4
    for (int r = threadIdx.x; r < rows; r += NT) {
      const int len = min(max(p.lens[r], 0), p.width * bs);
      s_len[r] = len;
      s_off[r] = p.select[r] != 0 ? (len + tile_tokens - 1) / tile_tokens : 0;  // :65-69
    }
    if (!on) return;  // runtime/audit_kernel.py:64
    __syncthreads();
    const int per = (rows + NT - 1) / NT;
    const int r0 = threadIdx.x * per;
    const int r1 = min(r0 + per, rows);
    int local = 0;
    for (int r = r0; r < r1; ++r) local += s_off[r];
    int total = 0;
    int base = block_exclusive_scan<NT>(local, s_scan, total);
    for (int r = r0; r < r1; ++r) {
      const int tiles = s_off[r];
      s_off[r] = base;
      base += tiles;
    }
    if (threadIdx.x == 0) s_off[rows] = total;
  }
  if (p.cycles != nullptr)
    for (int k = threadIdx.x; k < kCycleSlots; k += NT) s_cycles[k] = 0ull;
  __syncthreads();
  const int total_tiles = s_off[rows];

  const int lane = lane_id();
  const int n = lane & 15;  // A: token of the M-tile; B / C: query row
  const int c = lane >> 4;  // dim piece within a k-step; C: token quad
  const int nsub = p.nsub;  // chunks per tile
  const int G = p.group_rows;
  u32x4 *tr = s_tr[threadIdx.x / kWave];
  const int row_in = lane / S::kPieces;  // load instruction: the lane's row and piece
  const int piece = lane % S::kPieces;
  uint32_t voff[NLD];  // the lane's byte offset in an M-tile for load j (host-checked to fit)
#pragma unroll
  for (int j = 0; j < NLD; ++j) voff[j] = (uint32_t)((j * S::kTPI + row_in) * p.k_stride_pos + piece * 16);
  const float scale2 = p.scale * kLog2e;  // scores in log2 units: exp(s - m) = exp2(s2 - m2)

  // this workgroup's slice of the flat (tile, head) list
  const long long all = (long long)total_tiles * p.groups;
  const long long u_first = all * blockIdx.x / gridDim.x;
  const long long u_last = all * (blockIdx.x + 1) / gridDim.x;

  struct Tile {
    int row, h, k, id0, id1, qtok;
  };
  auto describe = [&](int i) -> Tile {
    const int4 d = s_desc[i];
    Tile t;
    t.row = __builtin_amdgcn_readfirstlane(d.x & 0xffff);
    t.h = __builtin_amdgcn_readfirstlane(d.x >> 16);
    t.k = __builtin_amdgcn_readfirstlane(d.y);
    t.id0 = __builtin_amdgcn_readfirstlane(d.z);
    t.id1 = __builtin_amdgcn_readfirstlane(d.w);
    t.qtok = __builtin_amdgcn_readfirstlane(s_qtok[i]);
    return t;
  };
  auto take = [&]() -> int {
    int v = 0;
    if (lane == 0) v = atomicAdd(&s_next, 1);
    return __builtin_amdgcn_readfirstlane(v);
  };

  // chunk `sub` of tile T: M-tile mt covers tile positions CH sub + 16 mt .. + 16, inside one block
  auto load_chunk = [&](u32x4 (&D)[MT * NLD], const Tile &T, int sub) {
    const int64_t head_off = (int64_t)(p.group_first + T.h) * p.k_stride_head;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int tpos = sub * CH + 16 * mt;
      const int id = tpos < bs ? T.id0 : T.id1;  // past the row the tile's first block stands in
      const char *src = p.keys + (int64_t)id * p.k_stride_block + head_off + (int64_t)(tpos % bs) * p.k_stride_pos;
#pragma unroll
      for (int j = 0; j < NLD; ++j) {
        uint32_t o = voff[j];
        asm volatile("" : "+v"(o));  // keeps the scalar-base + 32-bit-offset load form
        D[mt * NLD + j] = __builtin_nontemporal_load((const u32x4 *)(src + o));
      }
    }
  };
  // B operand: query row n of the group, the dims k-step s reads (zero past group_rows)
  auto load_query = [&](u32x4 (&Q)[KS], const Tile &T) {
    const char *qrow = p.q + (int64_t)T.qtok * p.q_stride_token + (int64_t)((p.group_first + T.h) * G + n) * p.q_stride_head;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      // 16-bit keys: piece 4s + c (8 dims); fp8 keys: 16-dim piece 4(s/2) + c, half s % 2
      const int dim = S::kFp8 ? 16 * (4 * (s / 2) + c) + 8 * (s % 2) : 8 * (4 * s + c);
      Q[s] = n < G ? *(const u32x4 *)(qrow + dim * 2) : (u32x4){0u, 0u, 0u, 0u};
    }
  };
  auto stash_chunk = [&](const u32x4 (&L)[MT * NLD]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < NLD; ++j) tr[mt * 16 * S::kPieces + tr_slot<S>(j * S::kTPI + row_in, piece)] = L[mt * NLD + j];
  };
  auto mma_stashed = [&](const u32x4 (&Q)[KS], f32x4_t (&acc)[MT]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      u32x4 D[NLD];
#pragma unroll
      for (int s = 0; s < NLD; ++s) D[s] = tr[mt * 16 * S::kPieces + tr_slot<S>(n, 4 * s + c)];
      acc[mt] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
      if constexpr (S::kFp8) {
#pragma unroll
        for (int s = 0; s < NLD; ++s) {
          u32x4 lo4, hi4;
          widen_fp8(D[s], lo4, hi4);
          acc[mt] = mfma_step<kModeBF16>(lo4, Q[2 * s], acc[mt]);
          acc[mt] = mfma_step<kModeBF16>(hi4, Q[2 * s + 1], acc[mt]);
        }
      } else {
#pragma unroll
        for (int s = 0; s < KS; ++s) acc[mt] = mfma_step<MODE>(D[s], Q[s], acc[mt]);
      }
    }
  };

  for (long long r0 = u_first; r0 < u_last; r0 += C::kRound) {
    const int count = (int)min((long long)C::kRound, u_last - r0);
    // ---- describe the round's tiles, one per thread ------------------------------------
    if (threadIdx.x < count) {
      const long long u = r0 + threadIdx.x;
      // tile-major: the audited KV heads of a tile are adjacent, so the waves of a CU read the
      // heads of the same token rows at about the same time (nearly whole rows for DRAM)
      const int t = (int)(u / p.groups);
      const int h = (int)(u - (long long)t * p.groups);
      int lo = 0, hi = rows;  // the row holding tile t: the last row with s_off[row] <= t
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (s_off[mid] <= t) lo = mid; else hi = mid;
      }
      const int k = t - s_off[lo];
      const int nb = (s_len[lo] + bs - 1) / bs;
      const int32_t *trow = p.table + (int64_t)lo * p.table_stride;
      const int id0 = trow[kTileBlocks * k];
      const int id1 = kTileBlocks * k + 1 < nb ? trow[kTileBlocks * k + 1] : id0;
      s_desc[threadIdx.x] = make_int4(lo | (h << 16), k, id0, id1);
      s_qtok[threadIdx.x] = p.qrow[lo];
    }
    if (threadIdx.x == 0) s_next = 0;
    __syncthreads();
    const int round_row0 = __builtin_amdgcn_readfirstlane(s_desc[0].x & 0xffff);  // the round's first row

    // ---- the waves take the round's tiles -------------------------------------------------
    int i = take();
    if (i < count) {
      Tile T = describe(i);
      int sub = 0;
      int ahead = take();  // the tile after T, taken early so its LDS round trip is hidden
      u32x4 A[MT * NLD], qb[KS], qn[KS];
      f32x4_t acc[MT];
      load_query(qb, T);
      load_chunk(A, T, 0);
      float m_run = -INFINITY, l_run = 0.0f;
      const bool timed = p.cycles != nullptr;
      uint64_t mark = timed ? __builtin_amdgcn_s_memtime() : 0;
      while (true) {
        // the chunk after this one: the next part of T, or the first of the tile taken ahead
        Tile N = T;
        int nsub_next = sub + 1;
        bool more = true, new_query = false;
        if (nsub_next == nsub) {
          more = ahead < count;
          if (more) {
            N = describe(ahead);
            nsub_next = 0;
            ahead = take();
            new_query = N.row != T.row || N.h != T.h;
          }
        }
        stash_chunk(A);  // waits for the chunk
        if (more) {
          load_chunk(A, N, nsub_next);
          if (new_query) load_query(qn, N);
        }
        mma_stashed(qb, acc);

        // ---- the chunk's tile max and sum (query row n, tokens 4c + i of each M-tile) ----
        const int len = s_len[T.row];
        const int tok0 = T.k * tile_tokens + sub * CH;
        float sc[4 * MT];
        if (tok0 + CH <= len) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) sc[4 * mt + e] = acc[mt][e] * scale2;
        } else {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int tok = tok0 + 16 * mt + 4 * c + e;
              sc[4 * mt + e] = tok < len ? acc[mt][e] * scale2 : -INFINITY;
            }
        }
        float mx = sc[0];
#pragma unroll
        for (int e = 1; e < 4 * MT; ++e) mx = fmaxf(mx, sc[e]);
        mx = rows_max(mx);
        // exponents are <= 0 (a score minus a max); v_exp_f32 gives 0 for -inf and for underflow
        float sum = 0.0f;
        if (mx != -INFINITY) {
#pragma unroll
          for (int e = 0; e < 4 * MT; ++e) sum += __builtin_amdgcn_exp2f(sc[e] - mx);
        }
        sum = rows_sum(sum);
        const float M = fmaxf(m_run, mx);
        if (M != -INFINITY) {
          const float a = m_run == -INFINITY ? 0.0f : l_run * __builtin_amdgcn_exp2f(m_run - M);
          const float b = mx == -INFINITY ? 0.0f : sum * __builtin_amdgcn_exp2f(mx - M);
          l_run = a + b;
          m_run = M;
        }
        if (sub == nsub - 1) {
          // the tile's record into each of its blocks the row reaches, runtime/audit_kernel.py:97-109
          // (lanes of token quads 0 and 1 take blocks 2k and 2k + 1)
          const int blk = kTileBlocks * T.k + c;
          if (c < kTileBlocks && n < G && blk < (len + bs - 1) / bs) {
            float *cell = p.lse + (int64_t)T.row * p.row_stride + T.h * G + (int64_t)blk * p.cells + n;
            cell[0] = m_run * kLn2;
            cell[p.plane_stride] = l_run;
          }
          m_run = -INFINITY;
          l_run = 0.0f;
          if (timed && (!more || N.row != T.row || N.h != T.h)) {
            // the wave's time since its previous tile goes to this tile's row (first KV head).  Over
            // a run of tiles of one row and head those intervals telescope, so the clock is read
            // once, where the run ends (a clock read waits for the wave's LDS traffic).
            const uint64_t now = __builtin_amdgcn_s_memtime();
            if (T.h == 0 && T.row < p.cycles_rows && lane == 0) {
              const int slot = T.row - round_row0;
              if (slot < kCycleSlots) atomicAdd(&s_cycles[slot], (unsigned long long)(now - mark));
              else atomicAdd((unsigned long long *)(p.cycles + T.row), (unsigned long long)(now - mark));
            }
            mark = now;
          }
        }
        if (!more) break;
        if (new_query) {
#pragma unroll
          for (int s = 0; s < KS; ++s) qb[s] = qn[s];
        }
        T = N;
        sub = nsub_next;
      }
    }
    __syncthreads();  // the next round rewrites the descriptors and the counter
    if (p.cycles != nullptr && threadIdx.x < kCycleSlots) {
      // the round's rows: one add each (cleared before the next round's barrier)
      const unsigned long long c = s_cycles[threadIdx.x];
      if (c != 0ull) {
        atomicAdd((unsigned long long *)(p.cycles + round_row0 + threadIdx.x), c);
        s_cycles[threadIdx.x] = 0ull;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// The step plan.  Every audit launch of a decode step reads the same view buffers (block
// table, lengths, selected rows, query tokens); only the layer, its queries and its keys
// change.  So the work list the self-contained kernel rebuilds in every launch -- the tiles of
// each selected row, their scan, each tile's row and block ids -- is built once per step (by one
// kernel up to 4096 rows, two small kernels past that) into a plan buffer that holds, for each
// workgroup of the audit grid, the count of its tiles and their descriptors, contiguous.  A planned
// launch then starts with one load of the wave's first descriptor before its first key requests,
// and reads its later descriptors one tile ahead, as the self-contained kernel reads them from LDS.
// Each row's tiles are padded to a multiple of kPlanRun, and each workgroup's list puts its whole
// runs of kPlanRun tiles first (plan_split_head), so that a launch can give a wave a run whose
// records fill whole cache lines.
//
// Plan buffer (PlanLayout): wg[kMaxGrid] int4 = (tiles, first row, whole runs, 0), first[kMaxGrid + 1]
// = the split points of the padded tile list over the grid, row_off[rows + 1] = each row's first
// padded tile, desc[grid][cap] = the tiles of each workgroup (its whole runs, then the rest).
// ---------------------------------------------------------------------------------------
constexpr int kSplitThreads = 1024;
constexpr int kFillThreads = 256;


struct PlanLayout {
  int64_t wg, first, row_off, desc, bytes;
  int32_t cap;  // descriptors per workgroup
};

inline int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

// The padded tiles of at most rows x width (plan_split_head).
inline int64_t plan_max_tiles(int rows, int width) {
  const int64_t tiles = (width + kTileBlocks - 1) / kTileBlocks;
  return (int64_t)rows * ((tiles + kPlanRun - 1) / kPlanRun * kPlanRun);
}

// The layout of a plan for batches of at most rows x width on a grid of `grid` workgroups.  The
// split gives workgroup b the tiles [T b / grid, T (b + 1) / grid) of the T padded tiles, at most
// ceil(T / grid) of them.
inline PlanLayout plan_layout(int rows, int width, int grid) {
  PlanLayout L;
  const int64_t max_tiles = plan_max_tiles(rows, width);
  L.cap = (int32_t)std::max<int64_t>(1, (max_tiles + grid - 1) / grid);
  L.wg = 0;
  L.first = align_up(L.wg + (int64_t)sizeof(int4) * kMaxGrid, 256);
  L.row_off = align_up(L.first + 4 * (int64_t)(kMaxGrid + 1), 256);
  L.desc = align_up(L.row_off + 4 * ((int64_t)rows + 1), 256);
  L.bytes = align_up(L.desc + (int64_t)grid * L.cap * (int64_t)sizeof(TileDesc), 256);
  return L;
}

struct PlanArgs {
  const int32_t *table;
  int64_t table_stride;
  const int32_t *lens;
  const int32_t *qrow;
  const uint8_t *select;
  const uint32_t *flag;
  int32_t rows, width, block_size, grid, cap;
  int4 *wg;
  int32_t *first;
  int32_t *row_off;
  TileDesc *desc;
};

__device__ __forceinline__ int plan_row_tiles(const PlanArgs &a, int r) {
  const int tile_tokens = kTileBlocks * a.block_size;
  if (a.select[r] == 0) return 0;
  const int len = min(max(a.lens[r], 0), a.width * a.block_size);
  return (len + tile_tokens - 1) / tile_tokens;  // runtime/audit_kernel.py:65-69
}
__device__ __forceinline__ int plan_padded(int tiles) { return (tiles + kPlanRun - 1) / kPlanRun * kPlanRun; }
// split point b of T padded tiles over G workgroups
__device__ __forceinline__ int plan_first(int64_t T, int64_t G, int64_t b) { return (int)(T * b / G); }
// split b's entry: (tiles, first row, whole runs listed first, 0)
__device__ __forceinline__ int4 plan_entry(int f, int cnt, int row) {
  return make_int4(cnt, row, plan_split_runs(f, cnt), 0);
}
// tile k of a row with `real` tiles: its descriptor (past `real`: a padding tile without tokens,
// whose block ids are the row's last, so that nothing reads past the row)
__device__ __forceinline__ TileDesc plan_desc(const PlanArgs &a, int row, int k, int real, int len, int qtok) {
  const int tile_tokens = kTileBlocks * a.block_size;
  const int nb = (len + a.block_size - 1) / a.block_size;
  const int32_t *trow = a.table + (int64_t)row * a.table_stride;
  const int kk = min(k, real - 1);
  TileDesc d;
  d.row = row;
  d.k = k;
  d.valid = k < real ? min(len - k * tile_tokens, tile_tokens) : 0;
  d.qtok = qtok;
  d.id0 = trow[kTileBlocks * kk];
  d.id1 = kTileBlocks * kk + 1 < nb ? trow[kTileBlocks * kk + 1] : d.id0;  // past the row: stands in
  d.pad0 = d.pad1 = 0;
  return d;
}

// One workgroup: the live tiles of every row (none with the flag off), their exclusive scan,
// and the grid's split points and per-workgroup counts.
__global__ __launch_bounds__(kSplitThreads) void plan_split_kernel(const PlanArgs a) {
  __shared__ int s_scan[kSplitThreads / kWave];
  const bool on = *(volatile const uint32_t *)a.flag != 0u;
  const int per = (a.rows + kSplitThreads - 1) / kSplitThreads;
  const int r0 = min((int)threadIdx.x * per, a.rows);
  const int r1 = min(r0 + per, a.rows);
  int local = 0;
  if (on)
    for (int r = r0; r < r1; ++r) local += plan_padded(plan_row_tiles(a, r));
  int total = 0;
  int base = block_exclusive_scan<kSplitThreads>(local, s_scan, total);
  for (int r = r0; r < r1; ++r) {
    a.row_off[r] = base;
    if (on) base += plan_padded(plan_row_tiles(a, r));
  }
  if (threadIdx.x == 0) a.row_off[a.rows] = total;
  for (int b = threadIdx.x; b <= kMaxGrid; b += kSplitThreads) {
    const int f = b <= a.grid ? plan_first(total, a.grid, b) : total;
    a.first[b] = f;
    if (b < kMaxGrid) {
      const int next = b + 1 <= a.grid ? plan_first(total, a.grid, b + 1) : total;
      a.wg[b] = plan_entry(f, next - f, 0);
    }
  }
}

// One workgroup per row: each of the row's tiles goes to the workgroup whose split holds it, at
// its place there; the workgroup's first tile also names its first row.
__global__ __launch_bounds__(kFillThreads) void plan_fill_kernel(const PlanArgs a) {
  __shared__ int s_first[kMaxGrid + 1];
  for (int b = threadIdx.x; b <= a.grid; b += kFillThreads) s_first[b] = a.first[b];
  __syncthreads();
  for (int row = blockIdx.x; row < a.rows; row += gridDim.x) {
    const int off = a.row_off[row];
    const int tiles = a.row_off[row + 1] - off;  // padded
    if (tiles <= 0) continue;
    const int real = plan_row_tiles(a, row);
    const int len = min(max(a.lens[row], 0), a.width * a.block_size);
    const int qtok = a.qrow[row];
    for (int k = threadIdx.x; k < tiles; k += kFillThreads) {
      const int t = off + k;
      int lo = 0, hi = a.grid;  // the workgroup b with first[b] <= t < first[b + 1]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (s_first[mid] <= t) lo = mid; else hi = mid;
      }
      const int f = s_first[lo], cnt = s_first[lo + 1] - f;
      const int pos = plan_split_pos(t - f, plan_split_head(f, cnt), plan_split_runs(f, cnt));
      a.desc[(int64_t)lo * a.cap + pos] = plan_desc(a, row, k, real, len, qtok);
      if (t == f) a.wg[lo].y = row;
    }
  }
}

// The plan in one launch, for batches of at most kPlanRowsLds rows: every workgroup scans all rows'
// padded tiles itself (a few hundred rows: one block scan) into LDS, so its rows' first tiles and
// the grid's split need no kernel before it, and the workgroup of tile t comes from arithmetic on
// the split (b = floor(((t + 1) G - 1) / T) is the last b with floor(T b / G) <= t).  The workgroups
// take rows blockIdx.x, blockIdx.x + gridDim.x, ...; the owner of a workgroup's first tile writes
// its (count, first row), and workgroup 0 writes the empty workgroups' zero counts.
constexpr int kPlanThreads = 256;
constexpr int kPlanRowsLds = 4096;

__global__ __launch_bounds__(kPlanThreads) void plan_kernel(const PlanArgs a) {
  __shared__ int s_scan[kPlanThreads / kWave];
  __shared__ int s_off[kPlanRowsLds + 1];
  const bool on = *(volatile const uint32_t *)a.flag != 0u;
  const int per = (a.rows + kPlanThreads - 1) / kPlanThreads;
  const int r0 = min((int)threadIdx.x * per, a.rows);
  const int r1 = min(r0 + per, a.rows);
  int local = 0;
  if (on)
    for (int r = r0; r < r1; ++r) local += plan_padded(plan_row_tiles(a, r));
  int total = 0;
  int base = block_exclusive_scan<kPlanThreads>(local, s_scan, total);
  for (int r = r0; r < r1; ++r) {
    s_off[r] = base;
    if (on) base += plan_padded(plan_row_tiles(a, r));
  }
  if (threadIdx.x == 0) s_off[a.rows] = total;
  const int64_t T = total, G = a.grid;
  auto first = [&](int64_t b) { return plan_first(T, G, b); };
  if (blockIdx.x == 0) {
    for (int b = threadIdx.x; b < kMaxGrid; b += kPlanThreads)
      if (b >= a.grid || first(b + 1) == first(b)) a.wg[b] = make_int4(0, 0, 0, 0);
  }
  __syncthreads();
  if (T == 0) return;
  for (int row = blockIdx.x; row < a.rows; row += gridDim.x) {
    const int off = s_off[row];
    const int tiles = s_off[row + 1] - off;  // padded
    if (tiles <= 0) continue;
    const int real = plan_row_tiles(a, row);
    const int len = min(max(a.lens[row], 0), a.width * a.block_size);
    const int qtok = a.qrow[row];
    for (int k = threadIdx.x; k < tiles; k += kPlanThreads) {
      const int t = off + k;
      const int b = (int)(((int64_t)(t + 1) * G - 1) / T);
      const int fb = first(b), cnt = first(b + 1) - fb;
      const int pos = plan_split_pos(t - fb, plan_split_head(fb, cnt), plan_split_runs(fb, cnt));
      a.desc[(int64_t)b * a.cap + pos] = plan_desc(a, row, k, real, len, qtok);
      if (t == fb) a.wg[b] = plan_entry(fb, cnt, row);
    }
  }
}


constexpr int kLdsBytes = 160 * 1024;  // a compute unit's LDS
constexpr int kLayersLdsFixed = 2048;   // tile_lse_layers_kernel's LDS besides its staging and held lines

// The planned form of tile_lse_cu_kernel over one or more layers: the same chunks, dots, records
// and timer.  For layer j of the launch, workgroup b takes the plan's split (b + j) mod grid, so
// that over the layers every workgroup's share of tiles differs from another's by at most one
// tile (the split gives the first T mod grid splits one tile more), and its splits are adjacent
// in the list (their rows follow one another).  Items run layer by layer; an item is
// (tile, audited head), tile-major.  The waves take runs of items from an LDS counter (wave w
// starts at run w), reading each item's descriptor one item ahead: a run is the tiles whose records
// share cache lines (record_run_tiles) times the audited heads, and its records are stored together
// when it ends.  The runs come from the whole runs each split lists first (plan_split_head), layer
// by layer; the last NW runs' worth of them and then the splits' other tiles are taken one at a
// time, so that the waves run out of work together (a launch of one layer takes most of its items
// so).
template <int MODE, int HEAD_DIM, int MT, int MT_REF, bool RUNS>
__global__ __launch_bounds__(kCuThreads) void tile_lse_layers_kernel(const Params p, const PlanView plan,
                                                                    const LayerSet ls) {
  static_assert(MT_REF == MT || MT_REF == 2 * MT, "a reduction chunk is one or two chunks");
  using S = MfmaShape<MODE, HEAD_DIM>;
  using C = CuShape<MODE, HEAD_DIM, MT>;
  constexpr int KS = S::kSteps, NLD = S::kLoads, CH = C::kChunk;
  constexpr int NW = C::kWaves;
  // items of a run whose records are held in registers (fewer where the shape's registers are taken)
  constexpr int kRecords = HEAD_DIM >= 256 ? 1 : 8;
  static_assert(sizeof(u32x4) * C::kStash >= 256 * sizeof(float), "the records pass through the chunk staging");

  __shared__ int s_next;    // the next untaken run
  __shared__ int s_single;  // past s_switch: the next untaken single item
  __shared__ int s_switch;  // the items from here on are taken one at a time
  // the launch's items in 2 nl segments: segment j < nl holds layer j's whole runs (its split's first
  // tiles), segment nl + j the rest of layer j's split; s_pref[k] items come before segment k
  __shared__ int s_pref[2 * kMaxLaunchLayers + 1];
  __shared__ int s_whole[kMaxLaunchLayers];  // tiles in layer j's whole runs
  __shared__ u32x4 s_tr[NW][C::kStash];
  // Whole record lines (32 floats per plane) of each wave's runs, held until the wave's items are
  // done: the lines then reach memory when few reads are left.  A line's blocks pair up into tiles
  // whose two blocks hold the same record (the line starts at a tile), so a slot keeps each pair
  // once: 16 floats of the max plane, 16 of the sum plane, and the line's address, in the LDS the
  // chunk staging leaves (at the Llama-3-8B shape 69 slots a wave, more than a wave has runs).
  constexpr int kHoldBytes = 32 * 4 + 8;
  constexpr int kHold = RUNS ? (int)((kLdsBytes - kLayersLdsFixed - sizeof(u32x4) * NW * C::kStash) / (NW * kHoldBytes)) : 0;
  __shared__ float s_hold[NW][kHold > 0 ? kHold : 1][32];
  __shared__ float *s_hold_at[NW][kHold > 0 ? kHold : 1];
  __shared__ unsigned long long s_cycles[kCycleSlots];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int groups = p.groups;
  const int grid = gridDim.x;
  const int nl = ls.n;
  auto split_of = [&](int j) { return (int)((blockIdx.x + (unsigned)j) % (unsigned)grid); };
  const int run_tiles = record_run_tiles(p.cells, groups);
  // items a wave takes at a time (RUNS: the form for launches of several layers; a launch of one
  // layer takes them one at a time, its waves having a few items each)
  const int run = RUNS ? run_tiles * groups : 1;
  // the flag, the first split's count and first row, the layers' counts and the wave's first
  // descriptor: one latency (a relaxed load: a volatile one is completed before the next is issued)
  uint32_t flag = __hip_atomic_load(p.flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int4 wg = plan.wg[blockIdx.x];
  int cnt = 0, whole_runs = 0;  // wave 0: lane j holds layer j's split count and whole runs
  if (wave == 0 && lane < nl) {
    const int4 e = plan.wg[split_of(lane)];
    cnt = e.x;
    whole_runs = e.z;
  }
  u32x4 d_lo;
  u32x2 d_hi;
  load_desc(plan.desc + (int64_t)blockIdx.x * plan.cap + min(wave * run / groups, plan.cap - 1), d_lo, d_hi);
  // all are waited for here, together: otherwise the compiler tests the flag before it issues the
  // other loads, a second memory latency before the first key request
  asm volatile("" : "+v"(flag), "+v"(wg.y), "+v"(cnt), "+v"(whole_runs) : "v"(d_lo), "v"(d_hi));
  // the first layer's parameters and the shared strides, read with the others (a scalar-cache miss
  // after the barrier would be one more latency)
  const char *keys0 = ls.l[0].keys, *q0 = ls.l[0].q;
  int64_t k_block = p.k_stride_block, k_pos = p.k_stride_pos, k_head = p.k_stride_head;
  int64_t q_tok = p.q_stride_token, q_head = p.q_stride_head;
  asm volatile("" : "+s"(keys0), "+s"(q0), "+s"(k_block), "+s"(k_pos), "+s"(k_head), "+s"(q_tok), "+s"(q_head));
  if (flag == 0u) return;  // runtime/audit_kernel.py:64
  if (wave == 0) {
    // items before each segment: an inclusive scan over wave 0's lanes (lane j < nl: layer j's whole
    // runs, lane nl + j: the rest of its split)
    const int tiles_j = min(cnt, plan.cap);
    const int whole_j = min(whole_runs * kPlanRun, tiles_j);
    const int rest_j = __shfl((tiles_j - whole_j) * groups, (lane - nl) & (kWave - 1), kWave);
    const int inc = wave_inclusive_scan(lane < nl ? whole_j * groups : (lane < 2 * nl ? rest_j : 0));
    if (lane < 2 * nl) s_pref[lane + 1] = inc;
    if (lane < nl) s_whole[lane] = whole_j;
    const int in_runs = nl > 0 ? __builtin_amdgcn_readlane(inc, nl - 1) : 0;
    if (lane == 0) {
      // every wave starts with a run (wave w with items w run ..), and runs are taken while every
      // wave has at least one more ahead of it; the last NW runs' worth of them and the tiles
      // outside whole runs go one at a time, so that the waves run out of work together
      s_pref[0] = 0;
      s_switch = max(NW * run, max(0, in_runs - NW * run) / run * run);
      s_next = NW * run;
      s_single = 0;
    }
  }
  if (p.cycles != nullptr)
    for (int k = threadIdx.x; k < kCycleSlots; k += kCuThreads) s_cycles[k] = 0ull;
  const int row0 = __builtin_amdgcn_readfirstlane(wg.y);  // the first split's first row: the timer slots' base
  __syncthreads();  // s_next, the layer offsets and the timer slots are set before any take
  const int items = __builtin_amdgcn_readfirstlane(s_pref[2 * nl]);
  const int switch_at = __builtin_amdgcn_readfirstlane(s_switch);

  const int n = lane & 15;  // A: token of the M-tile; B / C: query row
  const int c = lane >> 4;  // dim piece within a k-step; C: token quad
  const int nsub = p.nsub;  // chunks per tile
  const int bs = p.block_size;
  const int G = p.group_rows;
  const bool by_row = ls.q_by_row != 0;
  u32x4 *tr = s_tr[wave];
  const int row_in = lane / S::kPieces;  // load instruction: the lane's row and piece
  const int piece = lane % S::kPieces;
  uint32_t voff[NLD];
#pragma unroll
  for (int j = 0; j < NLD; ++j) voff[j] = (uint32_t)((j * S::kTPI + row_in) * k_pos + piece * 16);

  // A wave's position in the launch's items: the segment of its latest taken item, that segment's
  // item range, its layer and the place of its first item in the layer's split.  Items a wave takes
  // only grow, so the walk moves forward.
  struct Walk {
    int k, lo, hi, j, base;
  };
  auto walk_to = [&](Walk &w, int item) {
    while (item >= w.hi) {
      ++w.k;
      w.lo = w.hi;
      w.hi = __builtin_amdgcn_readfirstlane(s_pref[w.k + 1]);
      w.j = w.k < nl ? w.k : w.k - nl;
      w.base = w.k < nl ? 0 : __builtin_amdgcn_readfirstlane(s_whole[w.j]);
    }
  };
  auto desc_of = [&](const Walk &w, int item) {
    return plan.desc + (int64_t)split_of(w.j) * plan.cap + w.base + (item - w.lo) / groups;
  };

  struct Layer {
    const char *q, *keys;
    float *lse;
    float scale2;
    int group_first, q_head0;
  };
  auto layer_of = [&](int j) -> Layer {
    j = __builtin_amdgcn_readfirstlane(j);  // a uniform index: scalar loads of the kernel arguments
    Layer L;
    L.q = ls.l[j].q;
    L.keys = ls.l[j].keys;
    L.lse = ls.l[j].lse;
    L.scale2 = ls.l[j].scale2;
    L.group_first = ls.l[j].group_first;
    L.q_head0 = ls.l[j].q_head0;
    return L;
  };

  struct Tile {
    int row, h, k, valid, id0, id1, qtok, j;
  };
  auto describe = [&](const u32x4 &lo, const u32x2 &hi, const Walk &w, int item) -> Tile {
    Tile t;
    t.row = __builtin_amdgcn_readfirstlane((int)lo[0]);
    t.k = __builtin_amdgcn_readfirstlane((int)lo[1]);
    t.valid = __builtin_amdgcn_readfirstlane((int)lo[2]);
    t.qtok = __builtin_amdgcn_readfirstlane((int)lo[3]);
    t.id0 = __builtin_amdgcn_readfirstlane((int)hi[0]);
    t.id1 = __builtin_amdgcn_readfirstlane((int)hi[1]);
    t.h = groups == 1 ? 0 : (item - w.lo) % groups;
    t.j = w.j;  // the layer
    return t;
  };
  auto take = [&]() -> int {
    int v = 0;
    if (lane == 0) {
      v = atomicAdd(&s_next, run);
      if (v >= switch_at) v = switch_at + atomicAdd(&s_single, 1);
    }
    return __builtin_amdgcn_readfirstlane(v);
  };
  // the item after item i: the next of its run, or the first of a new run (or a single item)
  auto after = [&](int i) -> int { return i + 1 < switch_at && (i + 1) % run != 0 ? i + 1 : take(); };
  auto load_chunk = [&](u32x4 (&D)[MT * NLD], const Tile &T, const Layer &L, int sub) {
    const int64_t head_off = (int64_t)(L.group_first + T.h) * k_head;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int tpos = sub * CH + 16 * mt;
      const int id = tpos < bs ? T.id0 : T.id1;
      const char *src = L.keys + (int64_t)id * k_block + head_off + (int64_t)(tpos % bs) * k_pos;
#pragma unroll
      for (int j = 0; j < NLD; ++j) {
        uint32_t o = voff[j];
        asm volatile("" : "+v"(o));
        D[mt * NLD + j] = __builtin_nontemporal_load(as_global((const u32x4 *)(src + o)));
      }
    }
  };
  auto load_query = [&](u32x4 (&Q)[KS], const Tile &T, const Layer &L) {
    const int qi = by_row ? T.row : T.qtok;
    const char *qrow =
        L.q + (int64_t)qi * q_tok + (int64_t)((L.group_first + T.h) * G + n - L.q_head0) * q_head;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int dim = S::kFp8 ? 16 * (4 * (s / 2) + c) + 8 * (s % 2) : 8 * (4 * s + c);
      Q[s] = n < G ? *as_global((const u32x4 *)(qrow + dim * 2)) : (u32x4){0u, 0u, 0u, 0u};
    }
  };
  auto stash_chunk = [&](const u32x4 (&L)[MT * NLD]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < NLD; ++j) tr[mt * 16 * S::kPieces + tr_slot<S>(j * S::kTPI + row_in, piece)] = L[mt * NLD + j];
  };
  auto mma_stashed = [&](const u32x4 (&Q)[KS], f32x4_t (&acc)[MT]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      u32x4 D[NLD];
#pragma unroll
      for (int s = 0; s < NLD; ++s) D[s] = tr[mt * 16 * S::kPieces + tr_slot<S>(n, 4 * s + c)];
      acc[mt] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
      if constexpr (S::kFp8) {
#pragma unroll
        for (int s = 0; s < NLD; ++s) {
          u32x4 lo4, hi4;
          widen_fp8(D[s], lo4, hi4);
          acc[mt] = mfma_step<kModeBF16>(lo4, Q[2 * s], acc[mt]);
          acc[mt] = mfma_step<kModeBF16>(hi4, Q[2 * s + 1], acc[mt]);
        }
      } else {
#pragma unroll
        for (int s = 0; s < KS; ++s) acc[mt] = mfma_step<MODE>(D[s], Q[s], acc[mt]);
      }
    }
  };

  const bool timed = p.cycles != nullptr;
  // the timer: a run of one layer's, row's and head's tiles is timed once, where it ends
  auto time_tile = [&](const Tile &T, uint64_t &mark) {
    const uint64_t now = __builtin_amdgcn_s_memtime();
    if (T.h == 0 && T.row < p.cycles_rows && lane == 0) {
      const int slot = T.row - row0;
      if (slot >= 0 && slot < kCycleSlots) atomicAdd(&s_cycles[slot], (unsigned long long)(now - mark));
      else atomicAdd((unsigned long long *)(p.cycles + T.row), (unsigned long long)(now - mark));
    }
    mark = now;
  };
  // the chunk's tile max and sum, folded into the tile's running (m, l); at the tile's last chunk
  // its record goes into each of its blocks the row reaches (runtime/audit_kernel.py:97-109)
  int held = 0;  // lines in this wave's hold slots
  float held_sc[4 * MT];  // PAIRS = 2: the scores of a reduction chunk's first half
  auto hold_line = [&](int F, float *line, const float *stage) -> bool {
    if constexpr (kHold == 0) {
      return false;
    } else {
      // (cells <= 16: a line holds whole tiles, two blocks each; a line of 32 cells is one block)
      if (F != 32 || p.cells > 16 || held >= kHold) return false;
      // lane u < 16 keeps the max plane's float of pair u (its first block's), lane 16 + u the sum's
      const int u = lane & 15, f = (u / p.cells) * 2 * p.cells + u % p.cells;
      if (lane < 32) s_hold[wave][held][lane] = stage[(lane < 16 ? 0 : 128) + f];
      if (lane == 0) s_hold_at[wave][held] = line;
      ++held;
      return true;
    }
  };
  auto reduce_chunk = [&](const f32x4_t (&acc)[MT], const Tile &T, const Layer &L, int sub, float &m_run,
                          float &l_run, RunRecords<kRecords> &rec) {
    const int tok0 = sub * CH;  // within the tile
    float sc[4 * MT];
    if (tok0 + CH <= T.valid) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[4 * mt + e] = acc[mt][e] * L.scale2;
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int tok = tok0 + 16 * mt + 4 * c + e;
          sc[4 * mt + e] = tok < T.valid ? acc[mt][e] * L.scale2 : -INFINITY;
        }
    }
    // the max and sum over a reduction chunk of MT_REF M-tiles: this chunk, or with PAIRS = 2 the
    // previous one (held in `held_sc`) and this one, in the order a chunk of MT_REF M-tiles takes
    // them, so that the records are the same bits as the launches of one layer write
    constexpr int PAIRS = MT_REF / MT;
    if constexpr (PAIRS == 2) {
      if ((sub & 1) == 0) {
#pragma unroll
        for (int e = 0; e < 4 * MT; ++e) held_sc[e] = sc[e];
        return;
      }
    }
    float all[4 * MT_REF];
#pragma unroll
    for (int e = 0; e < 4 * MT; ++e) {
      if constexpr (PAIRS == 2) all[e] = held_sc[e];
      all[4 * MT_REF - 4 * MT + e] = sc[e];
    }
    float mx = all[0];
#pragma unroll
    for (int e = 1; e < 4 * MT_REF; ++e) mx = fmaxf(mx, all[e]);
    mx = rows_max(mx);
    float sum = 0.0f;
    if (mx != -INFINITY) {
#pragma unroll
      for (int e = 0; e < 4 * MT_REF; ++e) sum += __builtin_amdgcn_exp2f(all[e] - mx);
    }
    sum = rows_sum(sum);
    const float M = fmaxf(m_run, mx);
    if (M != -INFINITY) {
      const float a = m_run == -INFINITY ? 0.0f : l_run * __builtin_amdgcn_exp2f(m_run - M);
      const float b = mx == -INFINITY ? 0.0f : sum * __builtin_amdgcn_exp2f(mx - M);
      l_run = a + b;
      m_run = M;
    }
    if (sub == nsub - 1) {
      const int blk = kTileBlocks * T.k + c;
      int off = -1;
      if (c < kTileBlocks && n < G && c * bs < T.valid) off = T.h * G + blk * p.cells + n;
      float *row_base = L.lse + (int64_t)T.row * p.row_stride;
      if constexpr (RUNS) {
        rec.push(row_base, off, m_run * kLn2, l_run, p.plane_stride, (float *)tr, hold_line);
      } else if (off >= 0) {
        as_global(row_base)[off] = m_run * kLn2;
        as_global(row_base)[off + p.plane_stride] = l_run;
      }
      m_run = -INFINITY;
      l_run = 0.0f;
    }
  };

  const int first_item = wave * run;
  if (first_item < items) {
    Walk w{0, 0, __builtin_amdgcn_readfirstlane(s_pref[1]), 0, 0};
    // the descriptor loaded first is tile wave x run_tiles of the first layer's split: past the first
    // layer's whole runs the wave's first item is another, loaded now
    if (first_item >= w.hi) {
      walk_to(w, first_item);
      load_desc(desc_of(w, first_item), d_lo, d_hi);
    }
    Tile T = describe(d_lo, d_hi, w, first_item);
    Layer cur = T.j == 0 ? Layer{q0, keys0, ls.l[0].lse, ls.l[0].scale2, ls.l[0].group_first, ls.l[0].q_head0}
                         : layer_of(T.j);
    int ahead = after(first_item);  // the wave's next item, its descriptor read a tile early
    if (ahead < items) {
      walk_to(w, ahead);
      load_desc(desc_of(w, ahead), d_lo, d_hi);
    }
    float m_run = -INFINITY, l_run = 0.0f;
    RunRecords<kRecords> rec;
    rec.init();
    f32x4_t acc[MT];
    // one chunk in flight per wave: it goes to LDS when it arrives and the next is requested at once
    u32x4 A[MT * NLD], qb[KS], qn[KS];
    load_query(qb, T, cur);
    if (T.valid > 0) load_chunk(A, T, cur, 0);
    int sub = 0;
    uint64_t mark = timed ? __builtin_amdgcn_s_memtime() : 0;
    while (true) {
      Tile N = T;
      Layer next = cur;
      int nsub_next = sub + 1;
      bool more = true, new_query = false, run_ends = false;
      if (nsub_next == nsub) {
        more = ahead < items;
        if (more) {
          run_ends = ahead >= switch_at || ahead % run == 0;  // N starts a new run or is a single item
          N = describe(d_lo, d_hi, w, ahead);
          if (N.j != T.j) next = layer_of(N.j);
          nsub_next = 0;
          new_query = N.row != T.row || N.h != T.h || N.j != T.j;
        }
      }
      stash_chunk(A);  // waits for the chunk
      if (more) {
        if (N.valid > 0) load_chunk(A, N, next, nsub_next);  // a padding tile has no keys
        if (new_query) load_query(qn, N, next);
        if (nsub_next == 0) {
          // the descriptor of the item after N, requested after N's keys: the wait for a chunk
          // counts every load issued before the wait, so a descriptor requested ahead of the keys
          // would hold the keys back by its own latency
          asm volatile("" ::: "memory");
          ahead = after(ahead);
          if (ahead < items) {
            walk_to(w, ahead);
            load_desc(desc_of(w, ahead), d_lo, d_hi);
          }
        }
      }
      mma_stashed(qb, acc);
      reduce_chunk(acc, T, cur, sub, m_run, l_run, rec);
      if (timed && sub == nsub - 1 && (!more || new_query)) time_tile(T, mark);
      if constexpr (RUNS) {
        if (!more || run_ends) rec.flush(p.plane_stride, (float *)tr, hold_line);
      }
      if (!more) break;
      if (new_query) {
#pragma unroll
        for (int s = 0; s < KS; ++s) qb[s] = qn[s];
      }
      T = N;
      cur = next;
      sub = nsub_next;
    }
  }
  if constexpr (kHold > 0) {
    // the held lines: lanes 0-31 the max plane's, lanes 32-63 the sum plane's, float f of a line
    // from its block pair's slot
    const int f = lane & 31;
    const int u = (f / p.cells / 2) * p.cells + f % p.cells + (lane < 32 ? 0 : 16);
    for (int k = 0; k < held; ++k) {
      float *line = s_hold_at[wave][k];
      const float v = s_hold[wave][k][u];
      __builtin_nontemporal_store(v, as_global(lane < 32 ? line + f : line + p.plane_stride + f));
    }
  }
  if (p.cycles != nullptr) {
    __syncthreads();
    if (threadIdx.x < kCycleSlots) {
      const unsigned long long cyc = s_cycles[threadIdx.x];
      if (cyc != 0ull) atomicAdd((unsigned long long *)(p.cycles + row0 + threadIdx.x), cyc);
    }
  }
}

// The step's queries staged per layer, for a launch that audits several layers after they have
// run: staged[r][h][:] = q[qrow[r]][head_first + h][:] for the selected rows (nothing with the flag
// off).  A workgroup copies 16 rows in 16-byte pieces.
constexpr int kStageThreads = 256;
constexpr int kStageRows = 16;

__global__ __launch_bounds__(kStageThreads) void stage_queries_kernel(
    const char *q, int64_t q_stride_token, int64_t q_stride_head, int32_t head_first, int32_t heads,
    int32_t row_bytes, const int32_t *qrow, const uint8_t *select, const uint32_t *flag, int32_t rows, char *staged,
    int64_t staged_row_stride) {
  if (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u) return;
  const int pieces_head = row_bytes / 16;
  const int pieces_row = heads * pieces_head;
  const int r_first = blockIdx.x * kStageRows;
  const int r_end = min(r_first + kStageRows, rows);
  for (int i = threadIdx.x; i < (r_end - r_first) * pieces_row; i += kStageThreads) {
    const int r = r_first + i / pieces_row;
    if (select[r] == 0) continue;
    const int rem = i % pieces_row;
    const int h = rem / pieces_head;
    const int pc = rem % pieces_head;
    const u32x4 v = *(const u32x4 *)(q + (int64_t)qrow[r] * q_stride_token + (int64_t)(head_first + h) * q_stride_head +
                                     16 * pc);
    *(u32x4 *)(staged + (int64_t)r * staged_row_stride + (int64_t)h * row_bytes + 16 * pc) = v;
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
    case 2: return pick_gp<MODE, HD, 2>(gp);
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

// M-tiles per chunk: 8 KB of keys, within one tile (`wide`: a tile holds at least 64 tokens)
constexpr int chunk_mtiles(int row_bytes, bool wide) { return row_bytes > 256 ? 1 : (row_bytes > 128 || !wide ? 2 : 4); }
// The run form's chunks: 4 KB of keys where a chunk of 8 KB has two M-tiles or more.  A probe of the
// launch's access pattern streams as fast with 4 KB in flight per wave (12 waves a compute unit) as
// with 8 KB, and the LDS the smaller staging leaves holds more record lines until the reads are done.
constexpr int runs_mtiles(int row_bytes, bool wide) {
  return chunk_mtiles(row_bytes, wide) > 1 ? chunk_mtiles(row_bytes, wide) / 2 : 1;
}

template <int MODE, int HD>
KernelFn pick_mfma_mt(bool wide) {
  constexpr int kRowBytes = MfmaShape<MODE, HD>::kRowBytes;
  if constexpr (kRowBytes <= 128) {
    if (wide) return tile_lse_cu_kernel<MODE, HD, chunk_mtiles(kRowBytes, true)>;
  }
  return tile_lse_cu_kernel<MODE, HD, chunk_mtiles(kRowBytes, false)>;
}

template <int MODE>
KernelFn pick_mfma_hd(int hd, bool wide) {
  switch (hd) {
    case 32:
      if constexpr (MODE != kModeFp8Bf16) return pick_mfma_mt<MODE, 32>(wide);  // fp8 rows of 32 B: the VALU
      return nullptr;
    case 64: return pick_mfma_mt<MODE, 64>(wide);
    case 128: return pick_mfma_mt<MODE, 128>(wide);
    case 256: return pick_mfma_mt<MODE, 256>(wide);
  }
  return nullptr;
}

KernelFn pick_mfma(int mode, int hd, bool wide) {
  switch (mode) {
    case kModeF16: return pick_mfma_hd<kModeF16>(hd, wide);
    case kModeBF16: return pick_mfma_hd<kModeBF16>(hd, wide);
    case kModeFp8Bf16: return pick_mfma_hd<kModeFp8Bf16>(hd, wide);
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

// Workgroups of `fn` one compute unit holds at once with `lds` bytes of dynamic LDS and
// `threads` threads per workgroup (cached; 0 when one does not fit).
int resident_blocks(KernelFn fn, size_t lds, int threads) {
  struct Entry {
    KernelFn fn;
    size_t lds;
    int blocks;
  };
  static Entry cache[64];
  static int used = 0;
  static std::mutex lock;
  std::lock_guard<std::mutex> guard(lock);
  for (int i = 0; i < used; ++i)
    if (cache[i].fn == fn && cache[i].lds == lds) return cache[i].blocks;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void *>(fn), threads, lds) !=
          hipSuccess ||
      n < 0)
    n = 0;
  if (used < 64) cache[used++] = Entry{fn, lds, n};
  return n;
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

namespace ekv {
namespace audit {

using PlannedFn = void (*)(const Params, const PlanView, const LayerSet);

// (the run form's chunks, runs_mtiles, are reduced in pairs where they are half of chunk_mtiles)
template <int MODE, int HD, bool RUNS>
PlannedFn pick_planned_mt(bool wide) {
  constexpr int kRowBytes = MfmaShape<MODE, HD>::kRowBytes;
  constexpr auto mtiles = RUNS ? runs_mtiles : chunk_mtiles;
  if constexpr (kRowBytes <= 128) {
    if (wide)
      return tile_lse_layers_kernel<MODE, HD, mtiles(kRowBytes, true), chunk_mtiles(kRowBytes, true), RUNS>;
  }
  return tile_lse_layers_kernel<MODE, HD, mtiles(kRowBytes, false), chunk_mtiles(kRowBytes, false), RUNS>;
}

template <int MODE, bool RUNS>
PlannedFn pick_planned_hd(int hd, bool wide) {
  switch (hd) {
    case 32:
      if constexpr (MODE != kModeFp8Bf16) return pick_planned_mt<MODE, 32, RUNS>(wide);
      return nullptr;
    case 64: return pick_planned_mt<MODE, 64, RUNS>(wide);
    case 128: return pick_planned_mt<MODE, 128, RUNS>(wide);
    case 256: return pick_planned_mt<MODE, 256, RUNS>(wide);
  }
  return nullptr;
}

// the planned kernel of a shape; `runs`: the form for launches of several layers
PlannedFn pick_planned(int mode, int hd, bool wide, bool runs) {
  switch (mode) {
    case kModeF16: return runs ? pick_planned_hd<kModeF16, true>(hd, wide) : pick_planned_hd<kModeF16, false>(hd, wide);
    case kModeBF16:
      return runs ? pick_planned_hd<kModeBF16, true>(hd, wide) : pick_planned_hd<kModeBF16, false>(hd, wide);
    case kModeFp8Bf16:
      return runs ? pick_planned_hd<kModeFp8Bf16, true>(hd, wide) : pick_planned_hd<kModeFp8Bf16, false>(hd, wide);
  }
  return nullptr;
}

// The kernel choice and launch shape of one audit call.
struct Launch {
  KernelFn fn = nullptr;        // the self-contained kernel (none for some VALU shapes)
  PlannedFn planned = nullptr;       // the planned form, for the MFMA shapes
  PlannedFn planned_runs = nullptr;  // its form for launches of several layers
  int nsub_runs = 0;                 // that form's chunks per tile
  bool valu_planned = false;    // the planned form on the VALU (ekv_audit_valu.hip), for the others
  int mode = 0, head_dim = 0;
  int threads = kThreads;
  size_t lds = 0;
  int64_t blocks = 0;
};

// Checks the arguments of an audit call and fills its kernel parameters and launch shape.
int audit_setup(const void *q, int q_dtype, int64_t q_stride_token, int64_t q_stride_head, const void *keys,
                int kv_dtype, int64_t k_stride_block, int64_t k_stride_pos, int64_t k_stride_head, float k_scale,
                const int32_t *table, int64_t table_stride, const int32_t *lens, const int32_t *qrow,
                const uint8_t *select, const uint32_t *flag, float *lse, int64_t lse_plane_stride,
                int64_t lse_layer_stride, int64_t lse_row_stride, int32_t cells, uint64_t *cycles,
                int32_t cycles_rows, float scale, int32_t layer, int32_t group_first, int32_t groups,
                int32_t group_rows, int32_t rows, int32_t width, int32_t block_size, int32_t tile_blocks,
                int32_t head_dim, int32_t chunk_tiles, bool planned, Params &p, Launch &L) {
  if (q == nullptr || keys == nullptr || table == nullptr || lens == nullptr || qrow == nullptr ||
      select == nullptr || flag == nullptr || lse == nullptr)
    return fail(EKV_EINVAL, "ekv_audit_tile_lse: null pointer argument");
  if (tile_blocks != kTileBlocks)
    return fail(EKV_EUNSUPPORTED, "ekv_audit_tile_lse: tiles of %d blocks; the kernel records tiles of %d",
                tile_blocks, kTileBlocks);
  if (rows < 0 || width <= 0 || block_size <= 0 || layer < 0)
    return fail(EKV_EINVAL, "ekv_audit_tile_lse: rows %d, width %d, block %d, layer %d out of range", rows, width,
                block_size, layer);
  if (group_rows < 1 || group_rows > 16)
    return fail(EKV_EINVAL, "ekv_audit_tile_lse: %d query rows per KV head; at most 16 are recorded", group_rows);
  if (groups < 1 || groups > 32767 || group_first < 0 || cells < groups * group_rows)
    return fail(EKV_EINVAL, "ekv_audit_tile_lse: %d groups from %d need %d cells per block, the plane has %d",
                groups, group_first, groups * group_rows, cells);
  if (((kTileBlocks * block_size) & (kTileBlocks * block_size - 1)) != 0)
    return fail(EKV_EINVAL, "ekv_audit_tile_lse: a tile must hold a power of two of tokens");

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
  // 16-bit and fp8 keys use the MFMA form when a 32-token chunk fits the tile (and, for fp8, a
  // k-step holds two 16-byte pieces of the row); otherwise (fp32 keys, blocks of 8 tokens, fp8 rows
  // of 32 dimensions) the dot products run on the VALU
  const bool use_mfma = mode != kModeF32 && tile_tokens % 32 == 0 &&
                        (head_dim == 64 || head_dim == 128 || head_dim == 256 ||
                         (head_dim == 32 && mode != kModeFp8Bf16));
  L.mode = mode;
  L.head_dim = head_dim;
  int nsub = 1;
  if (use_mfma) {
    const bool wide = tile_tokens % 64 == 0;
    L.fn = pick_mfma(mode, head_dim, wide);
    L.planned = pick_planned(mode, head_dim, wide, false);
    L.planned_runs = pick_planned(mode, head_dim, wide, true);
    nsub = tile_tokens / (16 * chunk_mtiles(row_bytes, wide));  // chunks of up to 8 KB of keys
    L.nsub_runs = tile_tokens / (16 * runs_mtiles(row_bytes, wide));
    L.threads = kCuThreads;
  } else if (planned) {
    // the planned VALU form: lanes of 16, 8 or 4 bytes, so that a load instruction sits in a block
    L.valu_planned = valu_planned_shape(mode, head_dim, block_size);
    nsub = valu_planned_nsub(mode, head_dim, block_size, group_rows);
    if (!L.valu_planned || nsub < 1)
      return fail(EKV_EUNSUPPORTED, "ekv_audit_tile_lse: no planned kernel for dtype %d, head_dim %d, block size %d",
                  kv_dtype, head_dim, block_size);
  } else {
    // The self-contained VALU form: a chunk is NL load instructions of TPI tokens of 16-byte lanes
    // (8 KB of keys at NL = 8).  A load instruction must sit inside one block, and a chunk inside
    // one tile; other shapes take the planned form.
    if (block_size % tpi != 0)
      return fail(EKV_EUNSUPPORTED, "ekv_audit_tile_lse: block size %d is below the %d tokens of one load (a "
                  "step plan takes this shape)", block_size, tpi);
    const int nl = tile_tokens / tpi >= 8 ? 8 : tile_tokens / tpi;
    const int gp = group_rows <= 4 ? 4 : (group_rows <= 8 ? 8 : 16);
    L.fn = pick(mode, head_dim, nl, gp);
    nsub = tile_tokens / (nl * tpi);
    L.threads = kThreads;
  }
  if (L.fn == nullptr && L.planned == nullptr && !L.valu_planned)
    return fail(EKV_EUNSUPPORTED, "ekv_audit_tile_lse: no kernel for dtype %d, head_dim %d, block size %d (a step "
                "plan takes more shapes)", kv_dtype, head_dim, block_size);
  // the self-contained kernels keep per-row tile offsets in LDS; a planned launch reads them from the
  // plan and takes any number of rows
  const bool row_lds = !planned;
  if (row_lds && rows > kMaxRows)
    return fail(EKV_EINVAL, "ekv_audit_tile_lse: %d rows; a launch without a step plan takes at most %d", rows,
                kMaxRows);
  // 16-byte loads of key rows and query slices
  const uint64_t kaddr = (uint64_t)keys | (uint64_t)(k_stride_block * kbytes) |
                         (uint64_t)(k_stride_pos * kbytes) | (uint64_t)(k_stride_head * kbytes);
  const uint64_t qaddr = (uint64_t)q | (uint64_t)(q_stride_token * qbytes) | (uint64_t)(q_stride_head * qbytes);
  if ((kaddr & 15) != 0 || (qaddr & 15) != 0)
    return fail(EKV_EINVAL, "ekv_audit_tile_lse: key and query rows must be 16-byte aligned");
  // the MFMA form addresses the 16 positions of an M-tile with 32-bit lane offsets
  if (use_mfma && (k_stride_pos <= 0 || 16 * k_stride_pos * kbytes + row_bytes > ((int64_t)1 << 31)))
    return fail(EKV_EUNSUPPORTED, "ekv_audit_tile_lse: key position stride %lld (positive, 16 positions in 2 GiB)",
                (long long)k_stride_pos);

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
  p.chunk_tiles = chunk_tiles > 0 ? chunk_tiles : 1;
  p.nsub = nsub;
  p.nsub_log2 = 0;
  while ((1 << p.nsub_log2) < nsub) ++p.nsub_log2;

  // One resident wave per slot the GPU has: the work list is split evenly over the grid, so a
  // second round of workgroups would only add a tail.  chunk_tiles bounds the grid for small
  // batches (at least that many tiles per wave).
  if (!row_lds) return EKV_OK;  // the planned launch's grid is one workgroup per compute unit
  L.lds = (size_t)(use_mfma ? 2 * rows + 1 : rows + 1) * sizeof(int);
  const int64_t max_tiles = (int64_t)rows * ((width + kTileBlocks - 1) / kTileBlocks) * groups;
  const int64_t min_per_wave = p.chunk_tiles;
  const int waves = L.threads / kWave;
  int64_t blocks = (max_tiles + min_per_wave * waves - 1) / (min_per_wave * waves);
  const int resident = resident_blocks(L.fn, L.lds, L.threads);
  if (resident < 1)
    return fail(EKV_EUNSUPPORTED, "ekv_audit_tile_lse: a workgroup of %d threads with %zu bytes of row data does "
                "not fit a compute unit (rows %d)", L.threads, L.lds, rows);
  const int64_t cap = (int64_t)cu_count() * resident;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  L.blocks = blocks;
  return EKV_OK;
}

// The grid of a planned launch and of the plan it reads: one workgroup per compute unit.
int plan_grid() { return std::min(cu_count(), kMaxGrid); }

int check_plan(const void *plan, size_t plan_bytes, int32_t plan_rows, int32_t plan_width, int32_t rows,
               int32_t width, const char *who) {
  if (plan == nullptr) return fail(EKV_EINVAL, "%s: null plan", who);
  if (plan_rows <= 0 || plan_width <= 0 || rows > plan_rows || width > plan_width)
    return fail(EKV_EINVAL, "%s: a batch of %d x %d does not fit a plan for %d x %d", who, rows, width, plan_rows,
                plan_width);
  if (plan_max_tiles(plan_rows, plan_width) > INT32_MAX / 2)
    return fail(EKV_EINVAL, "%s: a plan for %d x %d holds more tiles than 32-bit indices count", who, plan_rows,
                plan_width);
  const PlanLayout Lp = plan_layout(plan_rows, plan_width, plan_grid());
  if ((int64_t)plan_bytes < Lp.bytes)
    return fail(EKV_EINVAL, "%s: the plan has %zu bytes, %lld are needed", who, plan_bytes, (long long)Lp.bytes);
  if (((uintptr_t)plan & 255) != 0) return fail(EKV_EINVAL, "%s: the plan must be 256-byte aligned", who);
  return EKV_OK;
}

// One planned launch of the layers `ls` on the plan's grid: the MFMA form, or the VALU one.
int launch_planned(const Launch &L, const Params &p, const LayerSet &ls, const void *plan, int32_t plan_rows,
                   int32_t plan_width, void *stream, const char *what) {
  const int grid = plan_grid();
  const PlanLayout Lp = plan_layout(plan_rows, plan_width, grid);
  PlanView v;
  v.wg = (const int4 *)((const char *)plan + Lp.wg);
  v.desc = (const TileDesc *)((const char *)plan + Lp.desc);
  v.cap = Lp.cap;
  if (L.planned == nullptr)
    return launch_valu_layers(L.mode, L.head_dim, p.block_size, p.group_rows, p, v, ls, grid, (hipStream_t)stream, what);
  if (ls.n > 1) {
    Params q = p;
    q.nsub = L.nsub_runs;
    hipLaunchKernelGGL(L.planned_runs, dim3(grid), dim3(kCuThreads), 0, (hipStream_t)stream, q, v, ls);
  } else {
    hipLaunchKernelGGL(L.planned, dim3(grid), dim3(kCuThreads), 0, (hipStream_t)stream, p, v, ls);
  }
  return check_hip(hipGetLastError(), what);
}

}  // namespace audit
}  // namespace ekv

extern "C" int ekv_audit_tile_lse(
    const void *q, int q_dtype, int64_t q_stride_token, int64_t q_stride_head, const void *keys,
    int kv_dtype, int64_t k_stride_block, int64_t k_stride_pos, int64_t k_stride_head, float k_scale,
    const int32_t *table, int64_t table_stride, const int32_t *lens, const int32_t *qrow,
    const uint8_t *select, const uint32_t *flag, float *lse, int64_t lse_plane_stride,
    int64_t lse_layer_stride, int64_t lse_row_stride, int32_t cells, uint64_t *cycles,
    int32_t cycles_rows, float scale, int32_t layer, int32_t group_first, int32_t groups,
    int32_t group_rows, int32_t rows, int32_t width, int32_t block_size, int32_t tile_blocks,
    int32_t head_dim, int32_t chunk_tiles, void *stream) {
  Params p;
  Launch L;
  const int rc = audit_setup(q, q_dtype, q_stride_token, q_stride_head, keys, kv_dtype, k_stride_block, k_stride_pos,
                             k_stride_head, k_scale, table, table_stride, lens, qrow, select, flag, lse,
                             lse_plane_stride, lse_layer_stride, lse_row_stride, cells, cycles, cycles_rows, scale,
                             layer, group_first, groups, group_rows, rows, width, block_size, tile_blocks, head_dim,
                             chunk_tiles, false, p, L);
  if (rc != EKV_OK || rows == 0) return rc;
  hipLaunchKernelGGL(L.fn, dim3((unsigned)L.blocks), dim3(L.threads), L.lds, (hipStream_t)stream, p);
  return check_hip(hipGetLastError(), "ekv_audit_tile_lse launch");
}

extern "C" size_t ekv_audit_plan_bytes(int32_t rows, int32_t width) {
  if (rows <= 0 || width <= 0 || plan_max_tiles(rows, width) > INT32_MAX / 2) return 0;
  return (size_t)plan_layout(rows, width, plan_grid()).bytes;
}

extern "C" int ekv_audit_plan(const int32_t *table, int64_t table_stride, const int32_t *lens,
                              const int32_t *qrow, const uint8_t *select, const uint32_t *flag, int32_t rows,
                              int32_t width, int32_t block_size, int32_t tile_blocks, void *plan,
                              size_t plan_bytes, int32_t plan_rows, int32_t plan_width, void *stream) {
  if (table == nullptr || lens == nullptr || qrow == nullptr || select == nullptr || flag == nullptr)
    return fail(EKV_EINVAL, "ekv_audit_plan: null pointer argument");
  if (tile_blocks != kTileBlocks)
    return fail(EKV_EUNSUPPORTED, "ekv_audit_plan: tiles of %d blocks; the kernel records tiles of %d",
                tile_blocks, kTileBlocks);
  if (rows < 0 || width <= 0 || block_size <= 0 || (int64_t)width * block_size > INT32_MAX)
    return fail(EKV_EINVAL, "ekv_audit_plan: rows %d, width %d, block %d out of range", rows, width, block_size);
  const int rc = check_plan(plan, plan_bytes, plan_rows, plan_width, rows, width, "ekv_audit_plan");
  if (rc != EKV_OK) return rc;
  const int grid = plan_grid();
  const PlanLayout Lp = plan_layout(plan_rows, plan_width, grid);
  char *base = (char *)plan;
  PlanArgs a;
  a.table = table;
  a.table_stride = table_stride;
  a.lens = lens;
  a.qrow = qrow;
  a.select = select;
  a.flag = flag;
  a.rows = rows;
  a.width = width;
  a.block_size = block_size;
  a.grid = grid;
  a.cap = Lp.cap;
  a.wg = (int4 *)(base + Lp.wg);
  a.first = (int32_t *)(base + Lp.first);
  a.row_off = (int32_t *)(base + Lp.row_off);
  a.desc = (TileDesc *)(base + Lp.desc);
  if (rows <= kPlanRowsLds) {  // one launch
    const int blocks = std::max(1, std::min(rows, 1024));
    hipLaunchKernelGGL(plan_kernel, dim3(blocks), dim3(kPlanThreads), 0, (hipStream_t)stream, a);
    return check_hip(hipGetLastError(), "ekv_audit_plan launch");
  }
  hipLaunchKernelGGL(plan_split_kernel, dim3(1), dim3(kSplitThreads), 0, (hipStream_t)stream, a);
  int rc2 = check_hip(hipGetLastError(), "ekv_audit_plan split launch");
  if (rc2 != EKV_OK || rows == 0) return rc2;
  const int fill_blocks = std::min(rows, 4096);
  hipLaunchKernelGGL(plan_fill_kernel, dim3(fill_blocks), dim3(kFillThreads), 0, (hipStream_t)stream, a);
  return check_hip(hipGetLastError(), "ekv_audit_plan fill launch");
}

extern "C" int ekv_audit_tile_lse_planned(
    const void *q, int q_dtype, int64_t q_stride_token, int64_t q_stride_head, const void *keys,
    int kv_dtype, int64_t k_stride_block, int64_t k_stride_pos, int64_t k_stride_head, float k_scale,
    const int32_t *table, int64_t table_stride, const int32_t *lens, const int32_t *qrow,
    const uint8_t *select, const uint32_t *flag, float *lse, int64_t lse_plane_stride,
    int64_t lse_layer_stride, int64_t lse_row_stride, int32_t cells, uint64_t *cycles,
    int32_t cycles_rows, float scale, int32_t layer, int32_t group_first, int32_t groups,
    int32_t group_rows, int32_t rows, int32_t width, int32_t block_size, int32_t tile_blocks,
    int32_t head_dim, const void *plan, size_t plan_bytes, int32_t plan_rows, int32_t plan_width,
    void *stream) {
  Params p;
  Launch L;
  int rc = audit_setup(q, q_dtype, q_stride_token, q_stride_head, keys, kv_dtype, k_stride_block, k_stride_pos,
                       k_stride_head, k_scale, table, table_stride, lens, qrow, select, flag, lse, lse_plane_stride,
                       lse_layer_stride, lse_row_stride, cells, cycles, cycles_rows, scale, layer, group_first,
                       groups, group_rows, rows, width, block_size, tile_blocks, head_dim, 0, true, p, L);
  if (rc != EKV_OK) return rc;
  rc = check_plan(plan, plan_bytes, plan_rows, plan_width, rows, width, "ekv_audit_tile_lse_planned");
  if (rc != EKV_OK || rows == 0) return rc;
  LayerSet ls{};
  ls.n = 1;
  ls.q_by_row = 0;
  ls.l[0] = LayerArgs{p.q, p.keys, p.lse, p.scale * kLog2e, p.group_first, 0, p.scale};
  return launch_planned(L, p, ls, plan, plan_rows, plan_width, stream, "ekv_audit_tile_lse_planned launch");
}

extern "C" int ekv_audit_shape(int q_dtype, int kv_dtype, int32_t head_dim, int32_t block_size) {
  int mode;
  if (kv_dtype == EKV_F32 && q_dtype == EKV_F32) mode = kModeF32;
  else if (kv_dtype == EKV_F16 && q_dtype == EKV_F16) mode = kModeF16;
  else if (kv_dtype == EKV_BF16 && q_dtype == EKV_BF16) mode = kModeBF16;
  else if (kv_dtype == EKV_FP8_E4M3 && q_dtype == EKV_BF16) mode = kModeFp8Bf16;
  else return 0;
  const int tile_tokens = kTileBlocks * block_size;
  if (block_size <= 0 || (tile_tokens & (tile_tokens - 1)) != 0) return 0;
  const int row_bytes = head_dim * dtype_bytes(kv_dtype);
  if (row_bytes < 16 || row_bytes > 1024 || (row_bytes & (row_bytes - 1)) != 0) return 0;
  const bool use_mfma = mode != kModeF32 && tile_tokens % 32 == 0 &&
                        (head_dim == 64 || head_dim == 128 || head_dim == 256 ||
                         (head_dim == 32 && mode != kModeFp8Bf16));
  if (use_mfma) return EKV_AUDIT_SELF_CONTAINED | EKV_AUDIT_PLANNED;
  int bits = valu_planned_shape(mode, head_dim, block_size) ? EKV_AUDIT_PLANNED : 0;
  const int tpi = kWave / (row_bytes / 16);
  if (block_size % tpi == 0) {
    const int nl = tile_tokens / tpi >= 8 ? 8 : tile_tokens / tpi;
    if (pick(mode, head_dim, nl, 4) != nullptr) bits |= EKV_AUDIT_SELF_CONTAINED;
  }
  return bits;
}

extern "C" int ekv_audit_tile_lse_layers(
    const ekv_audit_layer_t *layers, int32_t n_layers, int32_t q_by_row, int q_dtype, int64_t q_stride_token,
    int64_t q_stride_head, int kv_dtype, int64_t k_stride_block, int64_t k_stride_pos, int64_t k_stride_head,
    const int32_t *table, int64_t table_stride, const int32_t *lens, const int32_t *qrow, const uint8_t *select,
    const uint32_t *flag, float *lse, int64_t lse_plane_stride, int64_t lse_layer_stride, int64_t lse_row_stride,
    int32_t cells, uint64_t *cycles, int32_t cycles_rows, int32_t groups, int32_t group_rows, int32_t rows,
    int32_t width, int32_t block_size, int32_t tile_blocks, int32_t head_dim, const void *plan, size_t plan_bytes,
    int32_t plan_rows, int32_t plan_width, void *stream) {
  if (layers == nullptr || n_layers < 0) return fail(EKV_EINVAL, "ekv_audit_tile_lse_layers: no layer list");
  if (n_layers == 0) return EKV_OK;
  // the shared arguments, checked with the first layer's pointers; every layer's own below
  Params p;
  Launch L;
  int rc = audit_setup(layers[0].q, q_dtype, q_stride_token, q_stride_head, layers[0].keys, kv_dtype, k_stride_block,
                       k_stride_pos, k_stride_head, layers[0].k_scale, table, table_stride, lens, qrow, select, flag,
                       lse, lse_plane_stride, lse_layer_stride, lse_row_stride, cells, cycles, cycles_rows,
                       layers[0].scale, layers[0].layer, layers[0].group_first, groups, group_rows, rows, width,
                       block_size, tile_blocks, head_dim, 0, true, p, L);
  if (rc != EKV_OK) return rc;
  rc = check_plan(plan, plan_bytes, plan_rows, plan_width, rows, width, "ekv_audit_tile_lse_layers");
  if (rc != EKV_OK || rows == 0) return rc;
  const int qbytes = dtype_bytes(q_dtype);
  for (int i = 0; i < n_layers; ++i) {
    const ekv_audit_layer_t &e = layers[i];
    if (e.q == nullptr || e.keys == nullptr || e.layer < 0)
      return fail(EKV_EINVAL, "ekv_audit_tile_lse_layers: layer entry %d has a null pointer or a negative layer", i);
    if ((((uintptr_t)e.q | (uintptr_t)e.keys) & 15) != 0)
      return fail(EKV_EINVAL, "ekv_audit_tile_lse_layers: layer entry %d's query or key rows are not 16-byte aligned", i);
    if (e.group_first < 0 || e.q_head0 < 0 || e.q_head0 > e.group_first * group_rows)
      return fail(EKV_EINVAL, "ekv_audit_tile_lse_layers: layer entry %d: group %d with staged head %d", i,
                  e.group_first, e.q_head0);
  }
  (void)qbytes;
  for (int first = 0; first < n_layers; first += kMaxLaunchLayers) {
    LayerSet ls{};
    ls.n = std::min(kMaxLaunchLayers, n_layers - first);
    ls.q_by_row = q_by_row != 0;
    for (int i = 0; i < ls.n; ++i) {
      const ekv_audit_layer_t &e = layers[first + i];
      ls.l[i] = LayerArgs{(const char *)e.q, (const char *)e.keys, lse + (int64_t)e.layer * lse_layer_stride,
                          e.scale * e.k_scale * kLog2e, e.group_first, e.q_head0, e.scale * e.k_scale};
    }
    rc = launch_planned(L, p, ls, plan, plan_rows, plan_width, stream, "ekv_audit_tile_lse_layers launch");
    if (rc != EKV_OK) return rc;
  }
  return EKV_OK;
}

extern "C" int ekv_audit_stage_queries(const void *q, int q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                                       int32_t head_first, int32_t heads, int32_t head_dim, const int32_t *qrow,
                                       const uint8_t *select, const uint32_t *flag, int32_t rows, void *staged,
                                       int64_t staged_row_stride, void *stream) {
  if (q == nullptr || qrow == nullptr || select == nullptr || flag == nullptr || staged == nullptr)
    return fail(EKV_EINVAL, "ekv_audit_stage_queries: null pointer argument");
  const int qbytes = dtype_bytes(q_dtype);
  if (qbytes == 0 || q_dtype == EKV_FP8_E4M3)
    return fail(EKV_EUNSUPPORTED, "ekv_audit_stage_queries: query dtype %d", q_dtype);
  if (rows < 0 || heads <= 0 || head_first < 0 || head_dim <= 0)
    return fail(EKV_EINVAL, "ekv_audit_stage_queries: rows %d, heads %d from %d, head_dim %d", rows, heads, head_first,
                head_dim);
  const int64_t row_bytes = (int64_t)head_dim * qbytes;
  if (staged_row_stride < (int64_t)heads * head_dim)
    return fail(EKV_EINVAL, "ekv_audit_stage_queries: a staged row of %lld elements holds fewer than %d heads",
                (long long)staged_row_stride, heads);
  const uint64_t align = (uint64_t)q | (uint64_t)staged | (uint64_t)(q_stride_token * qbytes) |
                         (uint64_t)(q_stride_head * qbytes) | (uint64_t)(staged_row_stride * qbytes) |
                         (uint64_t)row_bytes;
  if ((align & 15) != 0) return fail(EKV_EINVAL, "ekv_audit_stage_queries: rows must be 16-byte aligned");
  if (rows == 0) return EKV_OK;
  const int blocks = (rows + kStageRows - 1) / kStageRows;
  hipLaunchKernelGGL(stage_queries_kernel, dim3(blocks), dim3(kStageThreads), 0, (hipStream_t)stream, (const char *)q,
                     q_stride_token * qbytes, q_stride_head * qbytes, head_first, heads, (int32_t)row_bytes, qrow,
                     select, flag, rows, (char *)staged, staged_row_stride * qbytes);
  return check_hip(hipGetLastError(), "ekv_audit_stage_queries launch");
}
