// The planned audit on the VALU, for the shapes without an MFMA form: fp32 keys, blocks of 8 tokens,
// and fp8 keys of 32 dimensions.  Semantics are those of tile_lse_kernel (runtime/audit_kernel.py
// :34-109): per (row, tile of 2 blocks, audited head, query row) the tile max m and the sum
// l = sum exp(s - m) of s = scale * <q, k> over the tile's keys, stored into each block of the tile
// that the row reaches.
//
// It reads the step plan (ekv_audit_plan) as the MFMA planned kernel does, so it takes any number of
// rows, and up to 32 layers per launch: for layer j of the launch, workgroup b takes the plan's split
// (b + j) mod grid, and the workgroup's waves take (tile, head) items from an LDS counter, one ahead.
//
// Loads.  A key row of row_bytes is read by LPT = row_bytes / LW lanes of LW bytes (16, 8 or 4), so
// that one load instruction covers TPI = 64 / LPT tokens of one block: LW shrinks for small rows in
// small blocks (fp8 or 16-bit rows of 64 bytes in 8-token blocks: 8-byte lanes; 32-byte fp8 rows in
// 8-token blocks: 4-byte lanes).  A chunk is NL instructions (up to 8); two chunks are in flight per
// wave, the next one requested before the current one is reduced, across tiles and items.
//
// Dots.  Each lane multiplies its slice of the key row with the same slice of the GP query rows
// (v_dot2 for 16-bit and widened fp8 keys, FMA for fp32), a transpose reduction over the LPT lanes
// of a token leaves each lane complete scores, and the tile's max and sum are wave reductions over
// the lanes holding one query row.  Scores are in natural units, as in the self-contained VALU
// kernel, so the records of both are the same bits.
#include <algorithm>

#include "ekv_audit.hpp"

namespace ekv {
namespace audit {

constexpr int kValuThreads = 512;  // 8 waves: one workgroup per compute unit

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <int LW>
struct LoadOf;
template <>
struct LoadOf<16> {
  typedef u32x4 T;
};
template <>
struct LoadOf<8> {
  typedef u32x2 T;
};
template <>
struct LoadOf<4> {
  typedef uint32_t T;
};

template <int LW>
__device__ __forceinline__ uint32_t word_of(const typename LoadOf<LW>::T &v, int e) {
  if constexpr (LW == 4) return v;
  else return v[e];
}

// The layout of one VALU shape: key row bytes split over LPT lanes of LW bytes, NL load instructions
// per chunk, GP query rows (padded) per audited head.
template <int MODE, int HEAD_DIM, int NL, int GP, int LW>
struct VShape {
  static constexpr int kKBytes = MODE == kModeF32 ? 4 : (MODE == kModeFp8Bf16 ? 1 : 2);
  static constexpr int kQBytes = MODE == kModeF32 ? 4 : 2;
  static constexpr int kRowBytes = HEAD_DIM * kKBytes;
  static constexpr int kLPT = kRowBytes / LW;          // lanes per key row
  static constexpr int kTPI = kLPT > 0 ? kWave / kLPT : 1;  // tokens per load instruction
  static constexpr int kKW = LW / 4;                   // key words per lane per load
  static constexpr int kOW = MODE == kModeFp8Bf16 ? 2 * kKW : kKW;  // operand words (fp8 widened to bf16)
  static constexpr int kQW = (LW / kKBytes) * kQBytes / 4;          // query words per row per lane
  static constexpr int kV = NL * GP;                   // partial dots per lane
  static constexpr int kVF = kLPT > 0 ? kV / kLPT : 0;  // scores per lane after the reduction
  static constexpr int kCT = NL * kTPI;                // tokens per chunk
  static constexpr bool kValid = kRowBytes % LW == 0 && kLPT >= 1 && kLPT <= kWave && (kLPT & (kLPT - 1)) == 0 &&
                                 kV >= kLPT && kQW == kOW;
  static constexpr int kLPH = !kValid ? 1 : (kVF <= NL ? NL / kVF : 1);  // lanes of a slot per head
  static constexpr int kHPL = !kValid ? 1 : (kVF <= NL ? 1 : kVF / NL);  // heads per lane
};

// The operand words of one key load: the raw words, or each fp8 word widened to two bf16 pairs.
template <int MODE, int LW, int OW>
__device__ __forceinline__ void key_words(const typename LoadOf<LW>::T &k, uint32_t (&op)[OW]) {
  constexpr int KW = LW / 4;
#pragma unroll
  for (int e = 0; e < KW; ++e) {
    const uint32_t w = word_of<LW>(k, e);
    if constexpr (MODE == kModeFp8Bf16) {
      op[2 * e] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, false));
      op[2 * e + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, true));
    } else {
      op[e] = w;
    }
  }
}

template <int OW>
__device__ __forceinline__ void load_words(const char *src, uint32_t (&w)[OW]) {
  if constexpr (OW % 4 == 0) {
#pragma unroll
    for (int v = 0; v < OW / 4; ++v) {
      const u32x4 x = *(const u32x4 *)(src + 16 * v);
#pragma unroll
      for (int e = 0; e < 4; ++e) w[4 * v + e] = x[e];
    }
  } else if constexpr (OW == 2) {
    const u32x2 x = *(const u32x2 *)src;
    w[0] = x[0];
    w[1] = x[1];
  } else {
    w[0] = *(const uint32_t *)src;
  }
}

template <int MODE, int HEAD_DIM, int NL, int GP, int LW>
__global__ __launch_bounds__(kValuThreads) void tile_lse_valu_layers_kernel(const Params p, const PlanView plan,
                                                                           const LayerSet ls) {
  using S = VShape<MODE, HEAD_DIM, NL, GP, LW>;
  static_assert(S::kValid, "invalid audit shape");
  constexpr int LPT = S::kLPT, TPI = S::kTPI, VF = S::kVF, OW = S::kOW, CT = S::kCT;
  constexpr int LPH = S::kLPH, HPL = S::kHPL;
  constexpr int NW = kValuThreads / kWave;
  using LT = typename LoadOf<LW>::T;

  __shared__ int s_next;
  __shared__ int s_pref[kMaxLaunchLayers + 1];  // items before each layer of the launch
  __shared__ unsigned long long s_cycles[kCycleSlots];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int groups = p.groups;
  const int grid = gridDim.x;
  const int nl = ls.n;
  auto split_of = [&](int j) { return (int)((blockIdx.x + (unsigned)j) % (unsigned)grid); };
  const uint32_t flag = __hip_atomic_load(p.flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int4 wg = plan.wg[blockIdx.x];
  int cnt = 0;  // wave 0: lane j holds layer j's split count
  if (wave == 0 && lane < nl) cnt = plan.wg[split_of(lane)].x;
  u32x4 d_lo;
  u32x2 d_hi;
  load_desc(plan.desc + (int64_t)blockIdx.x * plan.cap + min(groups == 1 ? wave : wave / groups, plan.cap - 1), d_lo,
            d_hi);
  if (flag == 0u) return;  // runtime/audit_kernel.py:64
  if (wave == 0) {
    const int inc = wave_inclusive_scan(min(cnt, plan.cap) * groups);
    if (lane < nl) s_pref[lane + 1] = inc;
    if (lane == 0) {
      s_pref[0] = 0;
      s_next = NW;
    }
  }
  if (p.cycles != nullptr)
    for (int k = threadIdx.x; k < kCycleSlots; k += kValuThreads) s_cycles[k] = 0ull;
  const int row0 = __builtin_amdgcn_readfirstlane(wg.y);  // the first split's first row: the timer slots' base
  __syncthreads();
  const int items = __builtin_amdgcn_readfirstlane(s_pref[nl]);

  const int slot = lane / LPT;  // token slot of a load instruction
  const int jc = lane % LPT;    // the lane's LW-byte column of the key row
  const int nsub = p.nsub;      // chunks per tile
  const int bs = p.block_size;
  const int G = p.group_rows;
  const bool by_row = ls.q_by_row != 0;
  const int64_t k_block = p.k_stride_block, k_pos = p.k_stride_pos, k_head = p.k_stride_head;
  const int64_t q_tok = p.q_stride_token, q_head = p.q_stride_head;
  const int64_t lane_off = (int64_t)slot * k_pos + jc * LW;

  struct Walk {
    int j, lo, hi;
  };
  auto walk_to = [&](Walk &w, int item) {
    while (item >= w.hi) {
      ++w.j;
      w.lo = w.hi;
      w.hi = __builtin_amdgcn_readfirstlane(s_pref[w.j + 1]);
    }
  };
  auto desc_of = [&](const Walk &w, int item) {
    return plan.desc + (int64_t)split_of(w.j) * plan.cap + (item - w.lo) / groups;
  };
  struct Layer {
    const char *q, *keys;
    float *lse;
    float scale;
    int group_first, q_head0;
  };
  auto layer_of = [&](int j) -> Layer {
    j = __builtin_amdgcn_readfirstlane(j);  // a uniform index: scalar loads of the kernel arguments
    return Layer{ls.l[j].q, ls.l[j].keys, ls.l[j].lse, ls.l[j].scale, ls.l[j].group_first, ls.l[j].q_head0};
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
    t.j = w.j;
    return t;
  };
  auto take = [&]() -> int {
    int v = 0;
    if (lane == 0) v = atomicAdd(&s_next, 1);
    return __builtin_amdgcn_readfirstlane(v);
  };
  // the query rows of the item's head: GP rows, zero past group_rows
  auto load_query = [&](uint32_t (&qw)[GP][OW], const Tile &T, const Layer &L) {
    const char *qbase = L.q + (int64_t)(by_row ? T.row : T.qtok) * q_tok +
                        (int64_t)((L.group_first + T.h) * G - L.q_head0) * q_head + (int64_t)jc * (OW * 4);
#pragma unroll
    for (int gg = 0; gg < GP; ++gg) {
      if (gg < G) {
        load_words<OW>(qbase + (int64_t)gg * q_head, qw[gg]);
      } else {
#pragma unroll
        for (int e = 0; e < OW; ++e) qw[gg][e] = 0u;
      }
    }
  };
  // chunk `sub` of tile T: instruction i reads tokens sub CT + i TPI .. + TPI, inside one block (TPI
  // divides the block size); past the row the tile's first block stands in, its scores masked
  auto load_chunk = [&](LT (&D)[NL], const Tile &T, const Layer &L, int sub) {
    const char *head = L.keys + (int64_t)(L.group_first + T.h) * k_head + lane_off;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int tpos = sub * CT + i * TPI;
      const int id = tpos < bs ? T.id0 : T.id1;
      D[i] = *(const LT *)(head + (int64_t)id * k_block + (int64_t)(tpos % bs) * k_pos);
    }
  };
  auto reduce_chunk = [&](const LT (&D)[NL], const uint32_t (&qw)[GP][OW], const Tile &T, const Layer &L, int sub,
                          float (&m_run)[HPL], float (&l_run)[HPL]) {
    float acc[GP * NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      uint32_t kw[OW];
      key_words<MODE, LW, OW>(D[i], kw);
#pragma unroll
      for (int gg = 0; gg < GP; ++gg) acc[gg * NL + i] = dot_words<MODE, OW>(qw[gg], kw);
    }
    transpose_reduce<GP * NL, LPT>(acc, lane);
    // acc[k] is the score of head (jc VF + k) / NL, instruction (jc VF + k) % NL
    float s[VF];
#pragma unroll
    for (int k = 0; k < VF; ++k) {
      const int i = (jc * VF + k) % NL;
      const int tok = sub * CT + i * TPI + slot;  // within the tile
      s[k] = tok < T.valid ? acc[k] * L.scale : -INFINITY;
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
      const float M = fmaxf(m_run[e], mx);
      if (M != -INFINITY) {
        const float a = m_run[e] == -INFINITY ? 0.0f : l_run[e] * exp2f((m_run[e] - M) * kLog2e);
        const float b = mx == -INFINITY ? 0.0f : sum * exp2f((mx - M) * kLog2e);
        l_run[e] = a + b;
        m_run[e] = M;
      }
    }
    if (sub == nsub - 1) {
      // the tile's record into each of its blocks the row reaches, runtime/audit_kernel.py:97-109
      if (slot == 0 && (jc % LPH) == 0) {
#pragma unroll
        for (int e = 0; e < HPL; ++e) {
          const int qr = (jc / LPH) * HPL + e;
          if (qr < G) {
#pragma unroll
            for (int b = 0; b < kTileBlocks; ++b) {
              if (b * bs < T.valid) {
                float *cell = L.lse + (int64_t)T.row * p.row_stride + T.h * G +
                              (int64_t)(T.k * kTileBlocks + b) * p.cells + qr;
                cell[0] = m_run[e];
                cell[p.plane_stride] = l_run[e];
              }
            }
          }
        }
      }
#pragma unroll
      for (int e = 0; e < HPL; ++e) {
        m_run[e] = -INFINITY;
        l_run[e] = 0.0f;
      }
    }
  };

  const bool timed = p.cycles != nullptr;
  // the timer: a run of one layer's, row's and head's tiles is timed once, where it ends
  auto time_tile = [&](const Tile &T, uint64_t &mark) {
    const uint64_t now = __builtin_amdgcn_s_memtime();
    if (T.h == 0 && T.row < p.cycles_rows && lane == 0) {
      const int r = T.row - row0;
      if (r >= 0 && r < kCycleSlots) atomicAdd(&s_cycles[r], (unsigned long long)(now - mark));
      else atomicAdd((unsigned long long *)(p.cycles + T.row), (unsigned long long)(now - mark));
    }
    mark = now;
  };

  if (wave < items) {
    Walk w{0, 0, __builtin_amdgcn_readfirstlane(s_pref[1])};
    if (wave >= w.hi) {  // a first layer with fewer items than waves: the wave's first item is later
      walk_to(w, wave);
      load_desc(desc_of(w, wave), d_lo, d_hi);
    }
    Tile T = describe(d_lo, d_hi, w, wave);
    Layer cur = layer_of(T.j);
    int ahead = take();
    if (ahead < items) {
      walk_to(w, ahead);
      load_desc(desc_of(w, ahead), d_lo, d_hi);
    }
    float m_run[HPL], l_run[HPL];
#pragma unroll
    for (int e = 0; e < HPL; ++e) {
      m_run[e] = -INFINITY;
      l_run[e] = 0.0f;
    }
    uint32_t qb[GP][OW], qn[GP][OW];
    load_query(qb, T, cur);
    LT A[NL], B[NL];
    if (T.valid > 0) load_chunk(A, T, cur, 0);
    int sub = 0;
    uint64_t mark = timed ? __builtin_amdgcn_s_memtime() : 0;
    // reduce the chunk in X after requesting the next one into Y; false after the wave's last chunk
    auto advance = [&](LT (&X)[NL], LT (&Y)[NL]) -> bool {
      Tile N = T;
      Layer next = cur;
      int nsub_next = sub + 1;
      bool more = true, new_query = false;
      if (nsub_next == nsub) {
        more = ahead < items;
        if (more) {
          N = describe(d_lo, d_hi, w, ahead);
          if (N.j != T.j) next = layer_of(N.j);
          nsub_next = 0;
          ahead = take();
          if (ahead < items) {
            walk_to(w, ahead);
            load_desc(desc_of(w, ahead), d_lo, d_hi);
          }
          new_query = N.row != T.row || N.h != T.h || N.j != T.j;
        }
      }
      if (more) {
        if (N.valid > 0) load_chunk(Y, N, next, nsub_next);  // a padding tile of the plan has no keys
        if (new_query) load_query(qn, N, next);
      }
      reduce_chunk(X, qb, T, cur, sub, m_run, l_run);
      if (timed && sub == nsub - 1 && (!more || new_query)) time_tile(T, mark);
      if (new_query) {
#pragma unroll
        for (int gg = 0; gg < GP; ++gg)
#pragma unroll
          for (int e = 0; e < OW; ++e) qb[gg][e] = qn[gg][e];
      }
      T = N;
      cur = next;
      sub = nsub_next;
      return more;
    };
    while (advance(A, B) && advance(B, A)) {
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

// ---------------------------------------------------------------------------------------
// The shape choice.  The VALU form takes what the MFMA form does not: fp32 keys, blocks of 8 tokens,
// and fp8 keys of 32 dimensions.  LW is the widest lane load that keeps one instruction inside a
// block; NL the instructions of a chunk (at most 8, inside a tile); GP the padded query rows, at least
// enough for the transpose reduction to leave every lane a score.
// ---------------------------------------------------------------------------------------
constexpr int kbytes_of(int mode) { return mode == kModeF32 ? 4 : (mode == kModeFp8Bf16 ? 1 : 2); }

constexpr bool mfma_shape(int mode, int hd, int bs) {
  const int tile = kTileBlocks * bs;
  if (mode == kModeF32 || tile % 32 != 0) return false;
  if (mode == kModeFp8Bf16) return hd == 64 || hd == 128 || hd == 256;
  return hd == 32 || hd == 64 || hd == 128 || hd == 256;
}

struct ValuConfig {
  int lw, nl, gp;  // 0: no kernel
};

// The lane width: the widest of 16, 8 and 4 bytes that keeps an instruction inside a block and the
// two query register sets (this item's and the next's, 2 GP OW words) within 128 VGPRs.  The
// instructions per chunk: at most 8, inside a tile, and as many as the registers left allow (the
// scores GP NL, two chunks 2 NL LW / 4); GP grows (or, at 16, NL) until the reduction leaves every
// lane a score.
constexpr ValuConfig valu_config(int mode, int hd, int bs, int group_rows) {
  const int row = hd * kbytes_of(mode);
  const int gp0 = group_rows <= 4 ? 4 : (group_rows <= 8 ? 8 : 16);
  int lw = 0, fallback = 0;
  for (int w = 16; w >= 4; w /= 2) {
    if (row % w != 0 || row / w < 1 || row / w > kWave || kWave / (row / w) > bs) continue;
    const int ow = mode == kModeFp8Bf16 ? w / 2 : w / 4;
    if (fallback == 0) fallback = w;
    if (2 * gp0 * ow <= 128) {
      lw = w;
      break;
    }
  }
  if (lw == 0) lw = fallback;
  if (lw == 0) return ValuConfig{0, 0, 0};
  const int lpt = row / lw, tpi = kWave / lpt, kw = lw / 4;
  const int ow = mode == kModeFp8Bf16 ? 2 * kw : kw;
  const int nl_max = kTileBlocks * bs / tpi >= 8 ? 8 : kTileBlocks * bs / tpi;
  int budget = (192 - 2 * gp0 * ow) / (gp0 + 2 * kw);
  if (budget < 1) budget = 1;
  int nl = 1;
  while (2 * nl <= nl_max && 2 * nl <= budget) nl *= 2;
  int gp = gp0;
  while (nl * gp < lpt) {
    if (gp < 16) gp *= 2;
    else if (nl < nl_max) nl *= 2;
    else return ValuConfig{0, 0, 0};
  }
  return ValuConfig{lw, nl, gp};
}

// whether (MODE, HD, NL, GP, LW) is chosen for some block size of 8 to 128 tokens and some group
constexpr bool reachable(int mode, int hd, int nl, int gp, int lw) {
  for (int bs = 8; bs <= 128; bs *= 2) {
    if (mfma_shape(mode, hd, bs)) continue;
    for (int g = 1; g <= 16; ++g) {
      const ValuConfig c = valu_config(mode, hd, bs, g);
      if (c.lw == lw && c.nl == nl && c.gp == gp) return true;
    }
  }
  return false;
}

using ValuFn = void (*)(const Params, const PlanView, const LayerSet);

template <int MODE, int HD, int NL, int GP, int LW>
ValuFn valu_if_reachable() {
  if constexpr (reachable(MODE, HD, NL, GP, LW) && VShape<MODE, HD, NL, GP, LW>::kValid)
    return tile_lse_valu_layers_kernel<MODE, HD, NL, GP, LW>;
  else
    return nullptr;
}

template <int MODE, int HD, int NL, int GP>
ValuFn valu_pick_lw(int lw) {
  switch (lw) {
    case 16: return valu_if_reachable<MODE, HD, NL, GP, 16>();
    case 8: return valu_if_reachable<MODE, HD, NL, GP, 8>();
    case 4: return valu_if_reachable<MODE, HD, NL, GP, 4>();
  }
  return nullptr;
}

template <int MODE, int HD, int NL>
ValuFn valu_pick_gp(int gp, int lw) {
  switch (gp) {
    case 4: return valu_pick_lw<MODE, HD, NL, 4>(lw);
    case 8: return valu_pick_lw<MODE, HD, NL, 8>(lw);
    case 16: return valu_pick_lw<MODE, HD, NL, 16>(lw);
  }
  return nullptr;
}

template <int MODE, int HD>
ValuFn valu_pick_nl(int nl, int gp, int lw) {
  switch (nl) {
    case 1: return valu_pick_gp<MODE, HD, 1>(gp, lw);
    case 2: return valu_pick_gp<MODE, HD, 2>(gp, lw);
    case 4: return valu_pick_gp<MODE, HD, 4>(gp, lw);
    case 8: return valu_pick_gp<MODE, HD, 8>(gp, lw);
  }
  return nullptr;
}

template <int MODE>
ValuFn valu_pick_hd(int hd, int nl, int gp, int lw) {
  switch (hd) {
    case 32: return valu_pick_nl<MODE, 32>(nl, gp, lw);
    case 64: return valu_pick_nl<MODE, 64>(nl, gp, lw);
    case 128: return valu_pick_nl<MODE, 128>(nl, gp, lw);
    case 256: return valu_pick_nl<MODE, 256>(nl, gp, lw);
  }
  return nullptr;
}

ValuFn valu_pick(int mode, int hd, int bs, int group_rows) {
  if (bs <= 0 || mfma_shape(mode, hd, bs)) return nullptr;
  const ValuConfig c = valu_config(mode, hd, bs, group_rows);
  if (c.lw == 0) return nullptr;
  switch (mode) {
    case kModeF32: return valu_pick_hd<kModeF32>(hd, c.nl, c.gp, c.lw);
    case kModeF16: return valu_pick_hd<kModeF16>(hd, c.nl, c.gp, c.lw);
    case kModeBF16: return valu_pick_hd<kModeBF16>(hd, c.nl, c.gp, c.lw);
    case kModeFp8Bf16: return valu_pick_hd<kModeFp8Bf16>(hd, c.nl, c.gp, c.lw);
  }
  return nullptr;
}

bool valu_planned_shape(int mode, int head_dim, int block_size) {
  return valu_pick(mode, head_dim, block_size, 1) != nullptr;
}

int valu_planned_nsub(int mode, int head_dim, int block_size, int group_rows) {
  const ValuConfig c = valu_config(mode, head_dim, block_size, group_rows);
  if (c.lw == 0) return 0;
  const int tpi = kWave / (head_dim * kbytes_of(mode) / c.lw);
  return kTileBlocks * block_size / (c.nl * tpi);
}

int launch_valu_layers(int mode, int head_dim, int block_size, int group_rows, const Params &p, const PlanView &plan,
                       const LayerSet &ls, int grid, hipStream_t stream, const char *what) {
  const ValuFn fn = valu_pick(mode, head_dim, block_size, group_rows);
  if (fn == nullptr)
    return fail(EKV_EUNSUPPORTED, "%s: no VALU kernel for dtype mode %d, head_dim %d, block size %d", what, mode,
                head_dim, block_size);
  hipLaunchKernelGGL(fn, dim3(grid), dim3(kValuThreads), 0, stream, p, plan, ls);
  return check_hip(hipGetLastError(), what);
}

}  // namespace audit
}  // namespace ekv
