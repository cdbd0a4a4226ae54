// The `sum` and `maxmin` budget splits across requests, on the device.
// Semantics: allocate(..., "sum" | "maxmin"), observe/allocation.py:55-166, with Request.shares
// and pinned_mask (observe/allocation.py:39-52).
//
// Every request's shares are max(s, 0) / total in float64, total being NumPy's sum of the clamped
// scores (equal shares 1 / n when total <= 0).  The totals are reproduced bit for bit: NumPy adds
// the pairwise sums of successive runs of at most 8192 values (its reduction buffer) to 0.0, a
// run's pairwise sum taking pieces of at most 128 values with eight accumulators and splitting
// longer pieces at n / 2 rounded down to a multiple of 8 (NumPy's published pairwise summation,
// numpy/_core/src/umath/loops_utils.h.src; checked against NumPy 2.2.6) -- which a wave evaluates
// with the leaves summed in parallel and combined in the recursion's order.
//
// sum: keep the `free` unpinned blocks of highest weight * share, a tie going to the newer block,
// then to the earlier request.  The threshold is found by a radix select over order-preserving
// 64-bit keys of the float64 gains (six passes of 11-bit digits over every open block, the gains
// recomputed in each pass), then among the blocks at the threshold by a select over the 30-bit
// (block desc, request asc) key (three passes).  A pass stops the select once the free blocks end at
// a bucket's end, and each pass's last workgroup picks its digit.  All state lives in a
// caller-provided workspace that the budget kernel clears first, so the launches need no host
// synchronisation and no memset.
//
// maxmin: raise the lowest retained share as far as the budget allows, then spend what is left on
// the lowest request first (observe/allocation.py:126-166).  Per request: the pinned shares' NumPy
// sum (base), its open blocks in stable descending share order (a radix sort over the same
// order-preserving keys, one workgroup per request, in LDS; past 12288 blocks in global memory), and
// their running float64 totals, added in that order as np.cumsum does.  The 60-step bisection of the level: a request's count at a level is
// min(1 + lower_bound(totals + 2 r, level - base - 1e-12 + 2 r), open), the shifted-by-2r comparison
// NumPy's single search makes.  Its first 20 steps are walks over counts that two kernels sum over
// every CU at the levels they can reach; the rest run in one workgroup, every request keeping the
// bracket of positions its count can still take.  The leftover goes to the requests tied at the
// lowest (retained share, index) level, a pass at a time, as the reference's heap hands it out.
#pragma clang fp contract(off)

#include <limits.h>
#include <math.h>

#include <algorithm>


#include "ekv_common.hpp"
#include "ekv_pairwise.hpp"

namespace ekv {
namespace alloc {

constexpr int kThreads = 256;
constexpr int kMaxWidth = 12288;          // maxmin: a request sorted in one workgroup's LDS
constexpr int kMaxMaxminWidth = 1 << 18;  // maxmin: positions in 16 bits up to 65535 blocks, 32 past it
constexpr int kMaxSumWidth = 1 << 18;     // sum: the per-row loops stream the row; the tie key's block field
constexpr int kMaxRows = (1 << 24) - 1;  // the tie key holds the request in 16 to 24 bits

enum Mode : int { kSelect = 0, kKeepAll = 1, kKeepOpen = 2, kPinnedOnly = 3 };

constexpr int kDigitBits = 11;  // radix digits of the select: six gain passes and three tie passes
constexpr int kBins = 1 << kDigitBits;

struct State {
  unsigned long long hist[kBins];
  unsigned long long prefix, mask, threshold;  // threshold: the gain key at the cut
  long long k_rem, free_blocks, must, sizes, open_total, requests, budget;
  int mode, error;
  // the select ended early: the free blocks end exactly at the end of a digit's bucket, so every
  // key with that prefix is kept and the later passes have nothing to rank (done_tie: in a pass
  // over the tie key, among the blocks at the gain threshold)
  int done, done_tie;
  int arrivals;  // a pass's workgroups that have flushed their histogram (0 between passes)
  int done_first;  // the select ended at the first pass: the second did not run (nor write its keeps)
};

struct RowStat {
  double total;  // NumPy's sum of the clamped scores
  int n, pinned, open, pad;
};

struct Params {
  const double *scores;
  int64_t scores_stride;
  const int32_t *blocks;
  const double *weights;  // per request, or null (1.0)
  const uint8_t *pinned;
  int64_t pinned_stride;
  int32_t rows, width;
  long long budget;
  uint8_t *keep;
  int64_t keep_stride;
  int64_t *summary;
  State *state;
  RowStat *row_stat;
  // sum: the open blocks whose gain key matched the first pass's digit, as (gain key, tie key) pairs,
  // listed by the second pass so that the later passes read them alone: each workgroup of the passes
  // lists its rows' blocks in its own region of `cand` (cand_region) and their number in cand_count
  unsigned long long *cand;
  unsigned int *cand_count;  // [workgroups of the passes]
  // the controller's rule (ekv_controller_keep): budget < 0 takes max(pinned, ceil(fraction * blocks))
  // over every block of the measured rows, from `ctl`, which also holds the request count
  double fraction;
  const struct CtlHeader *ctl;
  int32_t tie_rbits;  // the request's bits in the tie key: 16, or as many as the request count needs
};

// Written by ctl_plan_kernel: the measured rows' blocks (freed ones included) and their count.
struct CtlHeader {
  long long blocks;
  long long requests;
};

__device__ __forceinline__ int row_blocks(const Params &p, int r) { return min(max(p.blocks[r], 0), p.width); }

// Request.pinned_mask: the explicit mask, else the first and the last block
__device__ __forceinline__ bool pinned_at(const Params &p, int r, int b, int n) {
  if (p.pinned != nullptr) return p.pinned[(int64_t)r * p.pinned_stride + b] != 0;
  return b == 0 || b == n - 1;
}

// order-preserving key of a float64 gain: larger gain, larger key; both zeros one key; NaN the
// lowest key (1); key 0 marks a block that is not open
__device__ __forceinline__ unsigned long long gain_key(double g) {
  if (g != g) return 1ull;
  if (g == 0.0) g = 0.0;
  const unsigned long long bits = __builtin_bit_cast(unsigned long long, g);
  const unsigned long long k = (bits >> 63) ? ~bits : (bits | (1ull << 63));
  return k < 2ull ? 2ull : k;  // keep 0 and 1 free (only the most negative NaN-free values would map there)
}

// the float64 value of a key (both zeros decode to +0.0, which every comparison and sum treats
// as -0.0; key 1, NaN, decodes to NaN)
__device__ __forceinline__ double key_value(unsigned long long k) {
  if (k == 1ull) return __builtin_nan("");
  const unsigned long long bits = (k >> 63) ? (k & ~(1ull << 63)) : ~k;
  return __builtin_bit_cast(double, bits);
}

__device__ __forceinline__ double share_value(const RowStat &st, double score) {
  if (!(st.total > 0.0) && st.total == st.total) return 1.0 / (double)max(st.n, 1);  // total <= 0
  return clamp0(score) / st.total;
}
__device__ __forceinline__ double share_of(const Params &p, const RowStat &st, int r, int b) {
  return share_value(st, p.scores[(int64_t)r * p.scores_stride + b]);
}

// A row's blocks b0 + NT u (u < U) for one thread of NT: the scores and pinned flags loaded
// together before any is used (one memory latency per U blocks, not per block).  PIN: the pinned
// flags come from the caller's mask (p.pinned), else they are the row's first and last block.
template <int U, int NT, bool PIN>
struct BlockRun {
  double score[U];
  uint32_t pinned = 0, inside = 0;
  __device__ __forceinline__ void load(const Params &p, int r, int b0, int n) {
    const double *srow = p.scores + (int64_t)r * p.scores_stride;
    const uint8_t *prow = PIN ? p.pinned + (int64_t)r * p.pinned_stride : nullptr;
    uint8_t pin[U];
    // every load issued, the blocks past the row reading its block 0 (a row holds `width` >= 1
    // blocks): a load under a condition is followed by a wait for every load before it
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = b0 + u * NT;
      const int at = b < n ? b : 0;
      const double x = srow[at];
      score[u] = b < n ? x : 0.0;
      if constexpr (PIN) pin[u] = prow[at];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = b0 + u * NT;
      inside |= b < n ? (1u << u) : 0u;
      bool pn;
      if constexpr (PIN) pn = pin[u] != 0;
      else pn = b == 0 || b == n - 1;
      pinned |= (b < n && pn) ? (1u << u) : 0u;
    }
  }
};
constexpr int kRun = 8;  // blocks per thread per step of the per-row loops

__device__ __forceinline__ double weight_of(const Params &p, int r) { return p.weights != nullptr ? p.weights[r] : 1.0; }

// one workgroup per request: its total, its pinned and open blocks
constexpr int kPrepThreads = 256;
__global__ __launch_bounds__(kPrepThreads) void prepare_kernel(const Params p) {
  __shared__ PairwiseLds s_sum;
  __shared__ int s_red[kPrepThreads / kWave];
  const int r = blockIdx.x;
  const int n = row_blocks(p, r);
  const double *srow = p.scores + (int64_t)r * p.scores_stride;
  const double total = block_numpy_sum<kPrepThreads>([&](int i) { return clamp0(srow[i]); }, n, s_sum);
  int pinned = 0;
  if (p.pinned == nullptr) {
    pinned = threadIdx.x == 0 ? min(n, 2) : 0;  // the first and the last block
  } else {
    const uint8_t *prow = p.pinned + (int64_t)r * p.pinned_stride;
    for (int b0 = threadIdx.x; b0 < n; b0 += 8 * kPrepThreads) {
      uint8_t f[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) f[u] = b0 + u * kPrepThreads < n ? prow[b0 + u * kPrepThreads] : 0;
#pragma unroll
      for (int u = 0; u < 8; ++u) pinned += f[u] != 0 ? 1 : 0;
    }
  }
  pinned = block_sum<kPrepThreads>(pinned, s_red);
  if (threadIdx.x == 0) {
    RowStat st;
    st.total = total;
    st.n = n;
    st.pinned = pinned;
    st.open = n - pinned;
    st.pad = 0;
    p.row_stat[r] = st;
  }
}

// the requests' pinned, existing and open blocks, summed over the rows' statistics by one
// workgroup, then the budget's mode (allocation.py:57-76) and the select's start; the state
// (histogram, flags, counters) is cleared first
template <int NT>
__device__ void decide(const Params &p) {
  __shared__ long long s_red[3][NT / kWave];
  {
    unsigned long long *w = (unsigned long long *)p.state;
    for (int i = threadIdx.x; i < (int)(sizeof(State) / 8); i += NT) w[i] = 0ull;
  }
  long long v[3] = {0, 0, 0};  // must, sizes, open_total
  for (int r = threadIdx.x; r < p.rows; r += NT) {
    const RowStat st = p.row_stat[r];
    v[0] += st.pinned;
    v[1] += st.n;
    v[2] += st.open;
  }
  const int wave = threadIdx.x / kWave;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    v[k] = wave_sum_i64(v[k]);
    if (lane_id() == 0) s_red[k][wave] = v[k];
  }
  __syncthreads();  // also orders the clearing stores before thread 0's
  if (threadIdx.x != 0) return;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    v[k] = 0;
    for (int w = 0; w < NT / kWave; ++w) v[k] += s_red[k][w];
  }
  State *s = p.state;
  s->must = v[0];
  s->sizes = v[1];
  s->open_total = v[2];
  const long long requests = p.ctl != nullptr ? p.ctl->requests : p.rows;
  s->requests = requests;
  const long long must = v[0], sizes = v[1];
  long long budget = p.budget;
  if (budget < 0) {  // controller.py:435-437
    const long long want = (long long)ceil(p.fraction * (double)p.ctl->blocks);
    budget = want > must ? want : must;
  }
  s->budget = budget;
  s->error = (must > budget && budget < sizes) ? 1 : 0;
  const long long free_blocks = budget - must;
  s->free_blocks = free_blocks;
  int mode;
  if (budget >= sizes) mode = kKeepAll;
  else if (free_blocks <= 0) mode = kPinnedOnly;
  else if (free_blocks >= v[2]) mode = kKeepOpen;
  else mode = kSelect;
  s->mode = mode;
  s->k_rem = free_blocks;
  s->prefix = 0ull;
  s->mask = 0ull;
  if (p.summary != nullptr) {
    p.summary[0] = budget;
    p.summary[1] = sizes;
    p.summary[2] = must;
    p.summary[3] = s->error;
    p.summary[4] = requests;
    p.summary[5] = free_blocks;
  }
}
__global__ __launch_bounds__(kThreads) void decide_kernel(const Params p) { decide<kThreads>(p); }

// the select's two keys of an open block
__device__ __forceinline__ unsigned long long key_at(const Params &p, const RowStat &st, int r, int b) {
  return gain_key(weight_of(p, r) * share_of(p, st, r, b));
}
__device__ __forceinline__ unsigned long long tie_key(const Params &p, int r, int b) {
  const unsigned long long rmask = (1ull << p.tie_rbits) - 1ull;  // newer block, then earlier request
  return ((unsigned long long)b << p.tie_rbits) | (rmask - (unsigned long long)r);
}
// the tie key's request bits: 16 up to 65536 requests, else as many as the last request's index needs
inline int tie_request_bits(int rows) {
  int bits = 16;
  while (bits < 24 && rows > (1 << bits)) ++bits;
  return bits;
}
// the tie key's width: the request's bits below the block's (14 up to 16384 blocks, else 18)
inline int tie_bits(int width, int rbits) { return (width <= (1 << 14) ? 14 : 18) + rbits; }

// The digit where the k_rem-th largest key lies, and the next pass's prefix, from the pass's
// histogram: thread t holds the kBins / NT digits below kBins - (kBins / NT) t, in
// descending order (NT threads).  The histogram is read with device-coherent loads (the pass's workgroups added
// into it with device-scope atomics from every XCD) and cleared for the next pass.
template <int NT>
__device__ void pick_digit(const Params &p, int shift, int bits, int last_gain_pass, bool first_pass) {
  constexpr int kPer = kBins / NT;
  __shared__ long long s_scan[NT / kWave];
  __shared__ int s_whole;
  State *s = p.state;
  const int t = threadIdx.x;
  if (t == 0) s_whole = 0;
  long long h[kPer], mine = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    h[i] = (long long)__hip_atomic_load(&s->hist[kBins - 1 - (kPer * t + i)], __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
    mine += h[i];
  }
  // inclusive scan over the threads: the keys at digits >= this thread's lowest
  const int lane = lane_id(), wave = t / kWave;
  long long inc = mine;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const long long up = __shfl_up(inc, d, kWave);
    if (lane >= d) inc += up;
  }
  if (lane == kWave - 1) s_scan[wave] = inc;
  __syncthreads();
  long long base = 0;
  for (int w = 0; w < wave; ++w) base += s_scan[w];
  inc += base;
  long long before = inc - mine;
  const long long k_rem = s->k_rem;
  __syncthreads();
  if (before < k_rem && inc >= k_rem) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      if (before < k_rem && before + h[i] >= k_rem) {
        s->prefix |= (unsigned long long)(kBins - 1 - (kPer * t + i)) << shift;
        s->k_rem = k_rem - before;
        if (before + h[i] == k_rem) s_whole = 1;  // the bucket ends the free blocks
      }
      before += h[i];
    }
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) s->hist[kBins - 1 - (kPer * t + i)] = 0ull;
  __syncthreads();
  if (t == 0) {
    s->mask |= ((1ull << bits) - 1ull) << shift;
    if (s_whole) {
      s->done = 1;
      s->done_first = first_pass ? 1 : 0;
      s->done_tie = last_gain_pass < 0 ? 1 : 0;
    } else if (last_gain_pass > 0) {  // the gain threshold is complete: the tie passes start
      s->threshold = s->prefix;
      s->prefix = 0ull;
      s->mask = 0ull;
    }
  }
}

// One radix pass: the histogram of the `bits`-wide digit at `shift` over the open blocks whose key
// matches the prefix so far (tie passes: the blocks at the gain threshold, over the tie key).
// Workgroup w takes rows w, w + grid, ..., so each workgroup adds its LDS histogram into the global
// one once, with device-scope atomics; once they have completed it counts its arrival, and the
// pass's last workgroup picks the digit (pick_digit), so no second kernel runs per pass.
// last_gain_pass: 1 on the last gain pass, 0 on the others, -1 on tie passes.
// CAND_MODE: 1 (the second gain pass) also lists the blocks it counts, every one matching the first
// pass's digit, in p.cand; 2 (the later passes) reads that list instead of the rows, unless it
// outgrew its capacity.
constexpr int kCandPerRow = 1024;  // the list's room per request row
// The passes run one workgroup of kHistThreads per CU at most (rows w, w + grid, ... each): a pass's
// workgroups each add their histogram into the global one, and the adds to one digit from every
// workgroup are serialised in memory, so fewer, larger workgroups end the pass sooner.
constexpr int kHistThreads = 1024;

// Workgroup w of a pass takes rows w, w + grid, ...: its region of the list holds kCandPerRow pairs
// for each of them, after the regions of the workgroups before it.
__device__ __forceinline__ void cand_region(int rows, int w, int grid, long long &first, int &room) {
  const int per = rows / grid, extra = rows % grid;
  first = (long long)kCandPerRow * ((long long)w * per + min(w, extra));
  room = kCandPerRow * (per + (w < extra ? 1 : 0));
}

constexpr int kHistRows = 2;  // rows whose blocks a pass's workgroup loads together

template <bool TIE, int CAND_MODE, bool PIN>
__global__ __launch_bounds__(kHistThreads) void hist_kernel(const Params p, int shift, int bits, int last_gain_pass) {
  constexpr int cand_mode = CAND_MODE;
  __shared__ unsigned int s_hist[kBins];
  __shared__ int s_last;
  __shared__ unsigned int s_listed;
  State *s = p.state;
  if (s->mode != kSelect || s->error || s->done) return;
  for (int i = threadIdx.x; i < kBins; i += kHistThreads) s_hist[i] = 0u;
  if (threadIdx.x == 0) s_listed = 0u;
  __syncthreads();
  long long region;
  int room;
  cand_region(p.rows, blockIdx.x, gridDim.x, region, room);
  const unsigned int digit_mask = (1u << bits) - 1u;
  const unsigned long long prefix = s->prefix, mask = s->mask, threshold = s->threshold;
  const int lane = lane_id();
  // one key per lane of the wave, every lane taking part: when every counting lane has one digit
  // (the first passes), one add for all
  auto count = [&](bool counted, unsigned int digit) {
    const uint64_t active = __ballot(counted);
    if (active == 0) return;
    const unsigned int lead = (unsigned int)__builtin_amdgcn_readlane((int)digit, __ffsll((long long)active) - 1);
    const bool same = __ballot(counted && digit == lead) == active;
    if (counted) {
      if (same) {
        if (lane == __ffsll((long long)active) - 1) atomicAdd(&s_hist[lead], (unsigned int)__popcll(active));
      } else {
        atomicAdd(&s_hist[digit], 1u);
      }
    }
  };
  // which of a key's gain and tie key is ranked, and its digit when it matches the prefix
  auto consider = [&](unsigned long long k, unsigned long long tk, unsigned int &digit) {
    unsigned long long key = k;
    bool take = true;
    if constexpr (TIE) {
      take = k == threshold;
      key = tk;
    }
    const bool counted = take && (key & mask) == prefix;
    digit = (unsigned int)(key >> shift) & digit_mask;
    return counted;
  };
  const unsigned int listed = cand_mode == 2 ? p.cand_count[blockIdx.x] : 0u;
  if (cand_mode == 2 && listed <= (unsigned int)room) {  // this workgroup's list (else its rows again)
    const unsigned long long *list = p.cand + 2 * region;
    for (int c0 = 0; c0 < (int)listed; c0 += kHistThreads) {
      const int c = c0 + threadIdx.x;
      unsigned int digit = 0u;
      const bool counted = c < (int)listed && consider(list[2 * c], list[2 * c + 1], digit);
      count(counted, digit);
    }
  } else {
    // rows w, w + G, ... kHistRows at a time: every row's blocks of a step loaded before any is
    // counted (a step's list stores then wait for no load of the same step).  The second pass also
    // writes the keep of every block the first digit decides (pinned and past-the-row blocks 1, an
    // open block 1 or 0 as its digit is above or below the threshold's), across the whole width, and
    // leaves the blocks it lists to the keep kernel.
    const int G = gridDim.x;
    for (int r0 = blockIdx.x; r0 < p.rows; r0 += kHistRows * G) {
      int rr[kHistRows], nmax = 0;
      RowStat st[kHistRows];
      double weight[kHistRows];
#pragma unroll
      for (int i = 0; i < kHistRows; ++i) {
        const bool real = r0 + i * G < p.rows;
        rr[i] = real ? r0 + i * G : r0;  // a row past the last reads row r0's first block, counts nothing
        st[i] = p.row_stat[rr[i]];
        if (!real) st[i].n = 0;
        weight[i] = weight_of(p, rr[i]);
        nmax = max(nmax, st[i].n);
      }
      const int steps_to = cand_mode == 1 ? p.width : nmax;
      for (int c0 = 0; c0 < steps_to; c0 += kHistThreads * kRun) {
        BlockRun<kRun, kHistThreads, PIN> run[kHistRows];
#pragma unroll
        for (int i = 0; i < kHistRows; ++i) run[i].load(p, rr[i], c0 + threadIdx.x, st[i].n);
#pragma unroll
        for (int i = 0; i < kHistRows; ++i) {
#pragma unroll
          for (int u = 0; u < kRun; ++u) {
            const int b = c0 + threadIdx.x + u * kHistThreads;
            bool counted = false;
            unsigned int digit = 0u;
            unsigned long long k = 0ull;
            if (((run[i].inside & ~run[i].pinned) >> u) & 1u) {
              k = gain_key(weight[i] * share_value(st[i], run[i].score[u]));
              counted = consider(k, tie_key(p, rr[i], b), digit);
            }
            count(counted, digit);
            if constexpr (cand_mode == 1) {  // list the counted blocks: one slot reservation (in LDS) per wave
              const uint64_t active = __ballot(counted);
              if (active != 0) {
                const int first = __ffsll((long long)active) - 1;
                unsigned int at = 0u;
                if (lane == first) at = atomicAdd(&s_listed, (unsigned int)__popcll(active));
                at = (unsigned int)__shfl((int)at, first) +
                     __builtin_amdgcn_mbcnt_hi((uint32_t)(active >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)active, 0u));
                if (counted && at < (unsigned int)room) {
                  p.cand[2 * (region + at)] = k;
                  p.cand[2 * (region + at) + 1] = tie_key(p, rr[i], b);
                }
              }
              if (b < p.width && !counted && rr[i] == r0 + i * G) {
                const bool open = ((run[i].inside & ~run[i].pinned) >> u) & 1u;
                const uint8_t kv = !open || (k & mask) > prefix ? 1 : 0;
                p.keep[(int64_t)rr[i] * p.keep_stride + b] = kv;
              }
            }
          }
        }
      }
    }
  }
  __syncthreads();
  if constexpr (cand_mode == 1)
    if (threadIdx.x == 0) p.cand_count[blockIdx.x] = s_listed;  // may pass the room
  for (int i = threadIdx.x; i < kBins; i += kHistThreads) {
    const unsigned int c = s_hist[i];
    if (c) __hip_atomic_fetch_add(&s->hist[i], (unsigned long long)c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's adds have completed
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(&s->arrivals, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (int)gridDim.x - 1;
  __syncthreads();
  if (!s_last) return;
  if (threadIdx.x == 0) s->arrivals = 0;
  pick_digit<kHistThreads>(p, shift, bits, last_gain_pass, cand_mode == 0);
}

// The keep, on the passes' grid.  When the second pass ran, it has written every keep but those of
// the blocks it listed, and a workgroup writes its list's; otherwise (another mode, an error, a
// select that ended at the first pass) or when its list outgrew its room, the workgroup writes every
// block of its rows.
template <bool PIN>
__global__ __launch_bounds__(kHistThreads) void sum_keep_kernel(const Params p) {
  const State *s = p.state;
  const int mode = s->mode;
  const bool error = s->error != 0;
  const unsigned long long threshold = s->threshold, prefix = s->prefix, mask = s->mask;
  const bool done_gain = s->done && !s->done_tie;
  auto selected = [&](unsigned long long key, unsigned long long tk) -> uint8_t {
    if (done_gain) return (key & mask) >= prefix ? 1 : 0;  // every key from the last bucket on
    return (key > threshold || (key == threshold && (tk & mask) >= prefix)) ? 1 : 0;
  };
  long long region;
  int room;
  cand_region(p.rows, blockIdx.x, gridDim.x, region, room);
  const bool second_ran = mode == kSelect && !error && !s->done_first;
  const unsigned int listed = second_ran ? p.cand_count[blockIdx.x] : 0u;
  if (second_ran && listed <= (unsigned int)room) {
    const unsigned long long *list = p.cand + 2 * region;
    for (int c = threadIdx.x; c < (int)listed; c += kHistThreads) {
      const unsigned long long key = list[2 * c], tk = list[2 * c + 1];
      const unsigned long long rmask = (1ull << p.tie_rbits) - 1ull;
      const int r = (int)(rmask - (tk & rmask)), b = (int)(tk >> p.tie_rbits);
      p.keep[(int64_t)r * p.keep_stride + b] = selected(key, tk);
    }
    return;
  }
  for (int r = blockIdx.x; r < p.rows; r += gridDim.x) {
    const RowStat st = p.row_stat[r];
    const double weight = weight_of(p, r);
    uint8_t *krow = p.keep + (int64_t)r * p.keep_stride;
    for (int b0 = threadIdx.x; b0 - (int)threadIdx.x < p.width; b0 += kHistThreads * kRun) {
      BlockRun<kRun, kHistThreads, PIN> run;
      run.load(p, r, b0, st.n);
#pragma unroll
      for (int u = 0; u < kRun; ++u) {
        const int b = b0 + u * kHistThreads;
        if (b >= p.width) continue;
        uint8_t k;
        if (error || b >= st.n || mode == kKeepAll || ((run.pinned >> u) & 1u)) k = 1;
        else if (mode == kKeepOpen) k = 1;
        else if (mode == kPinnedOnly) k = 0;
        else k = selected(gain_key(weight * share_value(st, run.score[u])), tie_key(p, r, b));
        krow[b] = k;
      }
    }
  }
}

// ---- maxmin --------------------------------------------------------------------------------
constexpr int kBisectThreads = 1024;
constexpr int kMaxMaxminRegRows = kBisectThreads * 8;  // at most 8 requests per bisection thread in registers
constexpr int kMaxMaxminRows = (1 << 24) - 1;          // requests (past kMaxMaxminRegRows: the bisection state in memory)

struct MaxminRow {
  double base;  // NumPy's sum of the pinned shares
  int open, counts;
};

struct MaxminParams {
  Params p;
  MaxminRow *mrow;
  int32_t *vals_out;  // per request, its blocks' indices in sorted order
  double *prefix;     // per request, the running totals of its open shares in that order
  int32_t *order;     // the requests, longest first: the sorting workgroups' order
  int32_t *level_count;  // per level j / kLevels, the requests' counts summed
  void *level_pos;       // per request and level j / kLevels, its position there (16 or 32 bits: pos32)
  int32_t *level_count2;  // the second pass: per level low + j / kLevels^2 inside the first walk's bracket
  void *level_pos2;       // per request and such level, its position there
  int32_t pos32;          // positions in 32 bits (rows wider than 65535 blocks)
  // more requests than the bisection's registers hold (mm_bisect_mem_kernel): each request's
  // bracket, counts there and at the step's mid, and its count and retained share, in memory
  int32_t *b_lo, *b_hi, *b_flo, *b_fhi, *b_fmid, *b_pmid, *b_count;
  double *b_retained;
  // requests wider than a sort in LDS (width > kMaxWidth): the sort's second buffer, [rows][width]
  unsigned long long *keys_in;
};

// the bisection's first kLevelBits steps can only reach the levels j / 2^kLevelBits (0 < j < 2^kLevelBits,
// every one exact in float64, as are the steps' mids (low + high) / 2 on the way there)
constexpr int kLevelBits = 10;
constexpr int kLevels = 1 << kLevelBits;

// a stored level position of request r at level j (the arrays hold rows x kLevels entries)
__device__ __forceinline__ int pos_at(const MaxminParams &m, const void *a, int r, int j) {
  const int64_t i = (int64_t)r * kLevels + j;
  return m.pos32 ? (int)reinterpret_cast<const uint32_t *>(a)[i] : (int)reinterpret_cast<const uint16_t *>(a)[i];
}
__device__ __forceinline__ void set_pos(const MaxminParams &m, void *a, int r, int j, int v) {
  const int64_t i = (int64_t)r * kLevels + j;
  if (m.pos32) reinterpret_cast<uint32_t *>(a)[i] = (uint32_t)v;
  else reinterpret_cast<uint16_t *>(a)[i] = (uint16_t)v;
}


// per request, one wave: NumPy's sum of the pinned shares (the base) and the request's counts.  The
// pinned blocks are listed in order first: in LDS, or for rows wider than it holds (WIDE) in the
// request's row of vals_out, which the sort overwrites afterwards.
template <bool WIDE>
__global__ __launch_bounds__(kWave) void mm_base_kernel(const MaxminParams m) {
  __shared__ int s_start[kMaxLeaves], s_len[kMaxLeaves];
  __shared__ double s_leaf[kMaxLeaves];
  __shared__ unsigned short s_pin[WIDE ? 1 : kMaxWidth];  // the pinned blocks, in order
  const Params &p = m.p;
  const int r = blockIdx.x;
  const int lane = lane_id();
  const RowStat st = p.row_stat[r];
  int32_t *g_pin = m.vals_out + (int64_t)r * p.width;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int npin = 0;
  for (int b0 = 0; b0 < st.n; b0 += kWave) {
    const int b = b0 + lane;
    const bool pin = b < st.n && pinned_at(p, r, b, st.n);
    const uint64_t mask = __ballot(pin);
    if (pin) {
      if constexpr (WIDE) g_pin[npin + __popcll(mask & below)] = b;
      else s_pin[npin + __popcll(mask & below)] = (unsigned short)b;
    }
    npin += __popcll(mask);
  }
  __builtin_amdgcn_wave_barrier();
  if constexpr (WIDE) __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");  // the list's stores, then its loads
  else __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  const double base = numpy_sum([&](int k) { return share_of(p, st, r, WIDE ? g_pin[k] : (int)s_pin[k]); }, npin,
                                s_start, s_len, s_leaf);
  if (lane == 0) {
    MaxminRow mr;
    mr.base = base;
    mr.open = st.open;
    mr.counts = 0;
    m.mrow[r] = mr;
  }
}

// The base with the default pins (the first and the last block): NumPy sums fewer than 8 values in
// order from 0.0 and adds that to its 0.0 identity, so 0 + ((0 + share(0)) + share(n - 1)) for
// n >= 2 and 0 + (0 + share(0)) for n = 1.
__device__ __forceinline__ void base_default(const MaxminParams &m, int r) {
  const Params &p = m.p;
  const RowStat st = p.row_stat[r];
  double pinned = 0.0;
  if (st.n >= 1) pinned += share_of(p, st, r, 0);
  if (st.n >= 2) pinned += share_of(p, st, r, st.n - 1);
  MaxminRow mr;
  mr.base = 0.0 + pinned;
  mr.open = st.open;
  mr.counts = 0;
  m.mrow[r] = mr;
}

// per request, one workgroup: its n blocks in stable descending order of their gain keys (the
// pinned blocks keyed 0, after every open block, in block order), written as the sorted block
// indices (vals_out) and the open blocks' shares in that order (prefix, for the totals).
//
// The sort is a least-significant-digit radix sort in LDS, 8 bits a pass, over elements that pack
// a block's key bits 24-63 above its index (bits 0-13), so that one 64-bit word moves per block:
// shares computed from float32 scores that differ, differ in those bits (by at least 2^28 in their
// float64 bits).  The padding past n (key 0, index n and up) sorts after every block.  Where two
// neighbours agree in those bits and the later one's bits 0-23 are larger, every run of equal top
// bits is sorted again on (bits 0-23 descending, index ascending).
//
// A pass: each of the 16 waves owns a run of 64 * ITEMS consecutive positions and ranks it 64
// positions (one per lane) at a time.  The lanes that share a digit are found from eight ballots of
// its bits; a lane's rank in its wave is the wave's count of its digit so far (in LDS) plus the lanes
// before it that share the digit, and those lanes store the count raised by their number.  The waves' counts, scanned digit by digit (descending) then wave by wave,
// give each digit's first position for each wave, and every element moves to its place.  Equal digits
// keep their order, so the passes compose into a stable sort.
constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / kWave;
constexpr int kDigitBins = 256;
constexpr int kIndexBits = 14;    // block indices below 2^14
constexpr int kSortLowBits = 24;  // the key bits the first sort leaves out
static_assert(kMaxWidth <= (1 << kIndexBits), "a block index fits the packed element");
static_assert(kSortThreads == 4 * kDigitBins, "the count scan takes four counts of one digit a thread");

template <int MAX_ITEMS>
struct SortLds {
  unsigned long long elem[MAX_ITEMS * kSortThreads];
  unsigned int count[kSortWaves][kDigitBins];  // per wave and digit; scratch between the passes
};

// This wave's ranking of its ITEMS x 64 elements e (position order: i, then lane) by the digit at bit
// lo: info[i] = digit (bits 16-23, descending as ascending) << 16 | the element's rank among the
// wave's elements with that digit.  cnt (the wave's 256 counts in LDS) ends holding the wave's count
// of each digit.  Every lane of the wave must take part.
template <int ITEMS>
__device__ __forceinline__ void rank_wave(const unsigned long long (&e)[ITEMS], int lo, unsigned int *cnt,
                                          uint32_t (&info)[ITEMS]) {
  const int lane = lane_id();
  // cleared before the counting below: one wave's LDS accesses take effect in order
#pragma unroll
  for (int j = 0; j < kDigitBins / kWave; ++j) cnt[j * kWave + lane] = 0u;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const uint32_t d = 255u - (uint32_t)((e[i] >> lo) & 255u);
    // the lanes whose digit is d, as two 32-bit halves: for each bit, the ballot of the lanes that
    // have it, or its complement where d lacks it (f is all ones there)
    uint32_t peer_lo = ~0u, peer_hi = ~0u;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint32_t f = (uint32_t)__builtin_amdgcn_sbfe((int)~d, b, 1);  // all ones where d lacks the bit
      const uint64_t set = __ballot(f == 0u);
      peer_lo = __builtin_amdgcn_bitop3_b32(peer_lo, (uint32_t)set, f, 0x60);  // peer & (set ^ f)
      peer_hi = __builtin_amdgcn_bitop3_b32(peer_hi, (uint32_t)(set >> 32), f, 0x60);
    }
    // the wave's count of d so far, then every lane with d stores the same new count (no lane
    // diverges; this wave's LDS accesses take effect in order, so the next position reads it)
    const uint32_t before = cnt[d];
    cnt[d] = before + (uint32_t)(__popc(peer_lo) + __popc(peer_hi));
    info[i] = (d << 16) | (before + __builtin_amdgcn_mbcnt_hi(peer_hi, __builtin_amdgcn_mbcnt_lo(peer_lo, 0u)));
    // computed here: left to the compiler, the rank's parts (two masks and a count) would be carried
    // to the moves after the scan instead of this one word
    asm volatile("" : "+v"(info[i]));
  }
}

// One pass over bits [lo, lo + 8) of the ITEMS * kSortThreads elements in `elem`.
template <int ITEMS>
__device__ __forceinline__ void radix_pass(unsigned long long *elem, unsigned int (*count)[kDigitBins], int lo) {
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int run0 = wave * kWave * ITEMS;
  unsigned long long e[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) e[i] = elem[run0 + i * kWave + lane];
  uint32_t info[ITEMS];
  rank_wave<ITEMS>(e, lo, count[wave], info);
  __syncthreads();  // every wave's counts are final and every element is in registers
  {
    // the counts in (digit, wave) order: thread t takes digit t / 4 and waves 4 (t % 4) .. + 3; the
    // scan's scratch is the element array, free until the elements move
    const int d = threadIdx.x >> 2, w0 = (threadIdx.x & 3) * 4;
    uint32_t c[4];
    int sum = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      c[q] = count[w0 + q][d];
      sum += (int)c[q];
    }
    int total;
    int at = block_exclusive_scan<kSortThreads>(sum, reinterpret_cast<int *>(elem), total);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      count[w0 + q][d] = (uint32_t)at;
      at += (int)c[q];
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) elem[count[wave][info[i] >> 16] + (info[i] & 0xffffu)] = e[i];
  __syncthreads();
}

// the sort key of block b of a request from its score and pinned flag (0: pinned, or past its blocks)
__device__ __forceinline__ unsigned long long block_key(const RowStat &st, bool masked, int b, double score,
                                                        uint8_t pin) {
  const bool pinned = masked ? pin != 0 : (b == 0 || b == st.n - 1);
  const unsigned long long k = gain_key(share_value(st, score));
  return (b >= st.n || pinned) ? 0ull : k;
}

template <int ITEMS, int MAX_ITEMS>
__device__ __forceinline__ void sort_request(const MaxminParams &m, const RowStat &st, int r, SortLds<MAX_ITEMS> &lds) {
  static_assert(ITEMS <= MAX_ITEMS, "the LDS holds the sort");
  constexpr unsigned long long kIndexMask = (1ull << kIndexBits) - 1ull;
  constexpr unsigned long long kLow = (1ull << kSortLowBits) - 1ull;
  const Params &p = m.p;
  const int n = st.n, open = st.open;
  const int tid = threadIdx.x;
  const double *srow = p.scores + (int64_t)r * p.scores_stride;
  // Every load is unconditional and in range (indices clamped to the request's last block; without an
  // explicit mask the pinned flags are read from the scores and ignored), so none waits in a branch.
  const bool masked = p.pinned != nullptr;
  const uint8_t *prow = masked ? p.pinned + (int64_t)r * p.pinned_stride : reinterpret_cast<const uint8_t *>(srow);
  unsigned long long *elem = lds.elem;
  constexpr int kStep = ITEMS < 4 ? ITEMS : 4;  // positions loaded at a time
  // the full keys of the blocks that elements name, from their scores (in cache: just read), kStep
  // at a time with every load issued before any is used
  auto keys_of = [&](const int (&b)[ITEMS], unsigned long long (&k)[ITEMS]) {
#pragma unroll
    for (int i0 = 0; i0 < ITEMS; i0 += kStep) {
      double sc[kStep];
      uint8_t pn[kStep];
#pragma unroll
      for (int i = 0; i < kStep; ++i) {
        const int c = min(b[i0 + i], n - 1);
        sc[i] = srow[c];
        pn[i] = prow[c];
      }
#pragma unroll
      for (int i = 0; i < kStep; ++i) k[i0 + i] = block_key(st, masked, b[i0 + i], sc[i], pn[i]);
    }
  };
#pragma unroll
  for (int i0 = 0; i0 < ITEMS; i0 += kStep) {
    double score[kStep];
    uint8_t pin[kStep];
#pragma unroll
    for (int i = 0; i < kStep; ++i) {  // every load issued before any is used
      const int c = min((i0 + i) * kSortThreads + tid, n - 1);
      score[i] = srow[c];
      pin[i] = prow[c];
    }
#pragma unroll
    for (int i = 0; i < kStep; ++i) {
      const int pos = (i0 + i) * kSortThreads + tid;
      const unsigned long long k = block_key(st, masked, pos, score[i], pin[i]);
      elem[pos] = ((k >> kSortLowBits) << kIndexBits) | (unsigned long long)pos;
    }
  }
  __syncthreads();
#pragma unroll 1
  for (int lo = kIndexBits; lo < kIndexBits + 64 - kSortLowBits; lo += 8) radix_pass<ITEMS>(elem, lds.count, lo);

  // Neighbours that tie in the top bits: each thread takes ITEMS consecutive positions (so that a
  // scan over the threads numbers the runs of equal top bits in order) and the full keys of their blocks.
  // (The thread index passes through an empty asm before each phase that derives addresses from it:
  // otherwise the compiler computes every phase's addresses up front and holds them across the sort.)
  int t = tid;
  asm volatile("" : "+v"(t));
  unsigned long long key[ITEMS];
  int idx[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) idx[i] = (int)(elem[t * ITEMS + i] & kIndexMask);
  keys_of(idx, key);
  unsigned long long *last_key = reinterpret_cast<unsigned long long *>(&lds.count[0][0]);  // [kSortThreads]
  unsigned int *resort = &lds.count[kSortWaves - 1][kDigitBins - 1];  // past last_key
  static_assert(sizeof(unsigned long long) * kSortThreads < sizeof(lds.count), "the flag lies past last_key");
  last_key[t] = key[ITEMS - 1];
  if (t == 0) *resort = 0u;
  __syncthreads();
  const unsigned long long before = t > 0 ? last_key[t - 1] : 0ull;
  {
    bool unsorted = false;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int pos = t * ITEMS + i;
      const unsigned long long prev = i > 0 ? key[i - 1] : before;
      unsorted |= pos > 0 && pos < n && (key[i] >> kSortLowBits) == (prev >> kSortLowBits) && (key[i] & kLow) > (prev & kLow);
    }
    if (unsorted) *resort = 1u;
  }
  __syncthreads();
  if (*resort != 0u) {
    // each run of equal top bits again, on (bits 0-23, index): runs numbered in order by a scan of
    // their first positions, elements packed as (~run, bits 0-23, index) and sorted on bits 14-51
    // from the present order, which holds a run's blocks in block order
    int starts = 0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const unsigned long long prev = i > 0 ? key[i - 1] : before;
      starts += (t * ITEMS + i == 0 || (key[i] >> kSortLowBits) != (prev >> kSortLowBits)) ? 1 : 0;
    }
    int total_runs;
    int run = block_exclusive_scan<kSortThreads>(starts, reinterpret_cast<int *>(elem), total_runs) - 1;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const unsigned long long prev = i > 0 ? key[i - 1] : before;
      run += (t * ITEMS + i == 0 || (key[i] >> kSortLowBits) != (prev >> kSortLowBits)) ? 1 : 0;
      elem[t * ITEMS + i] = ((~(unsigned long long)run & kIndexMask) << (kIndexBits + kSortLowBits)) |
                              ((key[i] & kLow) << kIndexBits) | (unsigned long long)idx[i];
    }
    __syncthreads();
#pragma unroll 1
    for (int lo = kIndexBits; lo < 2 * kIndexBits + kSortLowBits; lo += 8) radix_pass<ITEMS>(elem, lds.count, lo);
  }
  // the outputs, striped (coalesced stores): position i * kSortThreads + thread
  const int64_t row0 = (int64_t)r * p.width;
  t = tid;
  asm volatile("" : "+v"(t));
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) idx[i] = (int)(elem[i * kSortThreads + t] & kIndexMask);
  keys_of(idx, key);
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int pos = i * kSortThreads + t;
    if (pos < n) m.vals_out[row0 + pos] = idx[i];
    if (pos < open) m.prefix[row0 + pos] = key_value(key[i]);
  }
}

// the requests by length, longest first (in classes of 256 blocks; any order within a class, as each
// sort writes only its own request's outputs), so the longest sorts start first and the short ones
// fill in behind them rather than leaving a long one to run alone at the end
constexpr int kOrderStep = 256;
constexpr int kOrderClasses = kMaxWidth / kOrderStep + 1;

// The requests longest first (by classes of kOrderStep blocks), for the totals' pairs of chains.
__device__ void order_requests(const MaxminParams &m) {
  __shared__ int s_count[kOrderClasses], s_next[kOrderClasses];
  const int tid = threadIdx.x;
  const int rows = m.p.rows;
  for (int j = tid; j < kLevels; j += kSortThreads) {  // summed into by the two level-count passes
    m.level_count[j] = 0;
    m.level_count2[j] = 0;
  }
  if (tid < kOrderClasses) s_count[tid] = 0;
  __syncthreads();
  auto cls = [&](int r) { return min(m.p.row_stat[r].n / kOrderStep, kOrderClasses - 1); };
  for (int r = tid; r < rows; r += kSortThreads) atomicAdd(&s_count[cls(r)], 1);
  __syncthreads();
  if (tid == 0) {
    int at = 0;
    for (int c = kOrderClasses - 1; c >= 0; --c) {
      s_next[c] = at;
      at += s_count[c];
    }
  }
  __syncthreads();
  for (int r = tid; r < rows; r += kSortThreads) m.order[atomicAdd(&s_next[cls(r)], 1)] = r;
}

// One workgroup before the sort: the requests' order, then (with the default pins) every request's
// base, then the budget's mode and the select's state (decide; its thread 0 finishes last).
template <bool DEFAULT_PINS>
__global__ __launch_bounds__(kSortThreads) void mm_plan_kernel(const MaxminParams m) {
  order_requests(m);
  if constexpr (DEFAULT_PINS)
    for (int r = threadIdx.x; r < m.p.rows; r += kSortThreads) base_default(m, r);
  decide<kSortThreads>(m.p);
}

// Two 16-wave sorting workgroups share a CU where their LDS allows it (sorts of up to 8192 blocks take
// 80 KB), at most 64 VGPRs each (8 waves per SIMD); the 12-key sort's 112 KB keeps it alone on a CU.
template <int MAX_ITEMS>
__global__ __launch_bounds__(kSortThreads) __attribute__((amdgpu_waves_per_eu(MAX_ITEMS <= 8 ? 8 : 4)))
void mm_sort_kernel(const MaxminParams m) {
  __shared__ SortLds<MAX_ITEMS> lds;
  const int r = m.order[blockIdx.x];
  const RowStat st = m.p.row_stat[r];
  if (st.n <= 0) return;
  if (st.n <= kSortThreads)
    sort_request<1>(m, st, r, lds);
  else if (st.n <= 2 * kSortThreads)
    sort_request<2>(m, st, r, lds);
  else if (MAX_ITEMS == 4 || st.n <= 4 * kSortThreads)
    sort_request<MAX_ITEMS < 4 ? MAX_ITEMS : 4>(m, st, r, lds);
  else if (MAX_ITEMS == 8 || st.n <= 8 * kSortThreads)
    sort_request<MAX_ITEMS < 8 ? MAX_ITEMS : 8>(m, st, r, lds);
  else
    sort_request<MAX_ITEMS>(m, st, r, lds);
}

// Requests wider than a sort in LDS: the same radix sort, one workgroup per request, its elements in
// global memory (keys_in and the request's prefix row, in turn) and streamed through the workgroup a
// tile of kWideTile at a time.  An element packs the key's bits 24-63 above an 18-bit index.  A pass
// counts the digit over the request, scans the counts into each digit's first position, then ranks
// the tiles in order as the LDS sort ranks its elements and moves each element to its digit's next
// position, which advances by the tile's count.  The runs that tie in the top bits are sorted again,
// as in the LDS sort, on (~run, bits 0-23, index) over six passes.
constexpr int kWideItems = 8;
constexpr int kWideTile = kWideItems * kSortThreads;
constexpr int kWideIndexBits = 18;
static_assert(kMaxMaxminWidth <= (1 << kWideIndexBits), "a block index fits the wide element");

struct WideSortLds {
  unsigned int count[kSortWaves][kDigitBins];
  unsigned int next[kDigitBins];  // each digit's next position in the destination
  int scan[kSortWaves];
  unsigned long long last[kSortThreads];  // the check: each thread's last key in the tile
  unsigned long long carry;               // the previous tile's last key
  int run_carry;                          // runs numbered before this tile
  unsigned int resort;
};

// one pass over bits [lo, lo + 8) of the n elements of src, into dst
__device__ __forceinline__ void wide_radix_pass(const unsigned long long *src, unsigned long long *dst, int n, int lo,
                                                WideSortLds &lds) {
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  const int run0 = wave * kWave * kWideItems;
  // the digit's count over the request (in the waves' counts, summed below)
#pragma unroll
  for (int j = 0; j < kDigitBins / kWave; ++j) lds.count[wave][j * kWave + lane] = 0u;
  __syncthreads();
  for (int t0 = 0; t0 < n; t0 += kWideTile) {
#pragma unroll
    for (int i = 0; i < kWideItems; ++i) {
      const int pos = t0 + run0 + i * kWave + lane;
      if (pos < n) atomicAdd(&lds.count[wave][255u - (uint32_t)((src[pos] >> lo) & 255u)], 1u);
    }
  }
  __syncthreads();
  {
    int total = 0;
    if (tid < kDigitBins)
      for (int w = 0; w < kSortWaves; ++w) total += (int)lds.count[w][tid];
    int all;
    const int at = block_exclusive_scan<kSortThreads>(total, lds.scan, all);
    if (tid < kDigitBins) lds.next[tid] = (unsigned int)at;
  }
  __syncthreads();
  for (int t0 = 0; t0 < n; t0 += kWideTile) {
    unsigned long long e[kWideItems];
#pragma unroll
    for (int i = 0; i < kWideItems; ++i) {
      const int pos = t0 + run0 + i * kWave + lane;
      e[i] = pos < n ? src[pos] : 0ull;  // past n: ranked after every element of the tile, never moved
    }
    uint32_t info[kWideItems];
    rank_wave<kWideItems>(e, lo, lds.count[wave], info);
    __syncthreads();
    if (tid < kDigitBins) {  // digit tid: the waves' first positions, and the digit's next after the tile
      unsigned int at = lds.next[tid];
      for (int w = 0; w < kSortWaves; ++w) {
        const unsigned int c = lds.count[w][tid];
        lds.count[w][tid] = at;
        at += c;
      }
      lds.next[tid] = at;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kWideItems; ++i) {
      const int pos = t0 + run0 + i * kWave + lane;
      if (pos < n) dst[lds.count[wave][info[i] >> 16] + (info[i] & 0xffffu)] = e[i];
    }
    __syncthreads();  // the counts are read before the next tile's ranking clears them
  }
}

__global__ __launch_bounds__(kSortThreads) void mm_wide_sort_kernel(const MaxminParams m) {
  __shared__ WideSortLds lds;
  constexpr unsigned long long kIndexMask = (1ull << kWideIndexBits) - 1ull;
  constexpr unsigned long long kLow = (1ull << kSortLowBits) - 1ull;
  const Params &p = m.p;
  const int r = blockIdx.x;
  const RowStat st = p.row_stat[r];
  const int n = st.n, open = st.open;
  if (n <= 0) return;
  const int tid = threadIdx.x;
  const int64_t row0 = (int64_t)r * p.width;
  const double *srow = p.scores + (int64_t)r * p.scores_stride;
  const bool masked = p.pinned != nullptr;
  const uint8_t *prow = masked ? p.pinned + (int64_t)r * p.pinned_stride : reinterpret_cast<const uint8_t *>(srow);
  auto key_of = [&](int b) {  // the full key of block b < n
    return block_key(st, masked, b, srow[b], prow[b]);
  };
  unsigned long long *buf[2] = {m.keys_in + row0, reinterpret_cast<unsigned long long *>(m.prefix + row0)};
  for (int pos = tid; pos < n; pos += kSortThreads)
    buf[0][pos] = ((key_of(pos) >> kSortLowBits) << kWideIndexBits) | (unsigned long long)pos;
  __syncthreads();
  int cur = 0;
#pragma unroll 1
  for (int lo = kWideIndexBits; lo < kWideIndexBits + 64 - kSortLowBits; lo += 8, cur ^= 1)
    wide_radix_pass(buf[cur], buf[cur ^ 1], n, lo, lds);
  // Neighbours that tie in the top bits, tile by tile: each thread its kWideItems consecutive positions
  if (tid == 0) {
    lds.resort = 0u;
    lds.carry = 0ull;
  }
  for (int t0 = 0; t0 < n; t0 += kWideTile) {
    unsigned long long key[kWideItems];
#pragma unroll
    for (int i = 0; i < kWideItems; ++i) {
      const int pos = t0 + tid * kWideItems + i;
      key[i] = pos < n ? key_of((int)(buf[cur][pos] & kIndexMask)) : 0ull;
    }
    lds.last[tid] = key[kWideItems - 1];
    __syncthreads();
    const unsigned long long before = tid > 0 ? lds.last[tid - 1] : lds.carry;
    bool unsorted = false;
#pragma unroll
    for (int i = 0; i < kWideItems; ++i) {
      const int pos = t0 + tid * kWideItems + i;
      const unsigned long long prev = i > 0 ? key[i - 1] : before;
      unsorted |= pos > 0 && pos < n && (key[i] >> kSortLowBits) == (prev >> kSortLowBits) && (key[i] & kLow) > (prev & kLow);
    }
    if (unsorted) lds.resort = 1u;
    __syncthreads();
    if (tid == kSortThreads - 1) lds.carry = key[kWideItems - 1];
  }
  __syncthreads();
  if (lds.resort != 0u) {
    // runs of equal top bits numbered in order (a scan of their first positions, tile by tile), the
    // elements packed as (~run, bits 0-23, index) into the other buffer, then six passes
    if (tid == 0) {
      lds.carry = 0ull;
      lds.run_carry = 0;
    }
    __syncthreads();
    for (int t0 = 0; t0 < n; t0 += kWideTile) {
      unsigned long long key[kWideItems];
      int idx[kWideItems];
#pragma unroll
      for (int i = 0; i < kWideItems; ++i) {
        const int pos = t0 + tid * kWideItems + i;
        idx[i] = pos < n ? (int)(buf[cur][pos] & kIndexMask) : 0;
        key[i] = pos < n ? key_of(idx[i]) : 0ull;
      }
      lds.last[tid] = key[kWideItems - 1];
      __syncthreads();
      const unsigned long long before = tid > 0 ? lds.last[tid - 1] : lds.carry;
      int starts = 0;
#pragma unroll
      for (int i = 0; i < kWideItems; ++i) {
        const int pos = t0 + tid * kWideItems + i;
        const unsigned long long prev = i > 0 ? key[i - 1] : before;
        starts += (pos < n && (pos == 0 || (key[i] >> kSortLowBits) != (prev >> kSortLowBits))) ? 1 : 0;
      }
      int tile_runs;
      int run = lds.run_carry + block_exclusive_scan<kSortThreads>(starts, lds.scan, tile_runs) - 1;
#pragma unroll
      for (int i = 0; i < kWideItems; ++i) {
        const int pos = t0 + tid * kWideItems + i;
        const unsigned long long prev = i > 0 ? key[i - 1] : before;
        run += (pos < n && (pos == 0 || (key[i] >> kSortLowBits) != (prev >> kSortLowBits))) ? 1 : 0;
        if (pos < n)
          buf[cur ^ 1][pos] = ((~(unsigned long long)run & kIndexMask) << (kWideIndexBits + kSortLowBits)) |
                              ((key[i] & kLow) << kWideIndexBits) | (unsigned long long)idx[i];
      }
      __syncthreads();
      if (tid == kSortThreads - 1) {
        lds.carry = key[kWideItems - 1];
        lds.run_carry += tile_runs;
      }
      __syncthreads();
    }
    cur ^= 1;
#pragma unroll 1
    for (int lo = kWideIndexBits; lo < 2 * kWideIndexBits + kSortLowBits; lo += 8, cur ^= 1)
      wide_radix_pass(buf[cur], buf[cur ^ 1], n, lo, lds);
  }
  // the outputs: each thread reads its positions before writing them (the final buffer may be the
  // prefix row itself)
  for (int pos0 = tid * kWideItems; pos0 < n; pos0 += kWideTile) {
    int idx[kWideItems];
#pragma unroll
    for (int i = 0; i < kWideItems; ++i) idx[i] = pos0 + i < n ? (int)(buf[cur][pos0 + i] & kIndexMask) : 0;
#pragma unroll
    for (int i = 0; i < kWideItems; ++i) {
      const int pos = pos0 + i;
      if (pos < n) m.vals_out[row0 + pos] = idx[i];
      if (pos < open) m.prefix[row0 + pos] = key_value(key_of(idx[i]));
    }
  }
}

// The running totals of the requests' sorted open shares (np.cumsum: t_i = fl(t_{i-1} + x_i) from
// t_{-1} = -0.0), in place, each request's by a wave in windows of kScanPer values a lane.  The
// shares are at least 0 (or -0.0, or NaN), so the totals never fall.  While a total t lies in one
// binade [2^E, 2^(E+1)), every float64 there is a multiple of its ulp u = 2^(E - 52), and as long as
// t + x stays below 2^(E+1) the rounded sum is t plus x / u rounded to the nearest integer, times u:
// x / u is exact (a scaling by a power of two) and, unless its fraction is exactly one half (a tie,
// decided by the parity of t / u), rounds the same way whatever t is.  So a window's totals are
// t + u * (inclusive prefix sums of those integers), an exact scan: every value up to the first
// one that ties, leaves the binade or is not finite takes its total that way.  From that value on,
// the next 64 values are added one at a time in order (a window stops where shares are about as
// large as the total, which the values after it mostly are too), as are values while t is not a
// positive normal float64 between 2^-960 and 2^1000 (-0.0 before the first value); a NaN total stays
// NaN to the end.  The integers and their sums stay below 2^53 wherever they are used, so they are
// exact in float64 too.  A long request of Dirichlet(0.1) shares takes ~19 windows of up to 512
// values and ~5 runs of 64 values added in order, against 8192 dependent adds of ~21 cycles for one
// chain.
//
// Beside each request's scan wave, a level wave places the levels j / kLevels (0 < j < kLevels) of
// the bisection's first steps in each chunk's totals while the scan wave takes the next chunk: a
// request's count at a level is its position among its totals shifted by 2r (np.searchsorted's left
// side, NaN above every level), so the levels are placed in increasing order, those a chunk holds
// being those at or below its last shifted total, each by a binary search of the chunk's totals in
// LDS.  The level wave also stores the chunk's totals with whole-wave stores.  It stores each
// position (level_pos) and adds the count into the workgroup's counts in LDS, added into level_count
// once at the end, so the first walk of the bisection needs no pass of its own.
constexpr int kTotalsChunk = 1024;  // values per chunk and request: 16 per lane
constexpr int kScanPer = 8;         // values a lane takes in a window (16: 6 us slower at 1024 x 8192)
constexpr int kTotalsReqs = 2;      // requests per workgroup: a scan wave and a level wave each
constexpr int kTotalsThreads = 2 * kTotalsReqs * kWave;
constexpr int kChunkSlots = kTotalsChunk + kTotalsChunk / 16;
static_assert(kTotalsChunk % (kWave * kScanPer) == 0, "whole windows per chunk");

// a chunk's value e in LDS: one spare slot after every 16, so a lane's 16 values start 17 slots
// after its neighbour's (two lanes a bank pair, not all of them)
__device__ __forceinline__ int chunk_slot(int e) { return e + (e >> 4); }

template <int CTRL, int ROW_MASK = 0xf, bool BOUND_ZERO = false>
__device__ __forceinline__ double dpp_move_f64(double v) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const int lo = dpp_move<CTRL, ROW_MASK, BOUND_ZERO>((int)(uint32_t)b);
  const int hi = dpp_move<CTRL, ROW_MASK, BOUND_ZERO>((int)(uint32_t)(b >> 32));
  return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}
// inclusive scan across the wave (wave_inclusive_scan's moves on both halves of a float64)
__device__ __forceinline__ double wave_inclusive_scan_f64(double v) {
  v += dpp_move_f64<0x111, 0xf, true>(v);
  v += dpp_move_f64<0x112, 0xf, true>(v);
  v += dpp_move_f64<0x114, 0xf, true>(v);
  v += dpp_move_f64<0x118, 0xf, true>(v);
  v += dpp_move_f64<0x142, 0xa>(v);
  v += dpp_move_f64<0x143, 0xc>(v);
  return v;
}
__device__ __forceinline__ double lane_f64(double v, int l) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// the totals of a chunk's first len values, in place in buf, from the total t before them; returns
// the total after them.  One wave, every lane active.
__device__ double scan_chunk(double *buf, int len, double t) {
  const int lane = lane_id();
  int pos = 0;
  bool alone = false;
  while (pos < len) {
    const uint64_t tb = (uint64_t)__double_as_longlong(t);
    const int eb = (int)((tb >> 52) & 0x7ff);  // t's biased exponent
    if (t != t) {                               // NaN: every later total is NaN
      for (int e = pos + lane; e < len; e += kWave) buf[chunk_slot(e)] = t;
      return t;
    }
    if (alone || !(t > 0.0) || eb < 63 || eb > 2022) {
      // -0.0, 0, below 2^-960 or above 2^1000, or after a window that stopped: the next kWave values
      // added one at a time, lane k holding value pos + k (a window stops where shares are about as
      // large as the total, which the values after it mostly are too)
      const int run = min(len - pos, kWave);
      const double x = buf[chunk_slot(pos + min(lane, run - 1))];
      double mine = 0.0;
      for (int k = 0; k < run; ++k) {
        t += lane_f64(x, k);
        if (lane == k) mine = t;
      }
      if (lane < run) buf[chunk_slot(pos + lane)] = mine;
      pos += run;
      alone = false;
      continue;
    }
    const double u = __longlong_as_double((long long)((uint64_t)(eb - 52) << 52));     // 2^(E - 52)
    const double inv = __longlong_as_double((long long)((uint64_t)(2098 - eb) << 52));  // 2^(52 - E)
    const double room = 0x1p53 - t * inv;  // (2^(E+1) - t) / u, an integer
    const int n = min(len - pos, kWave * kScanPer);
    const int first = pos + lane * kScanPer;
    double y[kScanPer], run[kScanPer];
    bool fits[kScanPer];
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < kScanPer; ++k) {
      const int e = first + k;
      const double yy = buf[chunk_slot(min(e, len - 1))] * inv;  // every read issued, none under a condition
      const bool in = e < pos + n && yy >= 0.0 && yy < 0x1p53;
      const double r = __builtin_floor(yy), f = yy - r;
      fits[k] = in && f != 0.5;
      y[k] = yy;
      sum += in ? r + (f > 0.5 ? 1.0 : 0.0) : 0.0;
      run[k] = sum;  // this lane's inclusive prefix
    }
    // the lanes before this one: the scan of the sums moved one lane up (wave_shr:1), so a lane's own
    // sum, which may hold values past its stop, never enters its prefix
    const double before = wave_inclusive_scan_f64(dpp_move_f64<0x138, 0xf, true>(sum));
    // the first value that cannot take the window: a tie, out of range, past the window, or one
    // whose sum with the total before it reaches 2^(E+1)
    int stop = kScanPer;
#pragma unroll
    for (int k = 0; k < kScanPer; ++k) {
      const double prior = before + (k > 0 ? run[k - 1] : 0.0);
      if (stop == kScanPer && !(fits[k] && y[k] < room - prior)) stop = k;
    }
    const uint64_t stopped = __builtin_amdgcn_ballot_w64(stop < kScanPer);
    const int sl = stopped ? __builtin_ctzll(stopped) : kWave;
    const int taken = stopped ? sl * kScanPer + __builtin_amdgcn_readlane(stop, sl) : kWave * kScanPer;
    // a value past the taken ones is written to the lane's spare slot (the one after values
    // 16 lane .. 16 lane + 15, which no value maps to), so no store waits on a branch
#pragma unroll
    for (int k = 0; k < kScanPer; ++k)
      buf[lane * kScanPer + k < taken ? chunk_slot(first + k) : 17 * lane + 16] = t + (before + run[k]) * u;
    if (taken > 0) {
      const int last = taken - 1, kl = last % kScanPer;
      double mine = 0.0;
#pragma unroll
      for (int k = 0; k < kScanPer; ++k)
        if (k == kl) mine = before + run[k];
      t = t + lane_f64(mine, last / kScanPer) * u;
    }
    pos += taken;
    alone = taken < n;  // the value that stopped the window and those after it, one at a time
  }
  return t;
}

// A request's scan wave and level wave hand its chunks over through kTotalsBufs LDS buffers and two
// progress counters in LDS (chunks scanned, chunks placed), not a workgroup barrier per chunk, so the
// scan runs up to kTotalsBufs - 1 chunks ahead of the placements (a request's first chunk holds most of
// its levels).  The scan waits only for placements kTotalsBufs chunks back and the level wave only for
// chunks already scanned, so neither waits on the other at once; each wait is also bounded by
// kProgressSpins sleeps, which a run never reaches.
constexpr int kTotalsBufs = 4;
constexpr int kProgressSpins = 1 << 22;

__device__ __forceinline__ void wait_progress(const int *counter, int target) {
  for (int spin = 0; *(volatile const int *)counter < target && spin < kProgressSpins; ++spin)
    __builtin_amdgcn_s_sleep(1);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}
// every LDS access of the wave before it completes, then lane 0 raises the counter
__device__ __forceinline__ void raise_progress(int *counter, int value) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  if (lane_id() == 0) *(volatile int *)counter = value;
}

__global__ __launch_bounds__(kTotalsThreads) void mm_totals_kernel(const MaxminParams m) {
  constexpr int kPer = kTotalsChunk / kWave;
  constexpr int Q = kTotalsReqs;
  // each request's chunks of shares in turn, overwritten by their totals
  __shared__ double s_chunk[kTotalsBufs][Q][kChunkSlots];
  __shared__ int s_count[kLevels];  // the level waves' counts of the workgroup's requests
  __shared__ int s_scanned[Q], s_placed[Q];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const bool scan_wave = wave < Q;
  const int q = scan_wave ? wave : wave - Q;  // this wave's request in the workgroup
  for (int j = threadIdx.x; j < kLevels; j += kTotalsThreads) s_count[j] = 0;
  if (threadIdx.x < Q) {
    s_scanned[threadIdx.x] = 0;
    s_placed[threadIdx.x] = 0;
  }
  __syncthreads();
  const int k = blockIdx.x * Q + q;
  const int req = k < m.p.rows ? m.order[k] : -1;
  const int open = req >= 0 ? m.p.row_stat[req].open : 0;
  const int chunks = (open + kTotalsChunk - 1) / kTotalsChunk;
  double *row = m.prefix + (int64_t)max(req, 0) * m.p.width;
  if (scan_wave) {
    // the request's next chunk in registers (loads at a clamped index, none under a condition;
    // value 0 of request 0's row stands in for a missing request)
    double v[kPer];
    auto fetch = [&](int c0) {
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int i = c0 + j * kWave + lane;
        const double x = row[min(i, max(open - 1, 0))];
        v[j] = i < open ? x : 0.0;
      }
    };
    fetch(0);
    double t = -0.0;  // the total before the chunk
    for (int c = 0; c < chunks; ++c) {
      if (c >= kTotalsBufs) wait_progress(&s_placed[q], c - kTotalsBufs + 1);  // the buffer is free
      double *buf = s_chunk[c % kTotalsBufs][q];
#pragma unroll
      for (int j = 0; j < kPer; ++j) buf[chunk_slot(j * kWave + lane)] = v[j];
      // the scan reads what every lane of the wave wrote
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_wave_barrier();
      fetch((c + 1) * kTotalsChunk);  // the next chunk, in flight during the scan
      t = scan_chunk(buf, min(open - c * kTotalsChunk, kTotalsChunk), t);
      raise_progress(&s_scanned[q], c + 1);
    }
  } else {
    int next = 1;  // the next level to place
    const double shift = 2.0 * (double)max(req, 0);
    const double base = req >= 0 ? m.mrow[req].base : 0.0;
    for (int c = 0; c < chunks; ++c) {
      // the chunk's totals: store them, and place every level at or below its last shifted total
      wait_progress(&s_scanned[q], c + 1);
      const int c0 = c * kTotalsChunk;
      const int len = min(open - c0, kTotalsChunk);
      const double *tot = s_chunk[c % kTotalsBufs][q];
      {  // lane b stores values 16b .. 16b + 15
        constexpr int kRun = kTotalsChunk / kWave;
        const int e0 = lane * kRun;
        double x[kRun];
#pragma unroll
        for (int i = 0; i < kRun; ++i) x[i] = tot[chunk_slot(e0 + i)];
        double *dst = row + c0 + e0;
        if (e0 + kRun <= len) {
#pragma unroll
          for (int i = 0; i < kRun; i += 2) *reinterpret_cast<double2 *>(dst + i) = double2{x[i], x[i + 1]};
        } else {
#pragma unroll
          for (int i = 0; i < kRun; ++i)
            if (e0 + i < len) dst[i] = x[i];
        }
      }
      const double last = tot[chunk_slot(len - 1)] + shift;
      while (next < kLevels) {
        const int j = next + lane;
        const double need = (double)j / kLevels - base;
        const double target = (need - 1e-12) + shift;
        const bool here = j < kLevels && !(last < target);  // the lanes that hold one: a prefix of the wave
        if (here) {
          int lo = 0, hi = len - 1;  // the first total whose shifted value is not below the target
          while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (tot[chunk_slot(mid)] + shift < target) lo = mid + 1;
            else hi = mid;
          }
          const int pos = c0 + lo;
          set_pos(m, m.level_pos, req, j, pos);
          const int count = need <= 1e-12 ? 0 : min(pos + 1, open);
          if (count > 0) atomicAdd(&s_count[j], count);
        }
        const int placed = __popcll(__ballot(here));
        next += placed;
        if (placed < kWave) break;
      }
      raise_progress(&s_placed[q], c + 1);  // the chunk's buffer is free
    }
    if (req >= 0) {  // the levels above every total: position `open`, count `open`
      for (int j = next + lane; j < kLevels; j += kWave) {
        set_pos(m, m.level_pos, req, j, open);
        const double need = (double)j / kLevels - base;
        const int count = need <= 1e-12 ? 0 : open;
        if (count > 0) atomicAdd(&s_count[j], count);
      }
    }
  }
  __syncthreads();
  for (int j = threadIdx.x; j < kLevels; j += kTotalsThreads)
    if (s_count[j] > 0) atomicAdd(&m.level_count[j], s_count[j]);
}

constexpr int kLevelThreads = 256;  // the second level-count pass's workgroups

// The first kLevelBits steps of the bisection over counts summed at kLevels levels: [jl, jh] of
// those levels, jh = jl + 1 (the same decisions: a level rises when its count fits the free blocks).
// A count never falls as the level rises (each request's count is 0 until its need passes 1e-12,
// then its position plus one, which only grows), so the steps end at jl = the number of levels
// 0 < j < kLevels whose count fits, which the workgroup counts at once rather than in ten dependent
// steps.  Contains barriers: every thread calls it.
template <int NT>
__device__ __forceinline__ void walk_levels(const int *s_level, long long free_blocks, int &jl, int &jh) {
  __shared__ int s_fit[NT / kWave];
  int fit = 0;
  for (int j = threadIdx.x; j < kLevels; j += NT) fit += (j >= 1 && (long long)s_level[j] <= free_blocks) ? 1 : 0;
  jl = block_sum<NT>(fit, s_fit);
  jh = jl + 1;
}

// The second level-count pass: the next kLevelBits steps the same way.  Every workgroup repeats the
// first walk (the summed counts staged in LDS), then counts each of its requests at the levels
// low + j / kLevels^2 (0 < j < kLevels) inside the walk's bracket [low, high] -- exactly the mids
// the bisection's next steps visit -- searching only between the request's positions at low and
// high from the first pass.  That range of the request's totals is staged in LDS first with coalesced
// loads (up to kStaged of them; a wider range is searched in memory), so a search waits on one load
// rather than on each of its steps.
constexpr int kStaged = 6144;  // totals of a request's bracket staged in LDS (48 KB)

__global__ __launch_bounds__(kLevelThreads) void mm_levels2_kernel(const MaxminParams m) {
  constexpr int kMine = (kLevels + kLevelThreads - 1) / kLevelThreads;
  __shared__ int s_level[kLevels];
  __shared__ double s_tot[kStaged];
  const Params &p = m.p;
  const State *s = p.state;
  if (s->mode != kSelect || s->error) return;
  for (int j = threadIdx.x; j < kLevels; j += kLevelThreads) s_level[j] = m.level_count[j];
  __syncthreads();
  int jl, jh;
  walk_levels<kLevelThreads>(s_level, s->free_blocks, jl, jh);
  const double low = (double)jl / kLevels;
  constexpr double kSub = 1.0 / ((double)kLevels * (double)kLevels);
  int mine[kMine];
#pragma unroll
  for (int i = 0; i < kMine; ++i) mine[i] = 0;
  for (int r = blockIdx.x; r < p.rows; r += gridDim.x) {
    const MaxminRow mr = m.mrow[r];
    const int open = mr.open;
    const int lo0 = jl > 0 ? pos_at(m, m.level_pos, r, jl) : 0;
    const int hi0 = jh < kLevels ? pos_at(m, m.level_pos, r, jh) : open;
    const double *pre = m.prefix + (int64_t)r * p.width;
    const double shift = 2.0 * (double)r;
    const int span = hi0 - lo0;
    const bool staged = span <= kStaged;
    __syncthreads();  // the previous request's searches are done with s_tot
    if (staged && span > 0) {
      // the whole bracket in one batch of loads (none under a condition), 6 or 24 a thread
      auto stage = [&](auto batch) {
        constexpr int B = decltype(batch)::value;
        double x[B];
#pragma unroll
        for (int u = 0; u < B; ++u) x[u] = pre[lo0 + min((int)threadIdx.x + u * kLevelThreads, span - 1)];
#pragma unroll
        for (int u = 0; u < B; ++u)
          if ((int)threadIdx.x + u * kLevelThreads < span) s_tot[threadIdx.x + u * kLevelThreads] = x[u];
      };
      if (span <= kStaged / 4) stage(std::integral_constant<int, kStaged / 4 / kLevelThreads>());
      else stage(std::integral_constant<int, kStaged / kLevelThreads>());
    }
    __syncthreads();

#pragma unroll
    for (int i = 0; i < kMine; ++i) {
      const int j = i * kLevelThreads + threadIdx.x;
      if (j < 1 || j >= kLevels) continue;
      const double level = low + (double)j * kSub;  // exact: both terms are multiples of kSub
      const double need = level - mr.base;
      const double q = (need - 1e-12) + shift;
      int a = lo0, b = hi0;
      if (staged) {
        while (a < b) {  // first position whose shifted total is >= q
          const int c = (a + b) >> 1;
          if (s_tot[c - lo0] + shift < q) a = c + 1; else b = c;
        }
      } else {
        while (a < b) {
          const int c = (a + b) >> 1;
          if (pre[c] + shift < q) a = c + 1; else b = c;
        }
      }
      set_pos(m, m.level_pos2, r, j, a);
      mine[i] += need <= 1e-12 ? 0 : min(a + 1, open);
    }
  }
#pragma unroll
  for (int i = 0; i < kMine; ++i) {
    const int j = i * kLevelThreads + threadIdx.x;
    if (j >= 1 && j < kLevels && mine[i] > 0) atomicAdd(&m.level_count2[j], mine[i]);
  }
}

// the level's bisection and the leftover, one workgroup
// RPT: requests per thread (1, 2, 4 or 8 by the request count), so the common case keeps its state
// in registers
template <int RPT>
__global__ __launch_bounds__(kBisectThreads) void mm_bisect_kernel(const MaxminParams m) {
  constexpr int kRowsPerThread = RPT;
  static_assert(RPT >= 1 && RPT * kBisectThreads <= kMaxMaxminRegRows, "requests per thread");
  __shared__ long long s_red[kBisectThreads / kWave];
  __shared__ double s_best[kBisectThreads / kWave];
  const Params &p = m.p;
  const State *s = p.state;
  if (s->mode != kSelect || s->error) return;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  const long long free_blocks = s->free_blocks;
  double base[kRowsPerThread];
  int open[kRowsPerThread], lo[kRowsPerThread], hi[kRowsPerThread], mid_pos[kRowsPerThread];
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    const int r = tid + j * kBisectThreads;
    const bool in = r < p.rows;
    base[j] = in ? m.mrow[r].base : 0.0;
    open[j] = in ? m.mrow[r].open : 0;
    lo[j] = 0;
    hi[j] = open[j];
  }
  // count of request r at a level: its position among its shifted totals, from the bracket
  auto count_at = [&](int j, double level, int &pos) -> int {
    const int r = tid + j * kBisectThreads;
    const double need = level - base[j];
    const double shift = 2.0 * (double)r;
    const double q = (need - 1e-12) + shift;
    const double *pre = m.prefix + (int64_t)r * p.width;
    int a = lo[j], b = hi[j];
    while (a < b) {  // first position whose shifted total is >= q
      const int c = (a + b) >> 1;
      if (pre[c] + shift < q) a = c + 1; else b = c;
    }
    pos = a;
    return need <= 1e-12 ? 0 : min(a + 1, open[j]);
  };
  // the first 2 kLevelBits steps: walks over the summed counts of the two level-count passes, at
  // the levels j / kLevels, then low + j / kLevels^2 inside the first walk's bracket
  __shared__ int s_level[kLevels];
  for (int j = tid; j < kLevels; j += kBisectThreads) s_level[j] = m.level_count[j];
  __syncthreads();
  int jl, jh;
  walk_levels<kBisectThreads>(s_level, free_blocks, jl, jh);
  __syncthreads();
  for (int j = tid; j < kLevels; j += kBisectThreads) s_level[j] = m.level_count2[j];
  __syncthreads();
  int jl2, jh2;
  walk_levels<kBisectThreads>(s_level, free_blocks, jl2, jh2);
  constexpr double kSub = 1.0 / ((double)kLevels * (double)kLevels);
  const double low1 = (double)jl / kLevels;
  double low = low1 + (double)jl2 * kSub, high = low1 + (double)jh2 * kSub;
  // the brackets those steps leave: the positions at low and high, where each side has moved.  A
  // request's count never falls as the level rises, so one whose counts at low and high agree keeps
  // that count at every level between them.
  int f_low[kRowsPerThread], f_high[kRowsPerThread], f_mid[kRowsPerThread];
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    f_low[j] = f_high[j] = f_mid[j] = 0;
    if (tid + j * kBisectThreads >= p.rows) continue;
    // the positions at the levels reached come from the level-count passes (a bracket end that the
    // second walk did not move is a first-pass level); the ends 0 and 1 (never a step's level) are
    // searched, for the counts there
    const int r = tid + j * kBisectThreads;

    int pos_low, pos_high;
    if (jl2 > 0 || jl > 0) {
      pos_low = jl2 > 0 ? pos_at(m, m.level_pos2, r, jl2) : pos_at(m, m.level_pos, r, jl);
      f_low[j] = (low - base[j]) <= 1e-12 ? 0 : min(pos_low + 1, open[j]);
    } else {
      f_low[j] = count_at(j, low, pos_low);
      pos_low = 0;
    }
    if (jh2 < kLevels || jh < kLevels) {
      pos_high = jh2 < kLevels ? pos_at(m, m.level_pos2, r, jh2) : pos_at(m, m.level_pos, r, jh);
      f_high[j] = (high - base[j]) <= 1e-12 ? 0 : min(pos_high + 1, open[j]);
    } else {
      f_high[j] = count_at(j, high, pos_high);
      pos_high = open[j];
    }
    lo[j] = pos_low;
    hi[j] = pos_high;
  }
  int it = 2 * kLevelBits;
  while (it < 60) {
    const double mid = (low + high) / 2;
    long long local = 0, active = 0;
#pragma unroll
    for (int j = 0; j < kRowsPerThread; ++j) {
      if (tid + j * kBisectThreads >= p.rows) continue;
      active += f_low[j] != f_high[j] ? 1 : 0;
      f_mid[j] = count_at(j, mid, mid_pos[j]);
      local += f_mid[j];
    }
    // the count (below 2^40) and the requests still changing (below 2^24), in one sum
    const long long packed = block_sum<kBisectThreads>(local + (active << 40), s_red);
    const long long total = packed & ((1ll << 40) - 1);
    const bool up = total <= free_blocks;
    if (up) low = mid; else high = mid;
#pragma unroll
    for (int j = 0; j < kRowsPerThread; ++j) {
      if (tid + j * kBisectThreads >= p.rows) continue;
      if (up) {
        lo[j] = mid_pos[j];
        f_low[j] = f_mid[j];
      } else {
        hi[j] = mid_pos[j];
        f_high[j] = f_mid[j];
      }
    }
    ++it;
    if ((packed >> 40) <= kWave) break;  // at most a wave's worth of requests can still change
  }
  if (it < 60) {
    // the rest of the steps in wave 0 over the requests still changing, lane i taking the i-th; the
    // others add a fixed count.  Their brackets stay with their owners, a superset of where the final
    // count lies, which the count at the final level finds again.
    __shared__ int s_nact, s_act_row[kWave], s_act_lo[kWave], s_act_hi[kWave], s_act_open[kWave];
    __shared__ double s_act_base[kWave], s_level_pair[2];
    if (tid == 0) s_nact = 0;
    __syncthreads();
    long long fixed_local = 0;
#pragma unroll
    for (int j = 0; j < kRowsPerThread; ++j) {
      const int r = tid + j * kBisectThreads;
      if (r >= p.rows) continue;
      if (f_low[j] != f_high[j]) {
        const int i = atomicAdd(&s_nact, 1);
        s_act_row[i] = r;
        s_act_lo[i] = lo[j];
        s_act_hi[i] = hi[j];
        s_act_open[i] = open[j];
        s_act_base[i] = base[j];
      } else {
        fixed_local += f_low[j];
      }
    }
    const long long fixed = block_sum<kBisectThreads>(fixed_local, s_red);  // its barriers publish the list
    if (wave == 0) {
      const bool mine = lane < s_nact;
      const int r = mine ? s_act_row[lane] : 0;
      int a_lo = mine ? s_act_lo[lane] : 0, a_hi = mine ? s_act_hi[lane] : 0;
      const int a_open = mine ? s_act_open[lane] : 0;
      const double a_base = mine ? s_act_base[lane] : 0.0;
      const double shift = 2.0 * (double)r;
      const double *pre = m.prefix + (int64_t)r * p.width;
      for (; it < 60; ++it) {
        const double mid = (low + high) / 2;
        int f = 0, pos = a_lo;
        if (mine) {
          const double need = mid - a_base;
          const double q = (need - 1e-12) + shift;
          int a = a_lo, b = a_hi;
          while (a < b) {  // first position whose shifted total is >= q
            const int c = (a + b) >> 1;
            if (pre[c] + shift < q) a = c + 1; else b = c;
          }
          pos = a;
          f = need <= 1e-12 ? 0 : min(a + 1, a_open);
        }
        const bool up = fixed + (long long)wave_sum_int(f) <= free_blocks;
        if (up) {
          low = mid;
          a_lo = pos;
        } else {
          high = mid;
          a_hi = pos;
        }
      }
      if (lane == 0) {
        s_level_pair[0] = low;
        s_level_pair[1] = high;
      }
    }
    __syncthreads();
    low = s_level_pair[0];
    high = s_level_pair[1];
  }
  // counts at the final level, then the leftover to the lowest (retained, index) first
  int counts[kRowsPerThread];
  double retained[kRowsPerThread];
  long long used = 0;
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    const int r = tid + j * kBisectThreads;
    counts[j] = 0;
    retained[j] = 0.0;
    if (r >= p.rows) continue;
    int pos;
    counts[j] = count_at(j, low, pos);
    used += counts[j];
    retained[j] = base[j] + (counts[j] ? m.prefix[(int64_t)r * p.width + counts[j] - 1] : 0.0);
  }
  long long leftover = free_blocks - block_sum<kBisectThreads>(used, s_red);
  // The leftover as the reference's heap hands it out (allocation.py:157-166): the request with the
  // lowest (retained, index) takes its next block, and its retained share grows by that block's
  // share.  A request's level never falls, so the pops are a merge of the requests' level sequences
  // by (level, index).  One pass serves every request tied at the lowest level L, in index order:
  // a request whose next share leaves L unchanged when added (zero, or below L's last bit) stays at
  // L and so takes every block it has left (its later shares, sorted descending, are no larger),
  // any other takes one block and rises above L.  The pass ends the leftover where it runs out.
  if constexpr (RPT <= 4) {
    __shared__ int s_scan[kBisectThreads / kWave];
    while (leftover > 0) {
      double low_level = INFINITY;
  #pragma unroll
      for (int j = 0; j < kRowsPerThread; ++j) {
        const int r = tid + j * kBisectThreads;
        if (r < p.rows && counts[j] < open[j]) low_level = fmin(low_level, retained[j]);
      }
      for (int msk = 32; msk >= 1; msk >>= 1) low_level = fmin(low_level, __shfl_xor(low_level, msk, kWave));
      if (lane == 0) s_best[wave] = low_level;
      __syncthreads();
      low_level = s_best[0];
      for (int w = 1; w < kBisectThreads / kWave; ++w) low_level = fmin(low_level, s_best[w]);
      __syncthreads();
      if (low_level == INFINITY) break;  // every request keeps all its blocks
      long long served = 0;  // blocks the tied requests before the current rows take
  #pragma unroll
      for (int j = 0; j < kRowsPerThread; ++j) {
        const int r = tid + j * kBisectThreads;
        const bool tied = r < p.rows && counts[j] < open[j] && retained[j] == low_level;
        double next_share = 0.0;
        int take = 0;
        if (tied) {
          const RowStat st = p.row_stat[r];
          next_share = share_of(p, st, r, m.vals_out[(int64_t)r * p.width + counts[j]]);
          take = low_level + next_share == low_level ? open[j] - counts[j] : 1;
        }
        int pass_total;
        const long long before = served + block_exclusive_scan<kBisectThreads>(take, s_scan, pass_total);
        const long long got = tied ? max(0LL, min((long long)take, leftover - before)) : 0LL;
        if (got > 0) {
          counts[j] += (int)got;
          if (take == 1) retained[j] = low_level + next_share;  // the level popped plus the kept block's share
        }
        served += pass_total;
      }
      leftover -= min(served, leftover);
    }
  } else {
    // with eight requests a thread, one block a pass (the per-row scans of the batched form would
    // not fit the registers)
    __shared__ int s_best_row[kBisectThreads / kWave];
    while (leftover > 0) {
      double best = INFINITY;
      int best_row = INT_MAX;
  #pragma unroll
      for (int j = 0; j < kRowsPerThread; ++j) {
        const int r = tid + j * kBisectThreads;
        if (r >= p.rows || counts[j] >= open[j]) continue;
        if (retained[j] < best || (retained[j] == best && r < best_row)) {
          best = retained[j];
          best_row = r;
        }
      }
      for (int msk = 32; msk >= 1; msk >>= 1) {
        const double ob = __shfl_xor(best, msk, kWave);
        const int orow = __shfl_xor(best_row, msk, kWave);
        if (ob < best || (ob == best && orow < best_row)) {
          best = ob;
          best_row = orow;
        }
      }
      if (lane == 0) {
        s_best[wave] = best;
        s_best_row[wave] = best_row;
      }
      __syncthreads();
      best = s_best[0];
      best_row = s_best_row[0];
      for (int w = 1; w < kBisectThreads / kWave; ++w) {
        if (s_best[w] < best || (s_best[w] == best && s_best_row[w] < best_row)) {
          best = s_best[w];
          best_row = s_best_row[w];
        }
      }
      __syncthreads();
      if (best_row == INT_MAX) break;  // every request keeps all its blocks
  #pragma unroll
      for (int j = 0; j < kRowsPerThread; ++j) {
        if (tid + j * kBisectThreads != best_row) continue;
        const int64_t row0 = (int64_t)best_row * p.width;
        const RowStat st = p.row_stat[best_row];
        const double sh = share_of(p, st, best_row, m.vals_out[row0 + counts[j]]);
        counts[j] += 1;
        retained[j] = best + sh;  // the level popped plus the kept block's share
      }
      --leftover;
    }
  }
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    const int r = tid + j * kBisectThreads;
    if (r < p.rows) m.mrow[r].counts = counts[j];
  }
}

// The bisection and the leftover for more requests than the register form holds: the same walks,
// steps, wave-0 finish and leftover passes as mm_bisect_kernel, each request's state in memory and
// every loop over the requests strided over the workgroup (requests r = tid, tid + 1024, ..., so a
// scan chunk by chunk keeps index order).
__global__ __launch_bounds__(kBisectThreads) void mm_bisect_mem_kernel(const MaxminParams m) {
  __shared__ long long s_red[kBisectThreads / kWave];
  __shared__ double s_best[kBisectThreads / kWave];
  __shared__ int s_level[kLevels];
  const Params &p = m.p;
  const State *s = p.state;
  if (s->mode != kSelect || s->error) return;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  const int rows = p.rows;
  const long long free_blocks = s->free_blocks;
  auto count_in = [&](int r, double base, int open, double level, int a, int b, int &pos) -> int {
    const double need = level - base;
    const double shift = 2.0 * (double)r;
    const double q = (need - 1e-12) + shift;
    const double *pre = m.prefix + (int64_t)r * p.width;
    while (a < b) {  // first position whose shifted total is >= q
      const int c = (a + b) >> 1;
      if (pre[c] + shift < q) a = c + 1; else b = c;
    }
    pos = a;
    return need <= 1e-12 ? 0 : min(a + 1, open);
  };
  // the first 2 kLevelBits steps: the two level-count passes' walks
  for (int j = tid; j < kLevels; j += kBisectThreads) s_level[j] = m.level_count[j];
  __syncthreads();
  int jl, jh;
  walk_levels<kBisectThreads>(s_level, free_blocks, jl, jh);
  __syncthreads();
  for (int j = tid; j < kLevels; j += kBisectThreads) s_level[j] = m.level_count2[j];
  __syncthreads();
  int jl2, jh2;
  walk_levels<kBisectThreads>(s_level, free_blocks, jl2, jh2);
  constexpr double kSub = 1.0 / ((double)kLevels * (double)kLevels);
  const double low1 = (double)jl / kLevels;
  double low = low1 + (double)jl2 * kSub, high = low1 + (double)jh2 * kSub;
  for (int r = tid; r < rows; r += kBisectThreads) {
    const MaxminRow mr = m.mrow[r];

    int pos_low, pos_high, f_low, f_high;
    if (jl2 > 0 || jl > 0) {
      pos_low = jl2 > 0 ? pos_at(m, m.level_pos2, r, jl2) : pos_at(m, m.level_pos, r, jl);
      f_low = (low - mr.base) <= 1e-12 ? 0 : min(pos_low + 1, mr.open);
    } else {
      f_low = count_in(r, mr.base, mr.open, low, 0, mr.open, pos_low);
      pos_low = 0;
    }
    if (jh2 < kLevels || jh < kLevels) {
      pos_high = jh2 < kLevels ? pos_at(m, m.level_pos2, r, jh2) : pos_at(m, m.level_pos, r, jh);
      f_high = (high - mr.base) <= 1e-12 ? 0 : min(pos_high + 1, mr.open);
    } else {
      f_high = count_in(r, mr.base, mr.open, high, 0, mr.open, pos_high);
      pos_high = mr.open;
    }
    m.b_lo[r] = pos_low;
    m.b_hi[r] = pos_high;
    m.b_flo[r] = f_low;
    m.b_fhi[r] = f_high;
  }
  int it = 2 * kLevelBits;
  while (it < 60) {
    const double mid = (low + high) / 2;
    long long local = 0, active = 0;
    for (int r = tid; r < rows; r += kBisectThreads) {
      const MaxminRow mr = m.mrow[r];
      active += m.b_flo[r] != m.b_fhi[r] ? 1 : 0;
      int pos;
      const int f = count_in(r, mr.base, mr.open, mid, m.b_lo[r], m.b_hi[r], pos);
      m.b_fmid[r] = f;
      m.b_pmid[r] = pos;
      local += f;
    }
    const long long packed = block_sum<kBisectThreads>(local + (active << 40), s_red);
    const long long total = packed & ((1ll << 40) - 1);
    const bool up = total <= free_blocks;
    if (up) low = mid; else high = mid;
    for (int r = tid; r < rows; r += kBisectThreads) {
      if (up) {
        m.b_lo[r] = m.b_pmid[r];
        m.b_flo[r] = m.b_fmid[r];
      } else {
        m.b_hi[r] = m.b_pmid[r];
        m.b_fhi[r] = m.b_fmid[r];
      }
    }
    ++it;
    if ((packed >> 40) <= kWave) break;  // at most a wave's worth of requests can still change
  }
  if (it < 60) {
    // the rest of the steps in wave 0 over the requests still changing, as in mm_bisect_kernel
    __shared__ int s_nact, s_act_row[kWave], s_act_lo[kWave], s_act_hi[kWave], s_act_open[kWave];
    __shared__ double s_act_base[kWave], s_level_pair[2];
    if (tid == 0) s_nact = 0;
    __syncthreads();
    long long fixed_local = 0;
    for (int r = tid; r < rows; r += kBisectThreads) {
      const int fl = m.b_flo[r];
      if (fl != m.b_fhi[r]) {
        const MaxminRow mr = m.mrow[r];
        const int i = atomicAdd(&s_nact, 1);
        s_act_row[i] = r;
        s_act_lo[i] = m.b_lo[r];
        s_act_hi[i] = m.b_hi[r];
        s_act_open[i] = mr.open;
        s_act_base[i] = mr.base;
      } else {
        fixed_local += fl;
      }
    }
    const long long fixed = block_sum<kBisectThreads>(fixed_local, s_red);  // its barriers publish the list
    if (wave == 0) {
      const bool mine = lane < s_nact;
      const int r = mine ? s_act_row[lane] : 0;
      int a_lo = mine ? s_act_lo[lane] : 0, a_hi = mine ? s_act_hi[lane] : 0;
      const int a_open = mine ? s_act_open[lane] : 0;
      const double a_base = mine ? s_act_base[lane] : 0.0;
      for (; it < 60; ++it) {
        const double mid = (low + high) / 2;
        int f = 0, pos = a_lo;
        if (mine) f = count_in(r, a_base, a_open, mid, a_lo, a_hi, pos);
        const bool up = fixed + (long long)wave_sum_int(f) <= free_blocks;
        if (up) {
          low = mid;
          a_lo = pos;
        } else {
          high = mid;
          a_hi = pos;
        }
      }
      if (lane == 0) {
        s_level_pair[0] = low;
        s_level_pair[1] = high;
      }
    }
    __syncthreads();
    low = s_level_pair[0];
    high = s_level_pair[1];
  }
  // counts at the final level (searched inside each request's bracket, a superset of where it lies)
  long long used = 0;
  for (int r = tid; r < rows; r += kBisectThreads) {
    const MaxminRow mr = m.mrow[r];
    int pos;
    const int c = count_in(r, mr.base, mr.open, low, m.b_lo[r], m.b_hi[r], pos);
    m.b_count[r] = c;
    m.b_retained[r] = mr.base + (c ? m.prefix[(int64_t)r * p.width + c - 1] : 0.0);
    used += c;
  }
  long long leftover = free_blocks - block_sum<kBisectThreads>(used, s_red);
  // the leftover by levels (allocation.py:157-166), as mm_bisect_kernel: one pass serves every
  // request tied at the lowest level in index order, the scan taken chunk by chunk of requests
  __shared__ int s_scan[kBisectThreads / kWave];
  while (leftover > 0) {
    double low_level = INFINITY;
    for (int r = tid; r < rows; r += kBisectThreads)
      if (m.b_count[r] < m.mrow[r].open) low_level = fmin(low_level, m.b_retained[r]);
    for (int msk = 32; msk >= 1; msk >>= 1) low_level = fmin(low_level, __shfl_xor(low_level, msk, kWave));
    if (lane == 0) s_best[wave] = low_level;
    __syncthreads();
    low_level = s_best[0];
    for (int w = 1; w < kBisectThreads / kWave; ++w) low_level = fmin(low_level, s_best[w]);
    __syncthreads();
    if (low_level == INFINITY) break;  // every request keeps all its blocks
    long long served = 0;  // blocks the tied requests of the earlier chunks take
    for (int r0 = 0; r0 < rows; r0 += kBisectThreads) {
      const int r = r0 + tid;
      int c = 0, open = 0, take = 0;
      double next_share = 0.0;
      bool tied = false;
      if (r < rows) {
        c = m.b_count[r];
        open = m.mrow[r].open;
        tied = c < open && m.b_retained[r] == low_level;
      }
      if (tied) {
        const RowStat st = p.row_stat[r];
        next_share = share_of(p, st, r, m.vals_out[(int64_t)r * p.width + c]);
        take = low_level + next_share == low_level ? open - c : 1;
      }
      int pass_total;
      const long long before = served + block_exclusive_scan<kBisectThreads>(take, s_scan, pass_total);
      const long long got = tied ? max(0LL, min((long long)take, leftover - before)) : 0LL;
      if (got > 0) {
        m.b_count[r] = c + (int)got;
        if (take == 1) m.b_retained[r] = low_level + next_share;  // the level popped plus the kept block's share
      }
      served += pass_total;
    }
    leftover -= min(served, leftover);
    __syncthreads();  // every request's count and share are stored before the next pass reads them
  }
  for (int r = tid; r < rows; r += kBisectThreads) m.mrow[r].counts = m.b_count[r];
}

// The keep: the first `counts` blocks of the request's sorted order marked in an LDS bitmap (rows
// up to kKeepBits blocks; wider rows are written, then the kept blocks set, in two sweeps), then every
// byte of the row written once.
constexpr int kKeepBits = 1 << 16;
__global__ __launch_bounds__(kThreads) void mm_keep_kernel(const MaxminParams m) {
  __shared__ uint32_t s_kept[kKeepBits / 32];
  const Params &p = m.p;
  const int r = blockIdx.x;
  const State *s = p.state;
  const RowStat st = p.row_stat[r];
  const bool all = s->error != 0 || s->mode == kKeepAll || s->mode == kKeepOpen;
  uint8_t *krow = p.keep + (int64_t)r * p.keep_stride;
  const int counts = (!all && s->mode == kSelect) ? m.mrow[r].counts : 0;
  const int64_t row0 = (int64_t)r * p.width;
  if (p.width > kKeepBits) {
    for (int b = threadIdx.x; b < p.width; b += kThreads)
      krow[b] = (all || b >= st.n || pinned_at(p, r, b, st.n)) ? 1 : 0;
    __syncthreads();
    for (int i = threadIdx.x; i < counts; i += kThreads) krow[m.vals_out[row0 + i]] = 1;
    return;
  }
  const int words = (p.width + 31) / 32;
  for (int w = threadIdx.x; w < words; w += kThreads) s_kept[w] = 0u;
  __syncthreads();
  constexpr int kLoads = 8;  // loads in flight per thread
  for (int i0 = threadIdx.x; i0 < counts; i0 += kLoads * kThreads) {
    int b[kLoads];
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const int i = i0 + u * kThreads;
      const int v = m.vals_out[row0 + min(i, counts - 1)];  // every load issued, none under a condition
      b[u] = i < counts ? v : -1;
    }
#pragma unroll
    for (int u = 0; u < kLoads; ++u)
      if (b[u] >= 0) atomicOr(&s_kept[b[u] >> 5], 1u << (b[u] & 31));
  }
  __syncthreads();
  for (int b = threadIdx.x; b < p.width; b += kThreads) {
    const bool kept = (s_kept[b >> 5] >> (b & 31)) & 1u;
    krow[b] = (all || b >= st.n || kept || pinned_at(p, r, b, st.n)) ? 1 : 0;
  }
}

// ---------------------------------------------------------------------------------------
// The controller's rule for `sum` and `maxmin` (Controller._allocate, observe/controller.py:398-451):
// a row takes part when it is longer than cap_above_blocks and has evidence; its request holds its
// existing blocks in order (freed blocks leave it, :425-431), block 0, the recent_blocks newest and
// the blocks from its audited length on being pinned (:420-424); the budget is
// max(pinned, ceil(fraction * blocks)) over every block of the taking-part rows, freed or not
// (:435-437); rows that take no part, and positions past a row, keep every block.  The requests
// are numbered in row order over the taking-part rows only -- `maxmin` shifts request r's running
// totals by 2r in its one search -- and the rows that take no part become empty requests after
// them, which change nothing.
// ---------------------------------------------------------------------------------------
struct CtlParams {
  const void *shares;
  int32_t shares_f64;  // float64 shares (else float32)
  int64_t shares_stride;
  const int32_t *lengths;
  const uint8_t *evidence;
  const int32_t *audited;  // may be null
  const uint8_t *released;  // may be null
  int64_t released_stride;
  const double *weights;  // may be null
  int32_t rows, width, recent, cap;
  CtlHeader *header;
  int32_t *row_slot;  // request of each row, -1: takes no part
  int32_t *slot_row;
  // the requests as the allocation reads them: [rows][width] scores and pins, block counts, weights
  double *req_scores;
  uint8_t *req_pinned;
  int32_t *req_blocks;
  double *req_weights;
  uint8_t *req_keep;
};

constexpr int kCtlPlanThreads = 1024;

__device__ __forceinline__ int ctl_blocks(const CtlParams &c, int r) { return min(max(c.lengths[r], 0), c.width); }
__device__ __forceinline__ bool ctl_takes_part(const CtlParams &c, int r) {
  return c.lengths[r] > c.cap && c.evidence[r] != 0;  // controller.py:402-408
}
__device__ __forceinline__ bool ctl_exists(const CtlParams &c, int r, int b) {
  return c.released == nullptr || c.released[(int64_t)r * c.released_stride + b] == 0;
}

// One workgroup: which rows take part, their requests' numbers, and their blocks.
__global__ __launch_bounds__(kCtlPlanThreads) void ctl_plan_kernel(const CtlParams c) {
  __shared__ int s_scan[kCtlPlanThreads / kWave];
  __shared__ long long s_sum[kCtlPlanThreads / kWave];
  long long blocks = 0;
  int before = 0;
  for (int r0 = 0; r0 < c.rows; r0 += kCtlPlanThreads) {
    const int r = r0 + threadIdx.x;
    const bool part = r < c.rows && ctl_takes_part(c, r);
    int chunk;
    const int slot = before + block_exclusive_scan<kCtlPlanThreads>(part ? 1 : 0, s_scan, chunk);
    if (r < c.rows) c.row_slot[r] = part ? slot : -1;
    if (part) {
      c.slot_row[slot] = r;
      blocks += ctl_blocks(c, r);
    }
    before += chunk;
  }
  blocks = block_sum<kCtlPlanThreads>(blocks, s_sum);
  if (threadIdx.x == 0) {
    c.header->blocks = blocks;
    c.header->requests = before;
  }
}

// One workgroup per request slot: the request's existing blocks in order, with their scores
// (float64) and pins; the slots after the last request are empty.
__global__ __launch_bounds__(kThreads) void ctl_compact_kernel(const CtlParams c) {
  __shared__ int s_scan[kThreads / kWave];
  const int j = blockIdx.x;
  if (j >= c.header->requests) {
    if (threadIdx.x == 0) {
      c.req_blocks[j] = 0;
      c.req_weights[j] = 1.0;
    }
    return;
  }
  const int r = c.slot_row[j];
  const int n = ctl_blocks(c, r);
  const int recent_at = max(0, n - 1 - c.recent);
  const int audited_at = c.audited != nullptr ? min(max(c.audited[r], 0), n) : n;  // controller.py:424
  double *srow = c.req_scores + (int64_t)j * c.width;
  uint8_t *prow = c.req_pinned + (int64_t)j * c.width;
  int base = 0;
  for (int b0 = 0; b0 < n; b0 += kThreads) {
    const int b = b0 + threadIdx.x;
    const bool e = b < n && ctl_exists(c, r, b);
    int chunk;
    const int at = base + block_exclusive_scan<kThreads>(e ? 1 : 0, s_scan, chunk);
    if (e) {
      double s;
      if (c.shares_f64) s = reinterpret_cast<const double *>(c.shares)[(int64_t)r * c.shares_stride + b];
      else s = (double)reinterpret_cast<const float *>(c.shares)[(int64_t)r * c.shares_stride + b];
      srow[at] = s;
      prow[at] = (b == 0 || b >= recent_at || b >= audited_at) ? 1 : 0;
    }
    base += chunk;
  }
  if (threadIdx.x == 0) {
    c.req_blocks[j] = base;
    c.req_weights[j] = c.weights != nullptr ? c.weights[r] : 1.0;
  }
}

// One workgroup per row: the request's keep back at the row's positions (a freed block 0, a
// position past the row 1, a row that takes no part all 1).
__global__ __launch_bounds__(kThreads) void ctl_scatter_kernel(const CtlParams c, uint8_t *keep, int64_t keep_stride) {
  __shared__ int s_scan[kThreads / kWave];
  const int r = blockIdx.x;
  const int j = c.row_slot[r];
  uint8_t *krow = keep + (int64_t)r * keep_stride;
  const int n = j >= 0 ? ctl_blocks(c, r) : 0;
  for (int b = n + threadIdx.x; b < c.width; b += kThreads) krow[b] = 1;
  if (j < 0) return;
  const uint8_t *qrow = c.req_keep + (int64_t)j * c.width;
  int base = 0;
  for (int b0 = 0; b0 < n; b0 += kThreads) {
    const int b = b0 + threadIdx.x;
    const bool e = b < n && ctl_exists(c, r, b);
    int chunk;
    const int at = base + block_exclusive_scan<kThreads>(e ? 1 : 0, s_scan, chunk);
    if (b < n) krow[b] = e ? qrow[at] : 0;
    base += chunk;
  }
}

int launch_sum(Params p, hipStream_t s);
int launch_maxmin(MaxminParams m, int rows, int width, hipStream_t s);

}  // namespace alloc
}  // namespace ekv

using namespace ekv;

namespace {
// The sum workspace from its 256-aligned base: the state, the row statistics, the passes' workgroups'
// list lengths (one per row at most), then the list of the second pass (kCandPerRow pairs per row),
// each right after the last (8-byte aligned).
static_assert(sizeof(alloc::State) % 8 == 0 && sizeof(alloc::RowStat) % 8 == 0, "the list is 8-byte aligned");
size_t sum_cand_offset(int32_t rows) {
  const size_t r = (size_t)(rows > 0 ? rows : 0);
  return sizeof(alloc::State) + r * sizeof(alloc::RowStat) + ((r * sizeof(unsigned int) + 7) & ~(size_t)7);
}
void set_sum_buffers(uintptr_t base, int32_t rows, alloc::Params &p) {
  p.state = (alloc::State *)base;
  p.row_stat = (alloc::RowStat *)(base + sizeof(alloc::State));
  p.cand_count = (unsigned int *)(base + sizeof(alloc::State) + (size_t)(rows > 0 ? rows : 0) * sizeof(alloc::RowStat));
  p.cand = (unsigned long long *)(base + sum_cand_offset(rows));
}
}  // namespace

extern "C" size_t ekv_rank_sum_workspace(int32_t rows) {
  const size_t r = (size_t)(rows > 0 ? rows : 0);
  return sum_cand_offset(rows) + r * alloc::kCandPerRow * 2 * sizeof(unsigned long long) + 256;
}

extern "C" int ekv_rank_sum(const double *scores, int64_t scores_stride, const int32_t *blocks,
                            const double *weights, const uint8_t *pinned, int64_t pinned_stride, int32_t rows,
                            int32_t width, int64_t budget, uint8_t *keep, int64_t keep_stride, int64_t *summary,
                            void *workspace, size_t workspace_bytes, void *stream) {
  if (scores == nullptr || blocks == nullptr || keep == nullptr || workspace == nullptr)
    return fail(EKV_EINVAL, "ekv_rank_sum: null pointer");
  if (rows < 0 || rows > alloc::kMaxRows || width < 1 || width > alloc::kMaxSumWidth)
    return fail(EKV_EINVAL, "ekv_rank_sum: rows %d (max %d), width %d (max %d)", rows, alloc::kMaxRows, width,
                alloc::kMaxSumWidth);
  if (budget < 0) return fail(EKV_EINVAL, "ekv_rank_sum: the budget cannot be negative");
  if (workspace_bytes < ekv_rank_sum_workspace(rows))
    return fail(EKV_EINVAL, "ekv_rank_sum: a workspace of %zu bytes is below the %zu needed", workspace_bytes,
                ekv_rank_sum_workspace(rows));
  if (rows == 0) return EKV_OK;
  alloc::Params p{};
  p.scores = scores;
  p.scores_stride = scores_stride;
  p.blocks = blocks;
  p.weights = weights;
  p.pinned = pinned;
  p.pinned_stride = pinned_stride;
  p.rows = rows;
  p.width = width;
  p.budget = budget;
  p.keep = keep;
  p.keep_stride = keep_stride;
  p.summary = summary;
  const uintptr_t base = ((uintptr_t)workspace + 255) & ~(uintptr_t)255;
  set_sum_buffers(base, rows, p);
  return alloc::launch_sum(p, (hipStream_t)stream);
}

namespace ekv {
namespace alloc {

// The `sum` pipeline on prepared parameters (state and row statistics in place).
int launch_sum(Params p, hipStream_t s) {
  const int rows = p.rows;
  p.tie_rbits = tie_request_bits(rows);
  hipLaunchKernelGGL(alloc::prepare_kernel, dim3(rows), dim3(alloc::kPrepThreads), 0, s, p);
  hipLaunchKernelGGL(alloc::decide_kernel, dim3(1), dim3(alloc::kThreads), 0, s, p);
  const dim3 grid((unsigned)std::min<int64_t>(rows, (int64_t)cu_count()));
  // the gain threshold, kDigitBits at a time from the top of the 64-bit key
  // (the second pass lists the blocks in the first pass's bucket; the later passes read that list)
  // the kernels for the caller's pins: a mask, or each row's first and last block
  const bool pin = p.pinned != nullptr;
  using Pass = void (*)(alloc::Params, int, int, int);
  const Pass first = pin ? alloc::hist_kernel<false, 0, true> : alloc::hist_kernel<false, 0, false>;
  const Pass second = pin ? alloc::hist_kernel<false, 1, true> : alloc::hist_kernel<false, 1, false>;
  const Pass listed = pin ? alloc::hist_kernel<false, 2, true> : alloc::hist_kernel<false, 2, false>;
  const Pass tied = pin ? alloc::hist_kernel<true, 2, true> : alloc::hist_kernel<true, 2, false>;
  int pass = 0;
  for (int top = 64; top > 0; top -= alloc::kDigitBits, ++pass) {
    const int shift = std::max(top - alloc::kDigitBits, 0), bits = top - shift;
    const int last = shift == 0 ? 1 : 0;
    const Pass kernel = pass == 0 ? first : pass == 1 ? second : listed;
    hipLaunchKernelGGL(kernel, grid, dim3(alloc::kHistThreads), 0, s, p, shift, bits, last);
  }
  // among the blocks at the threshold: newer block, earlier request (the tie key)
  static_assert(alloc::kMaxSumWidth <= (1 << 18), "the tie key's block field is at most 18 bits");
  for (int top = tie_bits(p.width, p.tie_rbits); top > 0; top -= alloc::kDigitBits) {
    const int shift = std::max(top - alloc::kDigitBits, 0), bits = top - shift;
    hipLaunchKernelGGL(tied, grid, dim3(alloc::kHistThreads), 0, s, p, shift, bits, -1);
  }
  hipLaunchKernelGGL(pin ? alloc::sum_keep_kernel<true> : alloc::sum_keep_kernel<false>, grid,
                     dim3(alloc::kHistThreads), 0, s, p);
  return check_hip(hipGetLastError(), "ekv_rank_sum launch");
}

}  // namespace alloc
}  // namespace ekv

namespace {

struct MaxminLayout {
  size_t state, row_stat, mrow, order, level_count, level_pos, level_count2, level_pos2, bisect, vals_out, prefix,
      total;
  size_t keys_in;  // rows wider than kMaxWidth: the sort's second buffer (0: none)
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

MaxminLayout maxmin_layout(int32_t rows, int32_t width) {
  MaxminLayout l{};
  const size_t cells = (size_t)rows * (size_t)width;
  size_t at = 0;
  l.state = at;
  at = align256(at + sizeof(alloc::State));
  l.row_stat = at;
  at = align256(at + (size_t)rows * sizeof(alloc::RowStat));
  l.mrow = at;
  at = align256(at + (size_t)rows * sizeof(alloc::MaxminRow));
  l.order = at;
  at = align256(at + (size_t)rows * sizeof(int32_t));
  l.level_count = at;
  at = align256(at + (size_t)alloc::kLevels * sizeof(int32_t));
  const size_t pos_bytes = width > 65535 ? sizeof(uint32_t) : sizeof(uint16_t);
  l.level_pos = at;
  at = align256(at + (size_t)rows * alloc::kLevels * pos_bytes);
  l.level_count2 = at;
  at = align256(at + (size_t)alloc::kLevels * sizeof(int32_t));
  l.level_pos2 = at;
  at = align256(at + (size_t)rows * alloc::kLevels * pos_bytes);
  l.bisect = at;  // seven int32 arrays and one double array of rows entries (the memory bisection's state)
  at = align256(at + (size_t)rows * (7 * sizeof(int32_t) + sizeof(double)) + 8 * 256);
  l.vals_out = at;
  at = align256(at + cells * 4);
  l.prefix = at;
  at = align256(at + cells * 8);
  if (width > alloc::kMaxWidth) {
    l.keys_in = at;
    at = align256(at + cells * 8);
  }
  l.total = at + 256;  // + 256: the base may be realigned
  return l;
}

// The maxmin buffers of a workspace laid out by maxmin_layout from `base`.
void set_maxmin_buffers(const MaxminLayout &l, uintptr_t base, alloc::MaxminParams &m) {
  m.p.state = (alloc::State *)(base + l.state);
  m.p.row_stat = (alloc::RowStat *)(base + l.row_stat);
  m.mrow = (alloc::MaxminRow *)(base + l.mrow);
  m.vals_out = (int32_t *)(base + l.vals_out);
  m.prefix = (double *)(base + l.prefix);
  m.order = (int32_t *)(base + l.order);
  m.level_count = (int32_t *)(base + l.level_count);
  m.level_pos = (void *)(base + l.level_pos);
  m.pos32 = m.p.width > 65535 ? 1 : 0;  // as the layout sized them
  m.level_count2 = (int32_t *)(base + l.level_count2);
  m.level_pos2 = (void *)(base + l.level_pos2);
  {
    const int rows = m.p.rows;  // set by the callers before the buffers
    uintptr_t at = base + l.bisect;
    auto take_ints = [&](int32_t *&dst) {
      dst = (int32_t *)at;
      at = (at + (size_t)rows * sizeof(int32_t) + 255) & ~(uintptr_t)255;
    };
    take_ints(m.b_lo);
    take_ints(m.b_hi);
    take_ints(m.b_flo);
    take_ints(m.b_fhi);
    take_ints(m.b_fmid);
    take_ints(m.b_pmid);
    take_ints(m.b_count);
    m.b_retained = (double *)at;
  }
  if (m.p.width > alloc::kMaxWidth) m.keys_in = (unsigned long long *)(base + l.keys_in);
}

}  // namespace

extern "C" size_t ekv_rank_maxmin_workspace(int32_t rows, int32_t width) {
  if (rows <= 0 || width <= 0) return 256;
  return maxmin_layout(rows, width).total;
}

extern "C" int ekv_rank_maxmin(const double *scores, int64_t scores_stride, const int32_t *blocks,
                               const uint8_t *pinned, int64_t pinned_stride, int32_t rows, int32_t width,
                               int64_t budget, uint8_t *keep, int64_t keep_stride, int64_t *summary,
                               void *workspace, size_t workspace_bytes, void *stream) {
  if (scores == nullptr || blocks == nullptr || keep == nullptr || workspace == nullptr)
    return fail(EKV_EINVAL, "ekv_rank_maxmin: null pointer");
  if (rows < 0 || rows > alloc::kMaxMaxminRows || width < 1 || width > alloc::kMaxMaxminWidth)
    return fail(EKV_EINVAL, "ekv_rank_maxmin: rows %d (max %d), width %d (max %d)", rows, alloc::kMaxMaxminRows,
                width, alloc::kMaxMaxminWidth);
  if (budget < 0) return fail(EKV_EINVAL, "ekv_rank_maxmin: the budget cannot be negative");
  if (rows == 0) return EKV_OK;
  const MaxminLayout l = maxmin_layout(rows, width);
  if (workspace_bytes < l.total)
    return fail(EKV_EINVAL, "ekv_rank_maxmin: a workspace of %zu bytes is below the %zu needed", workspace_bytes,
                l.total);
  const uintptr_t base = ((uintptr_t)workspace + 255) & ~(uintptr_t)255;
  alloc::MaxminParams m{};
  alloc::Params &p = m.p;
  p.scores = scores;
  p.scores_stride = scores_stride;
  p.blocks = blocks;
  p.weights = nullptr;
  p.pinned = pinned;
  p.pinned_stride = pinned_stride;
  p.rows = rows;
  p.width = width;
  p.budget = budget;
  p.keep = keep;
  p.keep_stride = keep_stride;
  p.summary = summary;
  set_maxmin_buffers(l, base, m);
  return alloc::launch_maxmin(m, rows, width, (hipStream_t)stream);
}

namespace ekv {
namespace alloc {

// The `maxmin` pipeline on prepared parameters (every workspace pointer in place).
int launch_maxmin(MaxminParams m, int rows, int width, hipStream_t s) {
  Params &p = m.p;
  hipLaunchKernelGGL(alloc::prepare_kernel, dim3(rows), dim3(alloc::kPrepThreads), 0, s, p);
  const bool wide = width > alloc::kMaxWidth;
  if (p.pinned == nullptr) {
    hipLaunchKernelGGL(alloc::mm_plan_kernel<true>, dim3(1), dim3(alloc::kSortThreads), 0, s, m);
  } else {
    hipLaunchKernelGGL(alloc::mm_plan_kernel<false>, dim3(1), dim3(alloc::kSortThreads), 0, s, m);
    if (wide) hipLaunchKernelGGL(alloc::mm_base_kernel<true>, dim3(rows), dim3(kWave), 0, s, m);
    else hipLaunchKernelGGL(alloc::mm_base_kernel<false>, dim3(rows), dim3(kWave), 0, s, m);
  }
  int rc = check_hip(hipGetLastError(), "ekv_rank_maxmin launch");
  if (rc != EKV_OK) return rc;
  if (wide) {
    hipLaunchKernelGGL(alloc::mm_wide_sort_kernel, dim3(rows), dim3(alloc::kSortThreads), 0, s, m);
  } else if (width <= 4 * alloc::kSortThreads)
    hipLaunchKernelGGL(alloc::mm_sort_kernel<4>, dim3(rows), dim3(alloc::kSortThreads), 0, s, m);
  else if (width <= 8 * alloc::kSortThreads)
    hipLaunchKernelGGL(alloc::mm_sort_kernel<8>, dim3(rows), dim3(alloc::kSortThreads), 0, s, m);
  else
    hipLaunchKernelGGL(alloc::mm_sort_kernel<12>, dim3(rows), dim3(alloc::kSortThreads), 0, s, m);
  rc = check_hip(hipGetLastError(), "ekv_rank_maxmin sort");
  if (rc != EKV_OK) return rc;
  hipLaunchKernelGGL(alloc::mm_totals_kernel, dim3((rows + alloc::kTotalsReqs - 1) / alloc::kTotalsReqs),
                     dim3(alloc::kTotalsThreads), 0, s, m);
  const dim3 level_grid((unsigned)std::min<int64_t>(rows, (int64_t)cu_count() * 2));
  hipLaunchKernelGGL(alloc::mm_levels2_kernel, level_grid, dim3(alloc::kLevelThreads), 0, s, m);
  if (rows > alloc::kMaxMaxminRegRows)
    hipLaunchKernelGGL(alloc::mm_bisect_mem_kernel, dim3(1), dim3(alloc::kBisectThreads), 0, s, m);
  else if (rows <= alloc::kBisectThreads)
    hipLaunchKernelGGL(alloc::mm_bisect_kernel<1>, dim3(1), dim3(alloc::kBisectThreads), 0, s, m);
  else if (rows <= 2 * alloc::kBisectThreads)
    hipLaunchKernelGGL(alloc::mm_bisect_kernel<2>, dim3(1), dim3(alloc::kBisectThreads), 0, s, m);
  else if (rows <= 4 * alloc::kBisectThreads)
    hipLaunchKernelGGL(alloc::mm_bisect_kernel<4>, dim3(1), dim3(alloc::kBisectThreads), 0, s, m);
  else
    hipLaunchKernelGGL(alloc::mm_bisect_kernel<8>, dim3(1), dim3(alloc::kBisectThreads), 0, s, m);
  hipLaunchKernelGGL(alloc::mm_keep_kernel, dim3(rows), dim3(alloc::kThreads), 0, s, m);
  return check_hip(hipGetLastError(), "ekv_rank_maxmin launch");
}

}  // namespace alloc
}  // namespace ekv

namespace {

// Workspace of ekv_controller_keep: the plan, the requests in allocation form, then the objective's
// own workspace.
struct CtlLayout {
  size_t header, row_slot, slot_row, req_blocks, req_weights, req_scores, req_pinned, req_keep, inner, total;
};

CtlLayout ctl_layout(int objective, int32_t rows, int32_t width) {
  CtlLayout l{};
  const size_t cells = (size_t)rows * (size_t)width;
  size_t at = 0;
  l.header = at;
  at = align256(at + sizeof(alloc::CtlHeader));
  l.row_slot = at;
  at = align256(at + (size_t)rows * 4);
  l.slot_row = at;
  at = align256(at + (size_t)rows * 4);
  l.req_blocks = at;
  at = align256(at + (size_t)rows * 4);
  l.req_weights = at;
  at = align256(at + (size_t)rows * 8);
  l.req_scores = at;
  at = align256(at + cells * 8);
  l.req_pinned = at;
  at = align256(at + cells);
  l.req_keep = at;
  at = align256(at + cells);
  l.inner = at;
  at += objective == EKV_OBJ_SUM ? ekv_rank_sum_workspace(rows) : ekv_rank_maxmin_workspace(rows, width);
  l.total = at + 256;  // + 256: the base may be realigned
  return l;
}

}  // namespace

extern "C" size_t ekv_controller_keep_workspace(int32_t objective, int32_t rows, int32_t width) {
  if ((objective != EKV_OBJ_SUM && objective != EKV_OBJ_MAXMIN) || rows <= 0 || width <= 0) return 256;
  return ctl_layout(objective, rows, width).total;
}

extern "C" int ekv_controller_keep(int32_t objective, const void *shares, int32_t shares_dtype, int64_t shares_stride,
                                   const int32_t *lengths, const uint8_t *evidence, const int32_t *audited_blocks,
                                   const uint8_t *released, int64_t released_stride, const double *weights,
                                   int32_t rows, int32_t width, int32_t recent_blocks, int32_t cap_above_blocks,
                                   double fraction, uint8_t *keep, int64_t keep_stride, int64_t *summary,
                                   void *workspace, size_t workspace_bytes, void *stream) {
  if (shares == nullptr || lengths == nullptr || evidence == nullptr || keep == nullptr || workspace == nullptr)
    return fail(EKV_EINVAL, "ekv_controller_keep: null pointer");
  if (objective != EKV_OBJ_SUM && objective != EKV_OBJ_MAXMIN)
    return fail(EKV_EINVAL, "ekv_controller_keep: objective %d is neither sum (%d) nor maxmin (%d)", objective,
                EKV_OBJ_SUM, EKV_OBJ_MAXMIN);
  if (objective == EKV_OBJ_MAXMIN && weights != nullptr)
    return fail(EKV_EINVAL, "ekv_controller_keep: the maxmin objective does not use request weights");
  if (shares_dtype != EKV_F32 && shares_dtype != EKV_F64)
    return fail(EKV_EUNSUPPORTED, "ekv_controller_keep: shares of dtype %d (float32 or float64)", shares_dtype);
  const int max_rows = objective == EKV_OBJ_SUM ? alloc::kMaxRows : alloc::kMaxMaxminRows;
  const int max_width = objective == EKV_OBJ_SUM ? alloc::kMaxSumWidth : alloc::kMaxMaxminWidth;
  if (rows < 0 || rows > max_rows || width < 1 || width > max_width)
    return fail(EKV_EINVAL, "ekv_controller_keep: rows %d (max %d), width %d (max %d)", rows, max_rows, width,
                max_width);
  if (recent_blocks < 0 || cap_above_blocks < 0)
    return fail(EKV_EINVAL, "ekv_controller_keep: recent_blocks %d, cap_above_blocks %d", recent_blocks,
                cap_above_blocks);
  if (!(fraction > 0.0 && fraction <= 1.0))
    return fail(EKV_EINVAL, "ekv_controller_keep: the budget fraction %g is not in (0, 1]", fraction);
  if (rows == 0) return EKV_OK;
  const CtlLayout l = ctl_layout(objective, rows, width);
  if (workspace_bytes < l.total)
    return fail(EKV_EINVAL, "ekv_controller_keep: a workspace of %zu bytes is below the %zu needed", workspace_bytes,
                l.total);
  const uintptr_t base = ((uintptr_t)workspace + 255) & ~(uintptr_t)255;
  alloc::CtlParams c{};
  c.shares = shares;
  c.shares_f64 = shares_dtype == EKV_F64 ? 1 : 0;
  c.shares_stride = shares_stride;
  c.lengths = lengths;
  c.evidence = evidence;
  c.audited = audited_blocks;
  c.released = released;
  c.released_stride = released_stride;
  c.weights = weights;
  c.rows = rows;
  c.width = width;
  c.recent = recent_blocks;
  c.cap = cap_above_blocks;
  c.header = (alloc::CtlHeader *)(base + l.header);
  c.row_slot = (int32_t *)(base + l.row_slot);
  c.slot_row = (int32_t *)(base + l.slot_row);
  c.req_blocks = (int32_t *)(base + l.req_blocks);
  c.req_weights = (double *)(base + l.req_weights);
  c.req_scores = (double *)(base + l.req_scores);
  c.req_pinned = (uint8_t *)(base + l.req_pinned);
  c.req_keep = (uint8_t *)(base + l.req_keep);
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(alloc::ctl_plan_kernel, dim3(1), dim3(alloc::kCtlPlanThreads), 0, s, c);
  hipLaunchKernelGGL(alloc::ctl_compact_kernel, dim3(rows), dim3(alloc::kThreads), 0, s, c);
  int rc = check_hip(hipGetLastError(), "ekv_controller_keep launch");
  if (rc != EKV_OK) return rc;
  // the objective over the requests (rows that take no part: empty requests after the others)
  alloc::Params p{};
  p.scores = c.req_scores;
  p.scores_stride = width;
  p.blocks = c.req_blocks;
  p.weights = objective == EKV_OBJ_SUM ? c.req_weights : nullptr;
  p.pinned = c.req_pinned;
  p.pinned_stride = width;
  p.rows = rows;
  p.width = width;
  p.budget = -1;  // the controller's: from the plan's header
  p.fraction = fraction;
  p.ctl = c.header;
  p.keep = c.req_keep;
  p.keep_stride = width;
  p.summary = summary;
  const uintptr_t inner = ((base + l.inner) + 255) & ~(uintptr_t)255;
  if (objective == EKV_OBJ_SUM) {
    set_sum_buffers(inner, rows, p);
    rc = alloc::launch_sum(p, s);
  } else {
    const MaxminLayout ml = maxmin_layout(rows, width);
    alloc::MaxminParams m{};
    m.p = p;
    set_maxmin_buffers(ml, inner, m);
    rc = alloc::launch_maxmin(m, rows, width, s);
  }
  if (rc != EKV_OK) return rc;
  hipLaunchKernelGGL(alloc::ctl_scatter_kernel, dim3(rows), dim3(alloc::kThreads), 0, s, c, keep, keep_stride);
  return check_hip(hipGetLastError(), "ekv_controller_keep scatter launch");
}
