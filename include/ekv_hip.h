/*
 * ekv_hip.h -- C ABI of libekv_hip.so, the MI355X (gfx950) implementation of KVScope's
 * audit / tile-share / ranking / block-table-view hot path.
 *
 * Every entry point takes raw device pointers, element strides, sizes and a hipStream_t
 * (passed as void*; NULL is the null stream).  No entry point allocates device memory
 * except the explicit memory helpers at the end, so the compute calls can run inside a
 * captured HIP graph.  Every call returns an int status:
 *
 *   EKV_OK           0   success
 *   EKV_EINVAL      -1   an argument is out of range (the Python layer raises ValueError)
 *   EKV_ELAUNCH     -2   a HIP call or kernel launch failed (RuntimeError)
 *   EKV_EUNSUPPORTED -3  the shape / dtype combination has no compiled kernel (ValueError)
 *
 * ekv_last_error() returns a message for the last failing call on the calling thread.
 *
 * Layout of the statistic planes (the layout the reference's pass and audit kernel write,
 * runtime/audit_kernel.py:97-109 and observe/tile_shares.py:4-11):
 *   float32 [2][layers][rows][width][cells]   plane 0 = tile max m, plane 1 = tile sum l
 * with `cells` = query rows recorded per block.  Unwritten cells keep whatever the caller
 * put there (the plane is NaN-filled once at allocation, runtime/audit_kernel.py:137).
 */
#ifndef EKV_HIP_H
#define EKV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EKV_OK 0
#define EKV_EINVAL (-1)
#define EKV_ELAUNCH (-2)
#define EKV_EUNSUPPORTED (-3)

/* element types of q / K */
#define EKV_F32 0
#define EKV_F16 1
#define EKV_BF16 2
#define EKV_FP8_E4M3 3 /* OCP e4m3fn, dequantised as k_scale * value */
#define EKV_F64 4      /* float64 shares (ekv_controller_keep) */

/* aggregates of the share normalisation (observe/tile_shares.py:55) */
#define EKV_AGG_MEAN 0
#define EKV_AGG_MAX 1

/* objectives of the controller's rule (Settings.objective, observe/controller.py:30) */
#define EKV_OBJ_SUM 0
#define EKV_OBJ_MAXMIN 1

const char *ekv_last_error(void);
int ekv_abi_version(void);

/*
 * The audit statistic of one attention layer.
 * Replaces tile_lse_kernel and its launch, runtime/audit_kernel.py:34-109 and :224-265.
 *
 * For every row r with *flag != 0 and select[r] != 0, every tile of tile_blocks (= 2) blocks
 * that starts before lens[r], and every query row q of the audited KV heads
 * group_first .. group_first + groups - 1, the kernel stores
 *     m = max_j s_j,   l = sum_j exp(s_j - m),   s_j = scale * k_scale * <q, k_j>
 * over the tile's keys j < lens[r], into plane 0 / plane 1 at
 *     lse[plane * lse_plane_stride + layer * lse_layer_stride + r * lse_row_stride
 *         + b * cells + h * group_rows + q]                 (h = 0 .. groups - 1)
 * for each block b of the tile with b * block_size < lens[r].  groups = 1 with
 * group_first = layer % kv_heads is the reference's one-group-per-layer audit
 * (runtime/audit_kernel.py:250); groups = kv_heads audits every KV head.
 *
 * q      : [tokens, q_heads, head_dim] with strides (q_stride_token, q_stride_head), row r's
 *          query is token qrow[r]; its KV head h uses query heads h*group_rows .. +group_rows-1.
 * keys   : element (blk, pos, h, dim) at blk*k_stride_block + pos*k_stride_pos + h*k_stride_head + dim
 *          (the keys view kv_cache[:, 0] of a [blocks, 2, block, heads, dim] cache).
 * table  : int32 [rows, >= width] with row stride table_stride; lens, qrow: int32 [rows];
 *          select: uint8 [rows]; flag: uint32 device scalar.
 * cycles : optional uint64 [cycles_rows]; when non-NULL every unit of work adds its
 *          s_memtime duration to cycles[r] (r < cycles_rows), for the first audited head only
 *          (the pass's timer, mlir_pass/lib/eKVTimer.cpp:1348-1387).
 * chunk_tiles: the fewest tiles one wavefront takes (0 = 1).  The live tiles of all selected rows
 *          form one list split into equal contiguous slices, one per wavefront of a grid the GPU
 *          holds at once; a larger value shrinks the grid for small batches.
 */
int ekv_audit_tile_lse(const void *q, int q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                       const void *keys, int kv_dtype, int64_t k_stride_block, int64_t k_stride_pos,
                       int64_t k_stride_head, float k_scale, const int32_t *table, int64_t table_stride,
                       const int32_t *lens, const int32_t *qrow, const uint8_t *select,
                       const uint32_t *flag, float *lse, int64_t lse_plane_stride,
                       int64_t lse_layer_stride, int64_t lse_row_stride, int32_t cells,
                       uint64_t *cycles, int32_t cycles_rows, float scale, int32_t layer,
                       int32_t group_first, int32_t groups, int32_t group_rows, int32_t rows,
                       int32_t width, int32_t block_size, int32_t tile_blocks, int32_t head_dim,
                       int32_t chunk_tiles, void *stream);

/*
 * The step plan of the audit: the work list every audit launch of one decode step shares.
 * Replaces the per-launch part of RecordingPlane.launch that recomputes the tiles of the selected
 * rows (runtime/audit_kernel.py:239-241 with the grid's early exits at :65-69): the launches of a
 * step read the same view table, lengths, selected rows and query tokens (runtime/block_view.py
 * :283-295 builds them once per step), so the list of (row, tile, block ids, query token) is built
 * once here, by two kernels on `stream`, and each ekv_audit_tile_lse_planned launch reads its
 * share of it.  With the flag off the plan is empty.
 * ekv_audit_plan_bytes(plan_rows, plan_width): device bytes of a plan for any batch of at most
 * plan_rows x plan_width on the current device (0 if too large); the buffer must be 256-byte
 * aligned and must not be in use by a running launch when it is rebuilt.
 */
size_t ekv_audit_plan_bytes(int32_t plan_rows, int32_t plan_width);
int ekv_audit_plan(const int32_t *table, int64_t table_stride, const int32_t *lens, const int32_t *qrow,
                   const uint8_t *select, const uint32_t *flag, int32_t rows, int32_t width,
                   int32_t block_size, int32_t tile_blocks, void *plan, size_t plan_bytes,
                   int32_t plan_rows, int32_t plan_width, void *stream);

/*
 * ekv_audit_tile_lse reading its work list from a plan built by ekv_audit_plan from the same
 * table, lengths, selection and query tokens: the same records and cycles, without the per-launch
 * scan of the rows, and for any number of rows (ekv_audit_tile_lse keeps per-row offsets in LDS and
 * takes at most 6000).  Replaces tile_lse_kernel + RecordingPlane.launch, runtime/audit_kernel.py
 * :34-109 and :224-265, as ekv_audit_tile_lse does.  Shapes without an MFMA form (fp32 keys,
 * 8-token blocks, fp8 rows of 32 dimensions) run its VALU form (ekv_audit_shape).
 */
int ekv_audit_tile_lse_planned(const void *q, int q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                               const void *keys, int kv_dtype, int64_t k_stride_block, int64_t k_stride_pos,
                               int64_t k_stride_head, float k_scale, const int32_t *table,
                               int64_t table_stride, const int32_t *lens, const int32_t *qrow,
                               const uint8_t *select, const uint32_t *flag, float *lse,
                               int64_t lse_plane_stride, int64_t lse_layer_stride, int64_t lse_row_stride,
                               int32_t cells, uint64_t *cycles, int32_t cycles_rows, float scale,
                               int32_t layer, int32_t group_first, int32_t groups, int32_t group_rows,
                               int32_t rows, int32_t width, int32_t block_size, int32_t tile_blocks,
                               int32_t head_dim, const void *plan, size_t plan_bytes, int32_t plan_rows,
                               int32_t plan_width, void *stream);

/*
 * Which audit launches have a kernel for a shape: EKV_AUDIT_SELF_CONTAINED (ekv_audit_tile_lse) and
 * EKV_AUDIT_PLANNED (ekv_audit_tile_lse_planned and ekv_audit_tile_lse_layers), or 0.  The planned
 * launch takes every shape the reference's kernel takes (runtime/audit_kernel.py:73, :128-131): fp32,
 * f16 and bf16 queries with keys of the same type, or fp8 keys with bf16 queries; head_dim 32 to 256
 * (rows of 16 to 1024 bytes, powers of two); tiles of a power of two of tokens, 16 or more.  On the
 * MFMA form: 16-bit or fp8 keys in tiles of 32 tokens or more (head_dim 32 for 16-bit keys, 64 to 256);
 * the VALU form takes the rest.  The self-contained launch lacks some VALU shapes (head_dim 32 or 256
 * on the VALU, rows of 64 bytes or less in 8-token blocks).
 */
#define EKV_AUDIT_SELF_CONTAINED 1
#define EKV_AUDIT_PLANNED 2
int ekv_audit_shape(int q_dtype, int kv_dtype, int32_t head_dim, int32_t block_size);

/* One layer of a multi-layer audit launch (ekv_audit_tile_lse_layers). */
typedef struct ekv_audit_layer {
  const void *q;       /* the layer's queries, with the call's shared strides */
  const void *keys;    /* the layer's key cache view, with the call's shared strides */
  int32_t layer;       /* the plane layer its records go to */
  int32_t group_first; /* its first audited KV head (layer % kv_heads for one group) */
  int32_t q_head0;     /* the query head that q's head 0 holds: 0, or group_first * group_rows
                          for a staged copy of the group's heads (ekv_audit_stage_queries) */
  float scale;         /* its logit scale */
  float k_scale;       /* its key dequantisation scale (1 for 16-bit keys) */
  int32_t pad;
} ekv_audit_layer_t;

/*
 * The planned audit of several layers of one decode step in one launch per 32 layers: the records
 * and cycles of ekv_audit_tile_lse_planned for each entry of `layers`, bit for bit, after every
 * layer has run.  Replaces the per-layer launches of RecordingPlane.record
 * (runtime/audit_kernel.py:196-265): a step's launches differ only in the layer (its queries, keys,
 * records and scale), so one launch amortises the launch's fixed costs (first key requests, the
 * spread of the workgroups' ends) over all of them.  The shared arguments are those of
 * ekv_audit_tile_lse_planned.  With q_by_row != 0, row r's query is row r of each layer's q (a
 * staged copy) instead of token qrow[r].  Every shape with EKV_AUDIT_PLANNED in ekv_audit_shape().
 */
int ekv_audit_tile_lse_layers(const ekv_audit_layer_t *layers, int32_t n_layers, int32_t q_by_row,
                              int q_dtype, int64_t q_stride_token, int64_t q_stride_head, int kv_dtype,
                              int64_t k_stride_block, int64_t k_stride_pos, int64_t k_stride_head,
                              const int32_t *table, int64_t table_stride, const int32_t *lens,
                              const int32_t *qrow, const uint8_t *select, const uint32_t *flag, float *lse,
                              int64_t lse_plane_stride, int64_t lse_layer_stride, int64_t lse_row_stride,
                              int32_t cells, uint64_t *cycles, int32_t cycles_rows, int32_t groups,
                              int32_t group_rows, int32_t rows, int32_t width, int32_t block_size,
                              int32_t tile_blocks, int32_t head_dim, const void *plan, size_t plan_bytes,
                              int32_t plan_rows, int32_t plan_width, void *stream);

/*
 * A layer's queries staged for ekv_audit_tile_lse_layers, so that a launch after the last layer
 * reads them after the engine has reused the query memory (the query tensor of runtime/audit_kernel.py
 * :196-203 lives only for its layer's forward):
 *     staged[r * staged_row_stride + h * head_dim + e] = q[qrow[r] * q_stride_token
 *                                                         + (head_first + h) * q_stride_head + e]
 * for h < heads, e < head_dim and every row r < rows with select[r] != 0, when *flag != 0 (nothing
 * otherwise, like the audit).  16-bit or fp32 queries; 16-byte-aligned rows.
 */
int ekv_audit_stage_queries(const void *q, int q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                            int32_t head_first, int32_t heads, int32_t head_dim, const int32_t *qrow,
                            const uint8_t *select, const uint32_t *flag, int32_t rows, void *staged,
                            int64_t staged_row_stride, void *stream);

/*
 * Exact per-block attention shares of the chosen rows, from the statistic planes.
 * Replaces read_tile_rows + normalize_tile_lse (observe/tile_shares.py:129-173 and :58-103),
 * computing on the device what the reference copies to the host and normalises with NumPy.
 *
 * For output row i the source row is row_ids[i] (row_ids NULL: row i), of row_blocks[i]
 * blocks (row_blocks NULL: all `width`).  The statistic is read for layers 0 .. layers-1 and
 * the `cells` query rows of each block:  u = m + log(l) - log(tile_blocks), a partial last tile's
 * blocks regain log(tile_blocks / valid_in_tail), cells at b >= row_blocks are dropped, each
 * (layer, query row) with a finite value is a softmax over the row's blocks, and the result
 * is their mean (EKV_AGG_MEAN) or the renormalised per-block max (EKV_AGG_MAX).
 * shares[i * shares_stride + b], float32, b < width: 0 beyond the row's blocks, all NaN for
 * a row with no finite value.
 */
int ekv_tile_shares(const float *lse, int64_t lse_plane_stride, int64_t lse_layer_stride,
                    int64_t lse_row_stride, int32_t layers, int32_t cells, int32_t width,
                    const int32_t *row_ids, const int32_t *row_blocks, int32_t nrows,
                    int32_t tile_blocks, int32_t aggregate, float *shares, int64_t shares_stride,
                    void *stream);

/*
 * ekv_tile_shares with a workspace, the same result (the same rules; float sums in another
 * fixed order): each row's layers are split over several workgroups, which write per-block
 * partial sums into the workspace, so a long row no longer sets the time on one compute unit.
 * For 4 query rows per block, rows of at most 512 blocks and at most 65536 rows, the last of a
 * row's workgroups to finish adds the partials and writes the row (it learns that it is last from
 * a per-row arrival counter in the workspace); other shapes combine them in a second kernel.
 * Replaces the same reference code as ekv_tile_shares.
 * workspace: ekv_tile_shares_workspace(nrows, width, layers) bytes of device memory (256 KB of
 * arrival counters, then the partials and their counts, which the last workgroup of a row reads
 * as they land: a slot reads zero until its value has arrived).  Fill it with zeros once before its
 * first use; every call leaves all of it at zero again, for calls of any shape, as long as nothing
 * else writes into the workspace.  Calls that share one workspace must not overlap.
 */
size_t ekv_tile_shares_workspace(int32_t nrows, int32_t width, int32_t layers);
int ekv_tile_shares_ws(const float *lse, int64_t lse_plane_stride, int64_t lse_layer_stride,
                       int64_t lse_row_stride, int32_t layers, int32_t cells, int32_t width,
                       const int32_t *row_ids, const int32_t *row_blocks, int32_t nrows,
                       int32_t tile_blocks, int32_t aggregate, float *shares, int64_t shares_stride,
                       void *workspace, size_t workspace_bytes, void *stream);

/*
 * ekv_tile_shares_ws without a workspace argument and without allocating: the split form's
 * partials go to a scratch array of EKV_TILE_SHARES_SCRATCH_BYTES that the library holds on every
 * device it runs on, from the first call on that device until the process ends.  The same
 * kernels, so the same shares as ekv_tile_shares_ws, bit for bit.
 * No counterpart in the reference: this entry point is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * A call whose ekv_tile_shares_workspace(nrows, width, layers) exceeds the scratch is refused
 * with EKV_EINVAL (e.g. 128 rows x 512 blocks x 32 layers need 8.7 MB and fit).  The scratch
 * starts zeroed, as a workspace must.  Every call on one
 * device uses that device's one scratch: calls that overlap on one device (two streams, two
 * threads, two graphs replayed at once) race, so a process calls it from one stream at a time
 * (or orders its streams).
 */
#define EKV_TILE_SHARES_SCRATCH_BYTES (16u << 20)
int ekv_tile_shares_noalloc(const float *lse, int64_t lse_plane_stride, int64_t lse_layer_stride,
                            int64_t lse_row_stride, int32_t layers, int32_t cells, int32_t width,
                            const int32_t *row_ids, const int32_t *row_blocks, int32_t nrows,
                            int32_t tile_blocks, int32_t aggregate, float *shares, int64_t shares_stride,
                            void *stream);

/*
 * The workspace's status, after a failure of the split form's wait.  The single-kernel form waits,
 * a bounded number of reloads, for the partials of a row's other workgroups; a partial that has not
 * landed by then is taken as lost, the row comes out as NaN, and the workspace's sticky status word
 * is set, because the lost value may still land in its slot after the call.  While it is set every
 * call on that workspace leaves the slots alone and returns NaN rows.  No counterpart in the
 * reference (its normalisation runs on the host).
 * ekv_tile_shares_status: waits for the device, then reads the status word of `workspace` (NULL:
 * this device's scratch of ekv_tile_shares_noalloc) into *status (0: sound).
 * ekv_tile_shares_reset: zeroes `workspace_bytes` of `workspace` (NULL: the scratch) on `stream`
 * with a kernel, status included, after the calls before it on that stream.
 * ekv_tile_shares_test_wait: for tests of this failure path only -- sets, for every later call in
 * the process, the reloads of the wait (0: the default) and, with lose != 0, makes every wait run
 * to its limit without taking a value, so that the path runs with every kernel ending normally.
 */
int ekv_tile_shares_status(const void *workspace, int32_t *status);
int ekv_tile_shares_reset(void *workspace, size_t workspace_bytes, void *stream);
int ekv_tile_shares_test_wait(int32_t spin_limit, int32_t lose);

/*
 * The same normalisation from u values already formed, u[layer][row][block][cell]
 * (normalize_tile_lse's own input, observe/tile_shares.py:58-103).
 */
int ekv_normalize_tile_lse(const float *u, int64_t u_layer_stride, int64_t u_row_stride,
                           int32_t layers, int32_t cells, int32_t width, const int32_t *row_blocks,
                           int32_t nrows, int32_t tile_blocks, int32_t aggregate, float *shares,
                           int64_t shares_stride, void *stream);

/*
 * The `uniform` budget split and the per-row ranking, on the device.
 * Replaces Controller._allocate's pin / budget rules (observe/controller.py:398-451) feeding
 * allocate(..., "uniform") (observe/allocation.py:39-91).
 *
 * Rows with measured[r] != 0 (measured NULL: every row) and blocks[r] > 0 take part.
 *  - pinned block of row r: pinned[r, b] != 0 when `pinned` is given (Request.pinned);
 *    otherwise block 0, blocks >= max(0, n-1-recent_blocks), and blocks >= pin_from[r]
 *    (pin_from NULL: none).
 *  - released[r, b] != 0 (NULL: none) removes block b from the request (controller.py:425-431).
 *  - budget >= 0 is used as given (allocate's budget); budget < 0 computes the controller's
 *    max(floor, ceil(fraction * total)) in IEEE double, total = sum of blocks[r].
 *  - free blocks are split by largest remainder in IEEE double, then each row keeps its quota
 *    of open blocks by (share desc, block index asc).  Shares are max(score, 0) as float32.
 * width at most 262144: rows up to 12288 blocks wide are ranked in registers and LDS by one
 * workgroup each, wider rows by a streaming workgroup per row over the scores in memory.
 * scores[r, b], pinned[r, b] and released[r, b] are read for every b < width (rows of `width`
 * readable entries; the values past blocks[r] are ignored).
 * keep[r, b] (uint8, row stride keep_stride) is written for every r < rows, b < width: 1 for
 * rows that do not take part and for b >= blocks[r], else pinned | chosen, 0 for released.
 * summary (optional int64[6]): budget, total, floor (pinned blocks), status, requests, free.
 * status != 0 means the budget could not hold the pinned blocks (allocate's ValueError).
 * Explicit pinned / released masks need ekv_rank_uniform_ws; ekv_rank_uniform rejects them.
 */
int ekv_rank_uniform(const float *scores, int64_t scores_stride, const int32_t *blocks,
                     const uint8_t *measured, const uint8_t *pinned, int64_t pinned_stride,
                     const int32_t *pin_from, int32_t recent_blocks, const uint8_t *released,
                     int64_t released_stride, int32_t rows, int32_t width, double fraction,
                     int64_t budget, uint8_t *keep, int64_t keep_stride, int64_t *summary,
                     void *stream);

/*
 * ekv_rank_uniform_ws for float64 scores, ranking the float64 shares themselves.  Replaces
 * allocate(..., "uniform") on float64 Request.scores (observe/allocation.py:39-91, with
 * Request.shares at :46-52) and the controller's pins and budget (observe/controller.py:398-451),
 * as ekv_rank_uniform_ws does.  Each request's share of an open block is max(s, 0) / total with
 * total NumPy's sum of the clamped scores of its existing blocks (1 / n for a total <= 0), so two
 * scores that divide to one share tie and go to the lower block index as the reference's stable
 * argsort orders them; NaN shares rank last.
 * workspace: ekv_rank_uniform64_workspace(rows) bytes of device memory the call may overwrite.
 */
size_t ekv_rank_uniform64_workspace(int32_t rows);
int ekv_rank_uniform64(const double *scores, int64_t scores_stride, const int32_t *blocks,
                       const uint8_t *measured, const uint8_t *pinned, int64_t pinned_stride,
                       const int32_t *pin_from, int32_t recent_blocks, const uint8_t *released,
                       int64_t released_stride, int32_t rows, int32_t width, double fraction,
                       int64_t budget, uint8_t *keep, int64_t keep_stride, int64_t *summary,
                       void *workspace, size_t workspace_bytes, void *stream);

/*
 * ekv_rank_uniform followed by ekv_compact_view on the keep it writes, in one kernel: the view
 * build of allocate(..., "uniform") (observe/allocation.py:39-91, with the controller's pins and
 * budget, observe/controller.py:398-451) and compact_block_table (runtime/block_view.py:36-56).
 * The reference runs the two as separate steps; here each row's workgroup compacts its table row
 * from the keep bytes it has just decided, kept in LDS.  keep, summary, view_table and view_lens
 * are written exactly as the two calls in sequence write them (rows of blocks[r] blocks for the
 * ranking, of ceil(seq_lens[r] / block_size) for the view).  No explicit pinned / released masks.
 * counts (int64[rows][5], NULL: none): DecodeView's read counters, accumulated as ekv_build_view
 * accumulates them for live decoding rows outside the audit with the same keep
 * (runtime/block_view.py:313-329); the view is then ekv_build_view's with that keep.
 */
int ekv_rank_uniform_view(const float *scores, int64_t scores_stride, const int32_t *blocks,
                          const uint8_t *measured, const int32_t *pin_from, int32_t recent_blocks,
                          int32_t rows, int32_t width, double fraction, int64_t budget, uint8_t *keep,
                          int64_t keep_stride, int64_t *summary, const int32_t *table, int64_t table_stride,
                          const int32_t *seq_lens, int32_t block_size, int32_t *view_table, int64_t view_stride,
                          int32_t *view_lens, int64_t *counts, void *stream);

/*
 * ekv_rank_uniform with a caller-owned device workspace of 2 * rows int32, where a first
 * kernel counts each row's existing and pinned blocks when explicit masks are given.
 */
int ekv_rank_uniform_ws(const float *scores, int64_t scores_stride, const int32_t *blocks,
                        const uint8_t *measured, const uint8_t *pinned, int64_t pinned_stride,
                        const int32_t *pin_from, int32_t recent_blocks, const uint8_t *released,
                        int64_t released_stride, int32_t rows, int32_t width, double fraction,
                        int64_t budget, uint8_t *keep, int64_t keep_stride, int64_t *summary,
                        int32_t *workspace, void *stream);

/*
 * The `sum` budget split: allocate(requests, budget, "sum"), observe/allocation.py:55-123.
 *
 * Row r is a request of blocks[r] blocks (at most width) with float64 scores, weight weights[r]
 * (NULL: 1.0) and pinned blocks pinned[r][b] (NULL: the first and the last).  Its shares are
 * max(s, 0) / total (NumPy's float64 sum, reproduced in its order) or 1 / n when total <= 0.  The
 * call keeps every pinned block and the free = budget - pinned unpinned blocks of highest
 * weight * share, ties to the newer block, then the earlier request; every block when budget >=
 * the blocks of all rows.  keep[r][b] is 1 or 0, and 1 past the row's blocks.  summary (int64[6],
 * may be NULL): budget, blocks of all rows, pinned blocks, status (1: the budget is below the
 * pinned blocks -- the reference raises ValueError -- and every block is kept), requests, free.
 * workspace: ekv_rank_sum_workspace(rows) bytes of device memory the call may overwrite (16 KB a
 * row of it lists the blocks left after the select's first digit).  rows at most 16777215 (the tie
 * key holds the request in 16 bits up to 65536 requests, in up to 24 past them), width at most
 * 262144 (the first two passes stream the rows from memory; the later ones read the list, or the
 * rows again when it outgrows its room).
 */
size_t ekv_rank_sum_workspace(int32_t rows);
int ekv_rank_sum(const double *scores, int64_t scores_stride, const int32_t *blocks, const double *weights,
                 const uint8_t *pinned, int64_t pinned_stride, int32_t rows, int32_t width, int64_t budget,
                 uint8_t *keep, int64_t keep_stride, int64_t *summary, void *workspace, size_t workspace_bytes,
                 void *stream);

/*
 * The `maxmin` budget split: allocate(requests, budget, "maxmin"), observe/allocation.py:55-76 and
 * :126-166.  Rows, shares, pins, keep and summary as ekv_rank_sum (no weights).  The call raises
 * the lowest retained share (pinned shares plus the kept open blocks, each request's open blocks
 * taken in stable descending share order) by the reference's 60-step bisection of the level, then
 * gives the leftover one block at a time to the request of the lowest (retained share, index).
 * rows <= 16777215 (past 8192 requests the bisection keeps each request's state in the workspace),
 * width <= 262144 (requests up to 12288 blocks sort in LDS, wider ones in global memory, in a
 * second buffer the workspace includes; the level positions take 32 bits past 65535 blocks).
 * workspace:
 * ekv_rank_maxmin_workspace(rows, width) bytes of device memory.
 */
size_t ekv_rank_maxmin_workspace(int32_t rows, int32_t width);
int ekv_rank_maxmin(const double *scores, int64_t scores_stride, const int32_t *blocks, const uint8_t *pinned,
                    int64_t pinned_stride, int32_t rows, int32_t width, int64_t budget, uint8_t *keep,
                    int64_t keep_stride, int64_t *summary, void *workspace, size_t workspace_bytes, void *stream);

/*
 * The controller's keep rule under the `sum` or `maxmin` objective: Controller._allocate,
 * observe/controller.py:398-451, with allocate(..., "sum" | "maxmin").  (The `uniform` objective is
 * ekv_rank_uniform_ws with the same rows, pins and released blocks.)
 *
 * Row r takes part when lengths[r] > cap_above_blocks and evidence[r] != 0 (:402-408).  Its request
 * is its n = min(lengths[r], width) blocks less the freed ones (released[r][b] != 0; NULL: none),
 * in order, scored by shares[r][b] (float32 or float64, zero past the row's evidence), weighted by
 * weights[r] (NULL: 1.0; `sum` only); block 0, blocks >= n - 1 - recent_blocks and blocks >=
 * audited_blocks[r] (NULL: none) are pinned (:420-424).  The budget is max(pinned, ceil(fraction *
 * blocks)) over every block of the taking-part rows, freed ones included (:435-437), and it is split
 * across the requests as ekv_rank_sum / ekv_rank_maxmin split theirs, the requests numbered in row
 * order.  keep[r][b] (uint8): the request's decision at a remaining block, 0 at a freed block, 1
 * past the row and in every row that takes no part.  summary (int64[6], may be NULL): budget, blocks
 * of the requests, pinned blocks, status, requests, free.  workspace:
 * ekv_controller_keep_workspace(objective, rows, width) bytes the call may overwrite.  rows at most
 * 16777215, width at most 262144 (`maxmin` past 12288 blocks: rows x width below 2^31).
 */
size_t ekv_controller_keep_workspace(int32_t objective, int32_t rows, int32_t width);
int ekv_controller_keep(int32_t objective, const void *shares, int32_t shares_dtype, int64_t shares_stride,
                        const int32_t *lengths, const uint8_t *evidence, const int32_t *audited_blocks,
                        const uint8_t *released, int64_t released_stride, const double *weights, int32_t rows,
                        int32_t width, int32_t recent_blocks, int32_t cap_above_blocks, double fraction,
                        uint8_t *keep, int64_t keep_stride, int64_t *summary, void *workspace,
                        size_t workspace_bytes, void *stream);

/*
 * compact_block_table (runtime/block_view.py:36-56).
 * keep'[r, b] = (keep[r, b] | b == 0 | b == n-1) & b < n,  n = ceil(seq_lens[r] / block_size).
 * view_table row r = table row r stably partitioned: keep' entries first, the rest after them,
 * each in original order (all `width` entries).  view_lens[r] = (sum keep' - 1) * block_size
 * + seq_lens[r] - (n-1) * block_size for n > 0, else 0.
 */
int ekv_compact_view(const int32_t *table, int64_t table_stride, const int32_t *seq_lens,
                     const uint8_t *keep, int64_t keep_stride, int32_t rows, int32_t width,
                     int32_t block_size, int32_t *view_table, int64_t view_stride,
                     int32_t *view_lens, void *stream);

/*
 * DecodeView.build's keep composition fused with the compaction and the read
 * counters (runtime/block_view.py:272-295 and :297-329).
 * keep = committed | !live | audited[r] | !decoding[r], then & !released  (committed NULL:
 * all ones; audited / decoding / released NULL: none / all decoding / none).
 * counts (optional int64[rows][5], row-major, accumulated): row r adds its read, full, audit,
 * untrimmed and expired blocks (decode rows only) to counts[5r .. 5r+4]; DecodeView._count's
 * five totals are the column sums.  Each row's workgroup owns its slot, so the counters need no
 * atomics; calls that share a counts buffer must be ordered (one stream).  view_table and
 * view_lens may be NULL (counts only, as DecodeView.skip needs).
 */
int ekv_build_view(const int32_t *table, int64_t table_stride, const int32_t *seq_lens,
                   const uint8_t *committed, int64_t committed_stride, const uint8_t *released,
                   int64_t released_stride, const uint8_t *audited, const uint8_t *decoding,
                   int32_t live, int32_t rows, int32_t width, int32_t block_size,
                   int32_t *view_table, int64_t view_stride, int32_t *view_lens, int64_t *counts,
                   void *stream);

/*
 * SGLang's key-value index list compaction, the token-granular form of the view.
 * Replaces plan_kernel, gather_kernel and SlotCompactor.compact, runtime/sglang_compact.py:22-167.
 *
 * Request r reads slots[indptr[r] .. indptr[r + 1]) (int32 offsets, slots of slot_bytes = 4 or
 * 8 bytes).  Each block_tokens consecutive entries form a block.  Row r keeps block b when
 *     b < blocks_r and (b == 0 or b == blocks_r - 1 or whole_r or (r < n_real and keep[r][b]))
 * with whole_r = !active or r >= n_real or (audit != NULL and r < n_real and audit[r]); a row
 * has at most `width` blocks.  The call writes table[r][k] (the k-th kept block), lens[r] (the
 * new length: kept blocks times block_tokens less the unfilled part of the last block, 0 for an
 * empty row), new_indptr[0 .. n_rows] (their running sum) and out[0 .. new_indptr[n_rows]) (the
 * kept entries in order), and adds to counts[0..4] (when non-NULL) the real rows' blocks read,
 * blocks a full read would read, blocks read by audited rows, blocks read by rows that kept every
 * token while the policy is live, and blocks read while it is not.  `entries` is indptr[n_rows],
 * which the host knows.  With write_back, new_indptr is copied into indptr and the new list into
 * slots[0 .. new total) in place (entries past the new total keep their old values).  No host
 * synchronisation; up to 6000 rows the gather keeps the offsets in LDS, more rows take one more
 * kernel that writes them to new_indptr first.
 */
int ekv_compact_slots(int32_t *indptr, void *slots, int32_t slot_bytes, const uint8_t *keep,
                      int64_t keep_stride, const uint8_t *audit, int32_t active, int32_t n_real,
                      int32_t n_rows, int32_t width, int32_t block_tokens, int64_t entries,
                      int32_t *new_indptr, int32_t *lens, int32_t *table, int64_t table_stride,
                      void *out, int64_t *counts, int32_t write_back, void *stream);

/*
 * Device memory, copies and IPC for the statistic planes.  They replace the ctypes calls
 * into libcudart of runtime/audit.py:17-23, :55-60, runtime/audit_kernel.py:146-158 and
 * observe/cuda.py:12-58.  These are not for hot loops.
 */
int ekv_malloc(void **ptr, size_t bytes);
int ekv_free(void *ptr);
int ekv_memset(void *ptr, int value, size_t bytes);
int ekv_memcpy_h2d(void *dst, const void *src, size_t bytes);
int ekv_memcpy_d2h(void *dst, const void *src, size_t bytes);
int ekv_ipc_handle(const void *ptr, uint8_t handle[64]);
int ekv_ipc_open(const uint8_t handle[64], void **ptr);
int ekv_synchronize(void);
int ekv_device_count(int *count);

#ifdef __cplusplus
}
#endif

#endif /* EKV_HIP_H */
