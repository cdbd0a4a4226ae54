"""End-to-end parity of the hot path at the benchmark configurations.

Each case runs the chain a decode step runs: every layer recorded through RecordingPlane (the engine's
protocol -- the layer table attached, the rows selected, the flag set, the step plan built at the
first layer), the split-form shares over all recorded layers, and the uniform ranking at budget 0.5
with block 0 and the 4 newest blocks pinned, compacted into the view by the same kernel.  Against the
oracle:

* the records within 1e-3 of oracle.audit.tile_lse (float64) on the same keys and queries;
* the shares within 1e-4 of oracle.tile_shares.normalize over the device's own records (read as
  read_tile_rows reads them);
* the keep mask and the budget bit-exact with oracle.controller.keep_rows on the device's own shares,
  and the view and its lengths bit-exact with oracle.block_view.compact of that keep.

Reference: runtime/audit_kernel.py:34-109, 196-265; observe/tile_shares.py:58-173;
observe/allocation.py:39-91; observe/controller.py:398-451; runtime/block_view.py:36-56.
"""

import numpy as np
import pytest
import torch

import workloads
from observe.tile_shares import tile_shares
from oracle import audit as oa
from oracle import block_view as obv
from oracle import controller as ocon
from oracle import tile_shares as ots
from runtime.audit_kernel import TILE_BLOCKS, RecordingPlane
from runtime.block_view import uniform_view

pytestmark = pytest.mark.gpu
LSE_TOL, SHARE_TOL = 1e-3, 1e-4
FRACTION, RECENT = 0.5, 4


def check_records(got, want, what):
    """got / want: ``[2, rows, width, cells]`` of one layer.  The same cells written; m and
    u = m + log l within 1e-3."""
    assert np.array_equal(np.isnan(got[0]), np.isnan(want[0])), f"{what}: written cells differ"
    live = ~np.isnan(want[0])
    assert live.any(), what
    dm = float(np.abs(got[0][live] - want[0][live]).max())
    du = float(np.abs(ots.log_weights(got[0], got[1], 1)[live].astype(np.float64)
                      - ots.log_weights(want[0], want[1], 1)[live]).max())
    assert dm < LSE_TOL and du < LSE_TOL, f"{what}: |dm| {dm:.2e}, |du| {du:.2e}"
    return max(dm, du)


def shares_rank_view(plane, layers, batch, table, lens):
    """The device chain after the records: split-form shares, then the fused ranking + view."""
    blocks = torch.from_numpy(batch.blocks.astype(np.int32)).cuda()
    shares = tile_shares(plane.lse_address, plane._layers, layers, batch.rows, batch.width, plane.cells, None, blocks,
                         TILE_BLOCKS)
    keep, summary, view, view_lens = uniform_view(shares, blocks, table, lens, batch.block_size, fraction=FRACTION,
                                                  recent_blocks=RECENT)
    torch.cuda.synchronize()
    return [t.cpu().numpy() for t in (shares, keep, summary, view, view_lens)]


def check_shares_rank_view(planes, layers, batch, shares, keep, summary, view, view_lens, what):
    want = ots.normalize(ots.read_rows(planes, layers, np.arange(batch.rows), TILE_BLOCKS), batch.blocks, TILE_BLOCKS)
    assert np.array_equal(np.isnan(shares), np.isnan(want)), f"{what}: rows without evidence differ"
    ds = float(np.nanmax(np.abs(shares.astype(np.float64) - want)))
    assert ds < SHARE_TOL, f"{what}: shares off by {ds:.2e}"
    want_keep, budget = ocon.keep_rows(shares.astype(np.float64), batch.blocks, np.ones(batch.rows), FRACTION,
                                       RECENT, 0)
    assert int(summary[0]) == budget, f"{what}: budget {int(summary[0])} != {budget}"
    assert np.array_equal(keep, want_keep), f"{what}: keep differs in {int((keep != want_keep).sum())} blocks"
    want_view, want_lens = obv.compact(batch.table, batch.lens, want_keep.astype(bool), batch.block_size)
    assert np.array_equal(view, want_view), f"{what}: view differs"
    assert np.array_equal(view_lens, want_lens), f"{what}: view lengths differ"
    ties = boundary_ties(shares, keep, batch.blocks)
    print(f"{what}: shares within {ds:.2e}, budget {budget}, {int(keep.sum())} kept, {ties} rows tied at "
          "their quota boundary; keep, view and lengths bit-exact", flush=True)
    return ties


def boundary_ties(shares, keep, blocks):
    """Rows whose lowest kept open share equals a dropped open share (a tie the index rule breaks)."""
    ties = 0
    for r in range(len(blocks)):
        n = int(blocks[r])
        if n <= 1 + RECENT + 1:
            continue
        open_ = np.ones(n, bool)
        open_[0] = False
        open_[max(0, n - 1 - RECENT):] = False
        s, k = shares[r, :n][open_], keep[r, :n][open_].astype(bool)
        if k.any() and (~k).any() and np.isin(s[k].min(), s[~k]):
            ties += 1
    return ties


def engine_plane(layers, batch, caches, **kw):
    plane = RecordingPlane(layers, batch.rows, batch.width, batch.group_rows, batch.block_size, **kw)
    plane.attach([int(c.data_ptr()) for c in caches])
    plane.select(np.ones(batch.rows, bool), np.arange(batch.rows))
    plane.set(True)
    return plane


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_small_audit_chain(dtype):
    # 4 rows of {17, 64, 200, 512} tokens, 8 query / 2 KV heads, d 64, two layers
    batch, kv, q = workloads.config1()
    kv_t = torch.from_numpy(kv).to(dtype).cuda()
    q_t = torch.from_numpy(q).to(dtype).cuda()
    table, lens = torch.from_numpy(batch.table).cuda(), torch.from_numpy(batch.lens).cuda()
    scale = batch.head_dim ** -0.5
    layers = 2
    plane = engine_plane(layers, batch, [kv_t] * layers)
    for layer in range(layers):
        plane.record(f"model.layers.{layer}.self_attn.attn", table, lens, q_t, kv_t, scale)
    got = shares_rank_view(plane, layers, batch, table, lens)
    planes = plane.read_planes()
    kvh, qh = kv_t.float().cpu().numpy(), q_t.float().cpu().numpy()
    for layer in range(layers):
        want = oa.new_planes(1, batch.rows, batch.width, batch.group_rows)
        oa.tile_lse(want, qh, kvh[:, 0], batch.table, batch.lens, np.arange(batch.rows), np.ones(batch.rows), 1, 0,
                    scale, batch.block_size, batch.group_rows, [layer % batch.kv_heads])
        check_records(planes[:, layer], want[:, 0], f"small audit {dtype} layer {layer}")
    check_shares_rank_view(planes, layers, batch, *got, f"small audit {dtype}")


def test_llama3_decode_step_chain():
    # 128 rows of U[512, 8192] tokens, 32 / 8 heads, d 128, bf16, block 16; 32 layers, layer L auditing
    # KV group L mod 8 of its own cache (four rotating 100k-block pools)
    batch = workloads.config2_batch()
    layers, npools = 32, 4
    pools = [workloads.device_pool(batch, torch.bfloat16, seed=batch.seed + 101 * p) for p in range(npools)]
    q = torch.from_numpy(workloads.queries(batch, layers)).to(torch.bfloat16).cuda()
    table, lens = torch.from_numpy(batch.table).cuda(), torch.from_numpy(batch.lens).cuda()
    scale = batch.head_dim ** -0.5
    plane = engine_plane(layers, batch, [pools[layer % npools] for layer in range(layers)])
    for layer in range(layers):
        plane.record(f"model.layers.{layer}.self_attn.attn", table, lens, q[layer], pools[layer % npools], scale)
    got = shares_rank_view(plane, layers, batch, table, lens)
    planes = plane.read_planes()
    worst = 0.0
    for group in range(batch.kv_heads):  # the layers auditing one (pool, group) share its host keys
        members = [layer for layer in range(layers) if layer % batch.kv_heads == group]
        keys, table_c = workloads.host_keys(batch, pools[members[0] % npools], heads=[group])
        for layer in members:
            want = oa.new_planes(1, batch.rows, batch.width, batch.group_rows)
            oa.tile_lse(want, q[layer].float().cpu().numpy(), keys, table_c, batch.lens, np.arange(batch.rows),
                        np.ones(batch.rows), 1, 0, scale, batch.block_size, batch.group_rows, [group], key_heads=[0])
            worst = max(worst, check_records(planes[:, layer], want[:, 0], f"llama3 step layer {layer}"))
        del keys
    print(f"llama3 step: 32 layers' records within {worst:.2e}", flush=True)
    del pools
    torch.cuda.empty_cache()
    check_shares_rank_view(planes, layers, batch, *got, "llama3 decode step")


def test_skewed_long_context_chain_with_ties():
    # 8 rows of 131072 tokens + 120 Zipf(1.2) rows on [1024, 4096], 0.5% planted heavy hitters aligned
    # to the queries: heavy-tailed shares
    batch = workloads.config3_batch()
    layers = 4
    pools = [workloads.device_pool(batch, torch.bfloat16, seed=batch.seed + p) for p in range(2)]
    q0 = torch.from_numpy(workloads.queries(batch, 1)[0]).to(torch.bfloat16).cuda()
    for pool in pools:
        workloads.plant_heavy_hitters(batch, pool, q0)
    table, lens = torch.from_numpy(batch.table).cuda(), torch.from_numpy(batch.lens).cuda()
    scale = batch.head_dim ** -0.5
    plane = engine_plane(layers, batch, [pools[layer % 2] for layer in range(layers)])
    for layer in range(layers):
        plane.record(f"model.layers.{layer}.self_attn.attn", table, lens, q0, pools[layer % 2], scale)
    got = shares_rank_view(plane, layers, batch, table, lens)
    planes = plane.read_planes()
    for layer in range(layers):
        group = layer % batch.kv_heads
        keys, table_c = workloads.host_keys(batch, pools[layer % 2], heads=[group])
        want = oa.new_planes(1, batch.rows, batch.width, batch.group_rows)
        oa.tile_lse(want, q0.float().cpu().numpy(), keys, table_c, batch.lens, np.arange(batch.rows),
                    np.ones(batch.rows), 1, 0, scale, batch.block_size, batch.group_rows, [group], key_heads=[0])
        check_records(planes[:, layer], want[:, 0], f"skewed mix layer {layer}")
        del keys
    del pools
    torch.cuda.empty_cache()
    check_shares_rank_view(planes, layers, batch, *got, "skewed long-context mix")
    # the same rows ranked on their shares rounded to multiples of 2^-16: every ordinary block's share
    # (~1e-10 beside the heavy hitters) becomes 0, so nearly every quota ends inside a run of tied
    # shares and the lower block index decides
    shares = got[0]
    coarse = (np.round(np.nan_to_num(shares).astype(np.float64) * 2.0**16) / 2.0**16).astype(np.float32)
    blocks = torch.from_numpy(batch.blocks.astype(np.int32)).cuda()
    keep, summary, view, view_lens = (t.cpu().numpy() for t in uniform_view(
        torch.from_numpy(coarse).cuda(), blocks, table, lens, batch.block_size, fraction=FRACTION,
        recent_blocks=RECENT))
    want_keep, budget = ocon.keep_rows(coarse.astype(np.float64), batch.blocks, np.ones(batch.rows), FRACTION, RECENT, 0)
    assert int(summary[0]) == budget and np.array_equal(keep, want_keep), "tied ranking differs"
    want_view, want_lens = obv.compact(batch.table, batch.lens, want_keep.astype(bool), batch.block_size)
    assert np.array_equal(view, want_view) and np.array_equal(view_lens, want_lens), "tied view differs"
    ties = boundary_ties(coarse, keep, batch.blocks)
    print(f"skewed mix, coarse shares: {ties} of {batch.rows} rows tied at their quota boundary; bit-exact", flush=True)
    assert ties > 0, "no row's quota boundary fell on tied shares"


class E4M3Keys:
    """fp8 e4m3 key bytes on the host, decoded per gather (``keys[block, pos, head, :]``)."""

    LUT = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()

    def __init__(self, raw: np.ndarray) -> None:
        self.raw = raw

    def __getitem__(self, index):
        return self.LUT[self.raw[index]]


@pytest.fixture(scope="module")
def fp8_step():
    # 256 rows of U[2048, 32768] tokens, block 32, fp8 e4m3 keys with a per-tensor scale, bf16 queries,
    # 32 layers over two pools, the per-row timer on; the chain runs once for the tests below
    batch = workloads.config5_batch()
    layers = 32
    fp8 = torch.float8_e4m3fn
    k_scale = batch.extra["k_scale"]
    pools = [workloads.device_pool(batch, fp8, seed=batch.seed + i) for i in range(2)]
    q = torch.from_numpy(workloads.queries(batch, layers)).to(torch.bfloat16).cuda()
    table, lens = torch.from_numpy(batch.table).cuda(), torch.from_numpy(batch.lens).cuda()
    scale = batch.head_dim ** -0.5
    plane = engine_plane(layers, batch, [pools[layer % 2] for layer in range(layers)], timer=True)
    plane.plan(table, lens)  # what record() does at the first layer; fp8 keys carry a scale record() has not
    for layer in range(layers):
        plane.launch(layer, table, lens, q[layer], pools[layer % 2][:, 0], scale, k_scale=k_scale, planned=True)
    got = shares_rank_view(plane, layers, batch, table, lens)
    state = {"batch": batch, "pools": pools, "q": q, "scale": scale, "k_scale": k_scale, "got": got,
             "planes": plane.read_planes(), "cycles": plane.read_cycles(), "layers": layers}
    yield state
    state.clear()
    torch.cuda.empty_cache()


def test_fp8_step_shares_rank_view(fp8_step):
    s = fp8_step
    assert (s["cycles"] > 0).all(), "a row's cycles were not counted"
    check_shares_rank_view(s["planes"], s["layers"], s["batch"], *s["got"], "fp8 full step")


@pytest.mark.parametrize("part", range(4))
def test_fp8_step_records(fp8_step, part):
    # the records of all 32 layers, eight per test: layers auditing group g read pool g mod 2
    s = fp8_step
    batch = s["batch"]
    n = batch.blocks
    rows = np.arange(batch.rows)
    used = np.unique(np.concatenate([batch.table[r, : n[r]] for r in rows] + [np.zeros(1, np.int32)]))
    remap = np.zeros(int(batch.table.max()) + 1, dtype=np.int32)
    remap[used] = np.arange(len(used), dtype=np.int32)
    table_c = np.zeros_like(batch.table)
    for r in rows:
        table_c[r, : n[r]] = remap[batch.table[r, : n[r]]]
    idx = torch.from_numpy(used.astype(np.int64)).cuda()
    for group in (2 * part, 2 * part + 1):
        pool = s["pools"][group % 2]
        raw = pool[idx, 0][:, :, group : group + 1].view(torch.uint8).cpu().numpy()
        keys = E4M3Keys(raw)
        for layer in range(group, s["layers"], batch.kv_heads):
            want = oa.new_planes(1, batch.rows, batch.width, batch.group_rows)
            oa.tile_lse(want, s["q"][layer].float().cpu().numpy(), keys, table_c, batch.lens, rows,
                        np.ones(batch.rows), 1, 0, s["scale"], batch.block_size, batch.group_rows, [group],
                        k_scale=s["k_scale"], key_heads=[0])
            err = check_records(s["planes"][:, layer], want[:, 0], f"fp8 step layer {layer}")
            print(f"fp8 step layer {layer}: records within {err:.2e}", flush=True)
