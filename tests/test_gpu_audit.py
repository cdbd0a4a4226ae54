"""GPU parity of the audit kernel (ekv_audit_tile_lse) with the oracle, through the drop-in
RecordingPlane: tile LSE within 1e-3, the tile max within 1e-3, the same cells written
(runtime/audit_kernel.py:34-109 and :190-265 of the reference)."""

import numpy as np
import pytest
import torch

import workloads
from oracle import audit as oa
from oracle import tile_shares as ots
from runtime.audit_kernel import TILE_BLOCKS, RecordingPlane

pytestmark = pytest.mark.gpu
LSE_TOL = 1e-3


def flag(plane, on=True):
    """The audit flag through the engine's protocol: attach once, then set."""
    plane.attach([0])
    plane.set(on)


def record(plane, layer, table, lens, q, keys, scale, select=None, **kw):
    rows = plane.rows
    plane.select(np.ones(rows, bool) if select is None else np.asarray(select, bool), np.arange(rows))
    plane.launch(layer, table, lens, q, keys, scale, **kw)
    torch.cuda.synchronize()
    return plane.read_planes()


def assert_parity(got, want, what=""):
    """Same cells written; m and u = m + log l within 1e-3."""
    assert np.array_equal(np.isnan(got[0]), np.isnan(want[0])), f"{what}: written cells differ"
    live = ~np.isnan(want[0])
    assert live.any()
    dm = np.abs(got[0][live] - want[0][live]).max()
    u_got = ots.log_weights(got[0], got[1], 1)[live]
    u_want = ots.log_weights(want[0], want[1], 1)[live]
    du = np.abs(u_got.astype(np.float64) - u_want).max()
    print(f"{what}: max |dm| {dm:.2e}, max |du| {du:.2e} over {live.sum()} cells", flush=True)
    assert dm < LSE_TOL and du < LSE_TOL, what


def config1_device(dtype):
    batch, kv, q = workloads.config1()
    kv_t = torch.from_numpy(kv).to(dtype).cuda()
    q_t = torch.from_numpy(q).to(dtype).cuda()
    # the oracle sees exactly the values the kernel reads
    return batch, kv_t, q_t, kv_t.float().cpu().numpy(), q_t.float().cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_config1_every_layer(dtype):
    batch, kv_t, q_t, kv, q = config1_device(dtype)
    scale = batch.head_dim ** -0.5
    layers = 4
    plane = RecordingPlane(layers, batch.rows, batch.width, batch.group_rows, batch.block_size)
    flag(plane)
    table = torch.from_numpy(batch.table).cuda()
    lens = torch.from_numpy(batch.lens).cuda()
    want = oa.new_planes(layers, batch.rows, batch.width, batch.group_rows)
    for layer in range(layers):
        plane.select(np.ones(batch.rows, bool), np.arange(batch.rows))
        plane.record(f"layer.{layer}", table, lens, q_t, kv_t, scale)
        oa.tile_lse(want, q, kv[:, 0], batch.table, batch.lens, np.arange(4), np.ones(4), 1, layer, scale,
                    batch.block_size, batch.group_rows, [layer % batch.kv_heads])
    torch.cuda.synchronize()
    assert plane.layer_names == [f"layer.{i}" for i in range(layers)]
    assert_parity(plane.read_planes(), want, f"config1 {dtype}")


def test_flag_and_selection_gate():
    batch, kv_t, q_t, kv, q = config1_device(torch.float32)
    plane = RecordingPlane(1, batch.rows, batch.width, batch.group_rows, batch.block_size)
    table = torch.from_numpy(batch.table).cuda()
    lens = torch.from_numpy(batch.lens).cuda()
    flag(plane, False)
    off = record(plane, 0, table, lens, q_t, kv_t[:, 0], 0.125)
    assert np.isnan(off).all(), "a launch with the flag off wrote the statistic"
    flag(plane, True)
    part = record(plane, 0, table, lens, q_t, kv_t[:, 0], 0.125, select=[1, 0, 1, 0])
    assert np.isnan(part[:, 0, 1]).all() and np.isnan(part[:, 0, 3]).all()
    assert not np.isnan(part[0, 0, 0, :2]).any() and not np.isnan(part[0, 0, 2, :13]).any()
    assert np.isnan(part[0, 0, 2, 13:]).all(), "cells past the row were written"


def test_chunking_does_not_change_a_bit():
    batch, kv_t, q_t, _, _ = config1_device(torch.bfloat16)
    table = torch.from_numpy(batch.table).cuda()
    lens = torch.from_numpy(batch.lens).cuda()
    results = []
    for chunk in (1, 2, 3, 16, 64):
        plane = RecordingPlane(1, batch.rows, batch.width, batch.group_rows, batch.block_size)
        flag(plane)
        results.append(record(plane, 0, table, lens, q_t, kv_t[:, 0], 0.125, chunk_tiles=chunk))
    for r in results[1:]:
        assert np.array_equal(r, results[0], equal_nan=True)


def test_workgroup_slices_of_several_rounds():
    # a large minimum of tiles per wave gives few workgroups, each taking several rounds of 768
    # described tiles, the rounds crossing rows and KV heads; every record is the default launch's
    batch = workloads.config2_batch()
    pool = workloads.device_pool(batch, torch.bfloat16, seed=batch.seed + 3)
    q = torch.from_numpy(workloads.queries(batch, 1)[0]).to(torch.bfloat16).cuda()
    table = torch.from_numpy(batch.table).cuda()
    lens = torch.from_numpy(batch.lens).cuda()
    scale = batch.head_dim ** -0.5
    results = []
    for chunk in (0, 300):
        plane = RecordingPlane(1, batch.rows, batch.width, batch.group_rows, batch.block_size, kv_heads=batch.kv_heads)
        flag(plane)
        results.append(record(plane, 0, table, lens, q, pool[:, 0], scale, chunk_tiles=chunk))
    assert not np.isnan(results[0][0]).all()
    assert np.array_equal(results[1], results[0], equal_nan=True)
    del pool
    torch.cuda.empty_cache()


def test_llama3_8b_decode_shape_one_layer():
    batch = workloads.config2_batch()
    pool = workloads.device_pool(batch, torch.bfloat16, seed=batch.seed)
    q = torch.from_numpy(workloads.queries(batch, 1)[0]).to(torch.bfloat16).cuda()
    layer = 5
    group = layer % batch.kv_heads
    plane = RecordingPlane(8, batch.rows, batch.width, batch.group_rows, batch.block_size)
    flag(plane)
    scale = batch.head_dim ** -0.5
    got = record(plane, layer, torch.from_numpy(batch.table).cuda(), torch.from_numpy(batch.lens).cuda(), q,
                 pool[:, 0], scale)[:, layer : layer + 1]
    keys, table = workloads.host_keys(batch, pool, heads=[group])
    want = oa.new_planes(1, batch.rows, batch.width, batch.group_rows)
    oa.tile_lse(want, q.float().cpu().numpy(), keys, table, batch.lens, np.arange(batch.rows), np.ones(batch.rows),
                1, 0, scale, batch.block_size, batch.group_rows, [group], key_heads=[0])
    assert_parity(got, want, "llama3-8b decode")
    del pool
    torch.cuda.empty_cache()


def test_every_kv_head_mode():
    batch = workloads.config2_batch()
    rows = list(range(16))
    pool = workloads.device_pool(batch, torch.bfloat16, seed=batch.seed + 1)
    q = torch.from_numpy(workloads.queries(batch, 1)[0]).to(torch.bfloat16).cuda()
    plane = RecordingPlane(1, batch.rows, batch.width, batch.group_rows, batch.block_size, kv_heads=batch.kv_heads)
    flag(plane)
    select = np.zeros(batch.rows, bool)
    select[rows] = True
    scale = batch.head_dim ** -0.5
    got = record(plane, 0, torch.from_numpy(batch.table).cuda(), torch.from_numpy(batch.lens).cuda(), q,
                 pool[:, 0], scale, select=select)
    keys, table = workloads.host_keys(batch, pool, rows=rows)
    want = oa.new_planes(1, batch.rows, batch.width, batch.group_rows * batch.kv_heads)
    oa.tile_lse(want, q.float().cpu().numpy(), keys, table, batch.lens, np.arange(batch.rows), select, 1, 0, scale,
                batch.block_size, batch.group_rows, list(range(batch.kv_heads)))
    assert_parity(got, want, "every KV head")
    del pool
    torch.cuda.empty_cache()


def test_long_rows_with_heavy_hitters():
    # the whole skewed mix: 8 rows of 131072 tokens and 120 Zipf rows, 0.5% planted heavy hitters
    batch = workloads.config3_batch()
    pool = workloads.device_pool(batch, torch.bfloat16, seed=batch.seed)
    q = torch.from_numpy(workloads.queries(batch, 1)[0]).to(torch.bfloat16).cuda()
    workloads.plant_heavy_hitters(batch, pool, q)
    plane = RecordingPlane(1, batch.rows, batch.width, batch.group_rows, batch.block_size)
    flag(plane)
    scale = batch.head_dim ** -0.5
    got = record(plane, 0, torch.from_numpy(batch.table).cuda(), torch.from_numpy(batch.lens).cuda(), q,
                 pool[:, 0], scale)
    keys, table = workloads.host_keys(batch, pool, heads=[0])
    del pool
    torch.cuda.empty_cache()
    want = oa.new_planes(1, batch.rows, batch.width, batch.group_rows)
    every = np.ones(batch.rows)
    oa.tile_lse(want, q.float().cpu().numpy(), keys, table, batch.lens, np.arange(batch.rows), every, 1, 0, scale,
                batch.block_size, batch.group_rows, [0], key_heads=[0])
    assert_parity(got, want, "long rows + heavy hitters")


def test_full_step_fp8_with_timer():
    # the 256-row full step: 32 layers over two fp8 pools (block 32, a per-tensor scale), the per-row
    # timer on.  Every layer writes exactly the cells of the rows' blocks, two layers match the oracle
    # in full, and every row's cycle counter grows with every step.
    batch = workloads.config5_batch()
    layers, rows, G, bs = 32, batch.rows, batch.group_rows, batch.block_size
    fp8 = torch.float8_e4m3fn
    k_scale = batch.extra["k_scale"]
    pools = [workloads.device_pool(batch, fp8, seed=batch.seed + i) for i in range(2)]
    q = torch.from_numpy(workloads.queries(batch, layers)).to(torch.bfloat16).cuda()
    plane = RecordingPlane(layers, rows, batch.width, G, bs, timer=True)
    flag(plane)
    plane.select(np.ones(rows, bool), np.arange(rows))
    table, lens = torch.from_numpy(batch.table).cuda(), torch.from_numpy(batch.lens).cuda()
    scale = batch.head_dim ** -0.5

    def step():
        for layer in range(layers):
            plane.launch(layer, table, lens, q[layer], pools[layer % 2][:, 0], scale, k_scale=k_scale)
        torch.cuda.synchronize()

    step()
    first = plane.read_cycles()
    step()
    second = plane.read_cycles()
    assert (first[:rows] > 0).all() and (second[:rows] > first[:rows]).all(), "a row's cycles did not grow"
    got = plane.read_planes()
    written = np.arange(batch.width)[None, :] < batch.blocks[:, None]  # [rows, width]
    for layer in range(layers):
        assert np.array_equal(~np.isnan(got[0, layer]), np.repeat(written[:, :, None], G, axis=2)), layer
    for layer in (0, 13):
        keys, table_c = workloads.host_keys(batch, pools[layer % 2], heads=[layer % batch.kv_heads])
        want = oa.new_planes(1, rows, batch.width, G)
        oa.tile_lse(want, q[layer].float().cpu().numpy(), keys, table_c, batch.lens, np.arange(rows), np.ones(rows),
                    1, 0, scale, bs, G, [layer % batch.kv_heads], k_scale=k_scale, key_heads=[0])
        assert_parity(got[:, layer : layer + 1], want, f"fp8 full step, layer {layer}")
    del pools
    torch.cuda.empty_cache()


def test_fp8_keys_dequantised_by_the_scale():
    batch = workloads.config5_batch()
    fp8 = torch.float8_e4m3fn
    rows = list(range(4))
    # a small pool holding just these rows' blocks keeps the test light
    n = batch.blocks
    small = workloads.Batch(batch.lens[rows].copy(), np.zeros((4, batch.width), np.int32), batch.block_size,
                            int(n[rows].sum()) + 1, 32, 8, 128, seed=batch.seed, extra=dict(batch.extra))
    cursor = 1
    for i, r in enumerate(rows):
        small.table[i, : n[r]] = np.arange(cursor, cursor + n[r])
        cursor += int(n[r])
    pool = workloads.device_pool(small, fp8, seed=small.seed)
    q = torch.from_numpy(workloads.queries(small, 1)[0]).to(torch.bfloat16).cuda()
    k_scale = small.extra["k_scale"]
    plane = RecordingPlane(1, small.rows, small.width, small.group_rows, small.block_size)
    flag(plane)
    scale = small.head_dim ** -0.5
    got = record(plane, 0, torch.from_numpy(small.table).cuda(), torch.from_numpy(small.lens).cuda(), q,
                 pool[:, 0], scale, k_scale=k_scale)
    keys = pool[:, 0, :, :1].float().cpu().numpy()  # e4m3 values, exactly representable in float32
    want = oa.new_planes(1, small.rows, small.width, small.group_rows)
    oa.tile_lse(want, q.float().cpu().numpy(), keys, small.table, small.lens, np.arange(4), np.ones(4), 1, 0, scale,
                small.block_size, small.group_rows, [0], k_scale=k_scale, key_heads=[0])
    assert_parity(got, want, "fp8 e4m3 keys")


def synthetic(kind, n_tokens, hq=32, hkv=8, d=128, seed=7):
    """The flat / ramp controls of the reference's live check (tests/_attn_share_live_check.py:156-172)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(hq, d, generator=g, device="cuda")
    k = torch.randn(n_tokens, hkv, d, generator=g, device="cuda")
    if kind == "ramp":
        q = torch.zeros(hq, d, device="cuda")
        q[:, 0] = 1.0
        k = torch.zeros(n_tokens, hkv, d, device="cuda")
        k[:, :, 0] = torch.linspace(0.0, 12.0 * d**0.5, n_tokens, device="cuda")[:, None]
    return q.half(), k.half()


@pytest.mark.parametrize("kind", ["flat", "ramp"])
def test_records_give_the_true_share(kind):
    # the reference's gate: per-tile total variation distance to the float64 true share < 1e-3, and the
    # observed top 25% of tiles holds all of the true top 25% share (tests/_audit_kernel_live_check.py:117-120)
    lengths = (512, 1024, 2048, 3072, 4096, 6144)
    bs, d, hkv, hq = 16, 128, 8, 32
    seqs = [synthetic(kind, n, seed=7 + i) for i, n in enumerate(lengths)]
    n_blocks = [-(-n // bs) for n in lengths]
    width = max(n_blocks) + TILE_BLOCKS
    pool = torch.zeros(sum(n_blocks) + 1, 2, bs, hkv, d, dtype=torch.float16, device="cuda")
    table = torch.zeros(len(lengths), width, dtype=torch.int32, device="cuda")
    perm = torch.randperm(sum(n_blocks), device="cuda", generator=torch.Generator(device="cuda").manual_seed(0)) + 1
    cursor = 0
    for i, (qq, k) in enumerate(seqs):
        ids = perm[cursor : cursor + n_blocks[i]]
        cursor += n_blocks[i]
        table[i, : n_blocks[i]] = ids.int()
        pad = n_blocks[i] * bs - lengths[i]
        pool[ids, 0] = torch.nn.functional.pad(k, (0, 0, 0, 0, 0, pad)).reshape(n_blocks[i], bs, hkv, d)
    query = torch.stack([qq for qq, _ in seqs])
    lens = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    plane = RecordingPlane(1, len(lengths), width, hq // hkv, bs)
    flag(plane)
    got = record(plane, 0, table, lens, query, pool[:, 0], d**-0.5)
    u = ots.log_weights(got[0], got[1], TILE_BLOCKS)
    shares = ots.normalize(u, np.array(n_blocks), TILE_BLOCKS)
    for i, (qq, k) in enumerate(seqs):
        true = oa.true_block_shares(qq[: hq // hkv].float().cpu().numpy(), k[:, 0].float().cpu().numpy(), d**-0.5, bs)
        obs = np.nan_to_num(shares[i, : len(true)])
        t_tiles = np.add.reduceat(true, np.arange(0, len(true), 2))
        o_tiles = np.add.reduceat(obs, np.arange(0, len(true), 2))
        tv = 0.5 * np.abs(o_tiles / o_tiles.sum() - t_tiles / t_tiles.sum()).sum()
        top = max(1, round(0.25 * len(t_tiles)))
        kept = t_tiles[np.argsort(o_tiles)[::-1][:top]].sum() / np.sort(t_tiles)[::-1][:top].sum()
        print(f"{kind} L={lengths[i]}: TV {tv:.2e} kept {kept:.6f}", flush=True)
        assert tv < 1e-3 and kept > 1.0 - 1e-9


def test_timer_over_rounds_of_many_short_rows():
    # One workgroup's rounds each span more rows than the kernel's 64 per-round cycle slots (the rows
    # past them add to the accumulator directly), with two KV heads audited (only the first head's
    # tiles are timed): every selected row's cycles grow at every launch, the others stay zero.
    rows, bs, hkv, hq, d = 400, 16, 2, 8, 64
    rng = np.random.default_rng(17)
    lens = rng.integers(1, 65, size=rows).astype(np.int32)  # one or two tiles of 32 tokens
    n = (lens + bs - 1) // bs
    width = int(n.max())
    table = np.zeros((rows, width), dtype=np.int32)
    cursor = 1
    for r in range(rows):
        table[r, : n[r]] = np.arange(cursor, cursor + n[r])
        cursor += int(n[r])
    pool = torch.randn(cursor, 2, bs, hkv, d, device="cuda").to(torch.bfloat16)
    q = torch.randn(rows, hq, d, device="cuda").to(torch.bfloat16)
    plane = RecordingPlane(1, rows, width, hq // hkv, bs, kv_heads=hkv, timer=True)
    flag(plane)
    select = np.ones(rows, bool)
    select[::7] = False
    table_t, lens_t = torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda()
    prev = plane.read_cycles()
    for _ in range(3):
        got = record(plane, 0, table_t, lens_t, q, pool[:, 0], d**-0.5, select=select, chunk_tiles=1000)
        cur = plane.read_cycles()
        assert (cur[select] > prev[select]).all(), "a selected row's cycles did not grow"
        assert (cur[~select] == 0).all(), "an unselected row was timed"
        prev = cur
    assert not np.isnan(got[0][0][select]).all()


def test_timer_accumulates_per_row_cycles():
    # rows with planted work (lengths 512 * (r + 1)); the accumulator only grows, unselected rows stay 0,
    # and the per-launch cycles of a row follow its work (tests/_row_cycles_check.py:61-69, 120-163).
    # As the reference's check keeps one program per SM so that a duration is its own work and not
    # co-residency, the launch asks for at least 16 tiles per wave (about one wave per compute unit).
    rows, bs, hkv, hq, d = 16, 16, 8, 32, 128
    lens = np.array([512 * (r + 1) for r in range(rows)], dtype=np.int32)
    n = (lens + bs - 1) // bs
    width = int(n.max())
    table = np.zeros((rows + 2, width), dtype=np.int32)
    cursor = 1
    for r in range(rows):
        table[r, : n[r]] = np.arange(cursor, cursor + n[r])
        cursor += int(n[r])
    pool = torch.randn(cursor, 2, bs, hkv, d, device="cuda").to(torch.bfloat16)
    q = torch.randn(rows + 2, hq, d, device="cuda").to(torch.bfloat16)
    lens_all = np.concatenate([lens, [4096, 4096]]).astype(np.int32)
    plane = RecordingPlane(1, rows + 2, width, hq // hkv, bs, timer=True)
    flag(plane)
    select = np.ones(rows + 2, bool)
    select[-2:] = False  # two unselected rows (with valid tables) must not light up
    table[rows:, :] = table[rows - 1, :]
    table_t, lens_t = torch.from_numpy(table).cuda(), torch.from_numpy(lens_all).cuda()
    prev = plane.read_cycles()
    assert (prev == 0).all()
    deltas = []
    for _ in range(16):
        record(plane, 0, table_t, lens_t, q, pool[:, 0], d**-0.5, select=select, chunk_tiles=16)
        cur = plane.read_cycles()
        assert (cur >= prev).all(), "the accumulator decreased"
        deltas.append((cur - prev).astype(np.float64))
        prev = cur
    assert (prev[-2:] == 0).all(), "unselected rows were timed"
    c = np.median(np.array(deltas), axis=0)[:rows]
    work = n[:rows].astype(np.float64)
    corr = float(np.corrcoef(work, c)[0, 1])
    slope, icpt = np.polyfit(work, c, 1)
    r2 = 1 - ((c - (slope * work + icpt)) ** 2).sum() / ((c - c.mean()) ** 2).sum()
    print(f"cycles vs blocks: slope {slope:.0f}/block, R^2 {r2:.4f}, corr {corr:.4f}", flush=True)
    assert slope > 0 and r2 > 0.95 and corr > 0.98
