"""GPU parity of the batched audit (ekv_audit_stage_queries + ekv_audit_tile_lse_layers behind
RecordingPlane.record): one launch over a step's layers writes the records and cycles the per-layer
launches write, bit for bit, and they agree with the oracle (runtime/audit_kernel.py:34-109, :196-265
of the reference).  Also the rows a shrinking batch leaves behind, through DecodeView: they are no longer
audited, so their records and cycles stay as they were."""

import time

import numpy as np
import pytest
import torch

import workloads
from cases import audit_on
from oracle import audit as oa
from runtime.audit_kernel import RecordingPlane
from runtime.block_view import DecodeView

pytestmark = pytest.mark.gpu


def random_batch(rng, rows, width, bs, kv_heads, group, dim, dtype, pool_factor=2):
    lens = rng.integers(1, width * bs + 1, size=rows).astype(np.int32)
    pool = pool_factor * rows * width + 1
    table = (1 + rng.permutation(pool - 1)[: rows * width]).reshape(rows, width).astype(np.int32)
    if dtype == torch.float8_e4m3fn:
        kv = (torch.randn(pool, 2, bs, kv_heads, dim, device="cuda") * 2).to(dtype)
    else:
        kv = torch.randn(pool, 2, bs, kv_heads, dim, device="cuda").to(dtype)
    return lens, table, kv


def run_steps(plane_args, plane_kwargs, steps, layers, batched):
    """Records and cycles after ``steps`` [(select, tokens, table, lens, queries per layer, caches per
    layer, scale)] recorded through record(), batched or one launch per layer."""
    plane = RecordingPlane(*plane_args, batch_layers=batched, **plane_kwargs)
    audit_on(plane)
    for select, tokens, table, lens, queries, caches, scale in steps:
        plane.select(select, tokens)
        for layer in range(layers):
            plane.record(f"model.layers.{layer}.attn", table, lens, queries[layer], caches[layer], scale)
    torch.cuda.synchronize()
    return plane.read_planes(), plane.read_cycles()


SHAPES = [
    # (q / key dtype, head_dim, block, kv_heads, group, rows, width, layers, every KV head, timer)
    (torch.bfloat16, 128, 16, 8, 4, 48, 40, 8, False, False),
    (torch.float16, 64, 16, 2, 4, 33, 24, 5, False, True),
    (torch.bfloat16, 256, 16, 2, 2, 20, 16, 4, False, False),
    (torch.bfloat16, 64, 32, 4, 8, 30, 12, 6, False, True),
    (torch.float8_e4m3fn, 128, 32, 8, 4, 40, 20, 9, False, True),
    (torch.bfloat16, 128, 16, 4, 4, 24, 20, 3, True, True),
    # every one of 8 KV heads: runs of 8 items, held 4 (d = 128) or 8 (d = 64) at a time
    (torch.bfloat16, 128, 16, 8, 4, 24, 20, 3, True, False),
    (torch.float16, 64, 16, 8, 4, 20, 16, 4, True, False),
    (torch.bfloat16, 128, 16, 2, 4, 12, 10, 40, False, False),  # 40 layers: two launches of 32 and 8
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}-d{s[1]}-b{s[2]}-L{s[7]}{'-all' if s[8] else ''}")
def test_batched_record_equals_per_layer_launches(shape):
    dtype, dim, bs, kvh, g, rows, width, layers, every, timed = shape
    rng = np.random.default_rng(dim * 1000 + bs * 10 + layers)
    qdtype = torch.bfloat16 if dtype == torch.float8_e4m3fn else dtype
    steps = []
    for s in range(3):  # three steps; the second selects fewer rows of a shorter batch
        n = rows if s != 1 else rows // 2
        lens, table, kv = random_batch(rng, rows, width, bs, kvh, g, dim, dtype)
        lens[n:] = 0
        tokens = rng.permutation(rows + 5)[:n]
        select = rng.random(n) < 0.8
        select[0] = True
        queries = [torch.randn(rows + 5, kvh * g, dim, device="cuda").to(qdtype) for _ in range(layers)]
        caches = [kv] * layers
        steps.append((select, tokens, torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda(), queries,
                      caches, dim ** -0.5))
    kwargs = {"timer": timed}
    if every:
        kwargs["kv_heads"] = kvh
    args = (layers, rows, width, g, bs)
    (a, ca), (b, cb) = (run_steps(args, kwargs, steps, layers, batched) for batched in (False, True))
    assert np.array_equal(a, b, equal_nan=True), "the batched records differ from the per-layer launches"
    cells = int((~np.isnan(b[0])).sum())
    assert cells > 0
    if timed:
        assert np.array_equal(ca > 0, cb > 0), "the batched launch timed other rows"
    # the last step against the oracle (the layers' last records are the last step's)
    select, tokens, table, lens, queries, caches, scale = steps[-1]
    want = oa.new_planes(layers, rows, width, g * (kvh if every else 1))
    kvf = caches[0].float().cpu().numpy()
    sel = np.zeros(rows)
    sel[: len(select)] = select
    qrow = np.zeros(rows, dtype=np.int64)
    qrow[: len(tokens)] = tokens
    for layer in range(layers):
        heads = list(range(kvh)) if every else [layer % kvh]
        oa.tile_lse(want, queries[layer].float().cpu().numpy(), kvf[:, 0], table.cpu().numpy(), lens.cpu().numpy(),
                    qrow, sel, 1, layer, scale, bs, g, heads)
    # the cells the last step wrote (earlier steps' records stay past its rows and lengths)
    live = ~np.isnan(want[0])
    assert not np.isnan(b[0][live]).any()
    assert np.abs(b[0][live] - want[0][live]).max() < 1e-3
    print(f"{shape}: {cells} cells bit-identical to the per-layer launches", flush=True)


def test_shrinking_batch_leaves_the_old_rows_alone():
    """An 8-row audit step, then a 4-row one through DecodeView: rows 4-7 are not audited again, so
    their records stay bit for bit and their cycles do not move, and rows 0-3 hold the new step's."""
    rng = np.random.default_rng(84)
    rows, width, bs, kvh, g, dim, layers = 8, 12, 16, 2, 4, 128, 4
    lens, table, kv = random_batch(rng, rows, width, bs, kvh, g, dim, torch.bfloat16)
    table_t, lens_t = torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda()
    plane = RecordingPlane(layers, rows, width, g, bs, timer=True)
    view = DecodeView(rows, width, bs, audit=plane)
    assert plane.attach([kv.data_ptr()] * layers)
    view.write_lease_deadline(time.monotonic_ns() + 3600 * 10**9)
    scale = dim ** -0.5

    def step(n, queries):
        t, l = view.build(table_t[:n], lens_t[:n], torch.ones(n, dtype=torch.int32))
        full_t, full_l = view.buffers
        for layer in range(layers):  # the engine's hook records with the view's whole buffers
            plane.record(f"layer.{layer}", full_t, full_l, queries[layer], kv, scale)
        torch.cuda.synchronize()

    q8 = [torch.randn(8, kvh * g, dim, device="cuda", dtype=torch.bfloat16) for _ in range(layers)]
    view.write_audit_rows(np.ones(rows, bool))
    step(8, q8)
    step(8, q8)  # completes the audit
    first, cycles_first = plane.read_planes().copy(), plane.read_cycles().copy()
    assert (cycles_first > 0).all()
    q4 = [torch.randn(4, kvh * g, dim, device="cuda", dtype=torch.bfloat16) for _ in range(layers)]
    view.write_audit_rows(np.ones(rows, bool))
    step(4, q4)  # a 4-row audit step: the query tensors have 4 tokens
    step(4, q4)
    second, cycles_second = plane.read_planes(), plane.read_cycles()
    assert np.array_equal(second[:, :, 4:], first[:, :, 4:], equal_nan=True), "rows 4-7 were audited again"
    assert np.array_equal(cycles_second[4:], cycles_first[4:]), "rows 4-7 were timed again"
    assert (cycles_second[:4] > cycles_first[:4]).all()
    want = oa.new_planes(layers, rows, width, g)
    kvf = kv.float().cpu().numpy()
    for layer in range(layers):
        oa.tile_lse(want, q4[layer].float().cpu().numpy(), kvf[:, 0], table, lens, np.arange(rows),
                    np.array([1, 1, 1, 1, 0, 0, 0, 0]), 1, layer, scale, bs, g, [layer % kvh])
    live = ~np.isnan(want[0][:, :4])
    assert np.abs(second[0][:, :4][live] - want[0][:, :4][live]).max() < 1e-3


def test_captured_step_reads_the_queries_in_place():
    """A step recorded under graph capture launches once over the layers and reads each query where
    it is; every replay (with eager work and a fresh selection between them) writes what the eager,
    staged step writes, bit for bit."""
    rng = np.random.default_rng(2024)
    rows, width, bs, kvh, g, dim, layers = 40, 24, 16, 4, 4, 128, 6
    lens, table, kv = random_batch(rng, rows, width, bs, kvh, g, dim, torch.bfloat16)
    table_t, lens_t = torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda()
    scale = dim ** -0.5
    queries = [torch.randn(rows, kvh * g, dim, device="cuda", dtype=torch.bfloat16) for _ in range(layers)]

    def record_step(plane):
        for layer in range(layers):
            # a fresh query tensor per layer, as an engine's projection makes it
            q = queries[layer] * 1.0
            plane.record(f"layer.{layer}", table_t, lens_t, q, kv, scale)

    eager = RecordingPlane(layers, rows, width, g, bs, timer=True)
    audit_on(eager)
    select = rng.random(rows) < 0.7
    eager.select(select, np.arange(rows))
    record_step(eager)  # registers the layers (one launch each)
    eager.clear()
    record_step(eager)  # the staged step: one launch over the layers
    torch.cuda.synchronize()
    want = eager.read_planes().copy()

    captured = RecordingPlane(layers, rows, width, g, bs, timer=True)
    audit_on(captured)
    captured.select(select, np.arange(rows))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        record_step(captured)  # warm-up: registers the layers
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        record_step(captured)
    assert captured._pending == [] and captured._held == []
    for replay in range(3):
        captured.clear()
        captured.select(select, np.arange(rows))
        _ = torch.randn(1 << 20, device="cuda").sum()  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = captured.read_planes()
        assert np.array_equal(got, want, equal_nan=True), f"replay {replay} differs from the eager staged step"
    assert (captured.read_cycles()[select] > 0).all()
