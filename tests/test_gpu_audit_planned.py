"""GPU parity of the planned audit (ekv_audit_plan + ekv_audit_tile_lse_planned): the records of a
planned launch are bit-identical to the self-contained launch's on the same inputs, and agree with the
oracle, for every configuration's shape; the plan is built once per step and shared by its layers
(runtime/audit_kernel.py:34-109, :196-265 of the reference)."""

import numpy as np
import pytest
import torch

import workloads
from cases import audit_on
from oracle import audit as oa
from runtime.audit_kernel import RecordingPlane

pytestmark = pytest.mark.gpu


def both(plane_args, plane_kwargs, launches, select=None, qrow=None):
    """Records of the same launches, self-contained and planned, on two fresh planes:
    ``launches(plane, planned)`` makes the launches of one step."""
    out = []
    for planned in (False, True):
        plane = RecordingPlane(*plane_args, **plane_kwargs)
        audit_on(plane)
        rows = plane.rows
        plane.select(np.ones(rows, bool) if select is None else np.asarray(select, bool),
                     np.arange(rows) if qrow is None else np.asarray(qrow))
        launches(plane, planned)
        torch.cuda.synchronize()
        out.append((plane.read_planes(), plane.read_cycles()))
    return out


def assert_same(a, b, what):
    assert np.array_equal(a, b, equal_nan=True), f"{what}: the planned records differ from the self-contained ones"
    print(f"{what}: {int((~np.isnan(a[0])).sum())} cells bit-identical", flush=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_config1_planned_equals_self_contained(dtype):
    batch, kv, q = workloads.config1()
    kv_t = torch.from_numpy(kv).to(dtype).cuda()
    q_t = torch.from_numpy(q).to(dtype).cuda()
    table = torch.from_numpy(batch.table).cuda()
    lens = torch.from_numpy(batch.lens).cuda()
    scale = batch.head_dim ** -0.5

    def launches(plane, planned):
        if planned:
            plane.plan(table, lens)
        for layer in range(4):
            plane.launch(layer, table, lens, q_t, kv_t[:, 0], scale, planned=planned)

    (a, _), (b, _) = both((4, batch.rows, batch.width, batch.group_rows, batch.block_size), {}, launches)
    assert_same(a, b, f"config1 {dtype}")
    want = oa.new_planes(4, batch.rows, batch.width, batch.group_rows)
    kvh, qh = kv_t.float().cpu().numpy(), q_t.float().cpu().numpy()
    for layer in range(4):
        oa.tile_lse(want, qh, kvh[:, 0], batch.table, batch.lens, np.arange(4), np.ones(4), 1, layer, scale,
                    batch.block_size, batch.group_rows, [layer % batch.kv_heads])
    live = ~np.isnan(want[0])
    assert np.array_equal(~np.isnan(b[0]), live)
    assert np.abs(b[0][live] - want[0][live]).max() < 1e-3


def test_record_plans_at_the_first_layer():
    # the engine path: record() builds the plan at the step's first layer and every layer reads it;
    # a second step with other selected rows and query tokens rebuilds it
    batch, kv, q = workloads.config1()
    kv_t = torch.from_numpy(kv).to(torch.bfloat16).cuda()
    q_t = torch.from_numpy(np.concatenate([q, q[::-1]])).to(torch.bfloat16).cuda()  # 8 query tokens
    table = torch.from_numpy(batch.table).cuda()
    lens = torch.from_numpy(batch.lens).cuda()
    scale = batch.head_dim ** -0.5
    planes = []
    for engine in (False, True):
        plane = RecordingPlane(3, batch.rows, batch.width, batch.group_rows, batch.block_size)
        plane.attach([kv_t.data_ptr()] * 3)
        plane.set(True)
        for select, tokens in (([1, 1, 1, 1], [0, 1, 2, 3]), ([0, 1, 0, 1], [4, 6, 5, 7])):
            plane.select(np.array(select, bool), np.array(tokens))
            for layer in range(3):
                if engine:
                    plane.record(f"model.layers.{layer}.attn", table, lens, q_t, kv_t, scale)
                else:
                    plane.launch(layer, table, lens, q_t, kv_t[:, 0], scale)
        torch.cuda.synchronize()
        planes.append(plane.read_planes())
    assert_same(planes[0], planes[1], "record() over two steps")


def test_flag_off_plans_nothing():
    batch, kv, q = workloads.config1()
    kv_t = torch.from_numpy(kv).to(torch.bfloat16).cuda()
    q_t = torch.from_numpy(q).to(torch.bfloat16).cuda()
    table = torch.from_numpy(batch.table).cuda()
    lens = torch.from_numpy(batch.lens).cuda()
    plane = RecordingPlane(1, batch.rows, batch.width, batch.group_rows, batch.block_size)
    plane.attach([kv_t.data_ptr()])
    plane.select(np.ones(batch.rows, bool), np.arange(batch.rows))
    plane.set(True)
    plane.set(False)
    plane.plan(table, lens)
    plane.set(True)  # a plan made with the flag off is empty: the launch records nothing
    plane.launch(0, table, lens, q_t, kv_t[:, 0], 0.125, planned=True)
    torch.cuda.synchronize()
    assert np.isnan(plane.read_planes()).all()


def test_llama3_decode_planned_every_layer_group():
    # the Llama-3-8B decode shape: one plan, eight layers each auditing its own KV group, some rows
    # unselected and the query tokens permuted; then every KV head in one launch
    batch = workloads.config2_batch()
    pool = workloads.device_pool(batch, torch.bfloat16, seed=batch.seed + 11)
    q = torch.from_numpy(workloads.queries(batch, 1)[0]).to(torch.bfloat16).cuda()
    table = torch.from_numpy(batch.table).cuda()
    lens = torch.from_numpy(batch.lens).cuda()
    scale = batch.head_dim ** -0.5
    rng = np.random.default_rng(5)
    select = rng.random(batch.rows) < 0.8
    qrow = rng.permutation(batch.rows)

    def launches(plane, planned):
        if planned:
            plane.plan(table, lens)
        for layer in range(8):
            plane.launch(layer, table, lens, q, pool[:, 0], scale, planned=planned)

    (a, _), (b, _) = both((8, batch.rows, batch.width, batch.group_rows, batch.block_size), {}, launches,
                          select=select, qrow=qrow)
    assert_same(a, b, "llama3 decode, 8 layers")
    keys, table_c = workloads.host_keys(batch, pool, heads=[3])
    want = oa.new_planes(1, batch.rows, batch.width, batch.group_rows)
    oa.tile_lse(want, q.float().cpu().numpy(), keys, table_c, batch.lens, qrow, select, 1, 0, scale,
                batch.block_size, batch.group_rows, [3], key_heads=[0])
    live = ~np.isnan(want[0])
    assert np.array_equal(~np.isnan(b[0, 3]), live[0])
    assert np.abs(b[0, 3][live[0]] - want[0, 0][live[0]]).max() < 1e-3

    def every_head(plane, planned):
        if planned:
            plane.plan(table, lens)
        plane.launch(0, table, lens, q, pool[:, 0], scale, planned=planned)

    (a, _), (b, _) = both((1, batch.rows, batch.width, batch.group_rows, batch.block_size),
                          {"kv_heads": batch.kv_heads}, every_head, select=select, qrow=qrow)
    assert_same(a, b, "llama3 decode, every KV head")
    del pool
    torch.cuda.empty_cache()


def test_skewed_long_context_planned():
    batch = workloads.config3_batch()
    pool = workloads.device_pool(batch, torch.bfloat16, seed=batch.seed + 2)
    q = torch.from_numpy(workloads.queries(batch, 1)[0]).to(torch.bfloat16).cuda()
    workloads.plant_heavy_hitters(batch, pool, q)
    table = torch.from_numpy(batch.table).cuda()
    lens = torch.from_numpy(batch.lens).cuda()
    scale = batch.head_dim ** -0.5

    def launches(plane, planned):
        if planned:
            plane.plan(table, lens)
        for layer in range(2):
            plane.launch(layer, table, lens, q, pool[:, 0], scale, planned=planned)

    (a, _), (b, _) = both((2, batch.rows, batch.width, batch.group_rows, batch.block_size), {}, launches)
    assert_same(a, b, "skewed long-context mix")
    del pool
    torch.cuda.empty_cache()


def test_fp8_full_step_planned_with_timer():
    # the 256-row fp8 step, 32 layers, the per-row timer on: records bit-identical, every row timed
    batch = workloads.config5_batch()
    fp8 = torch.float8_e4m3fn
    k_scale = batch.extra["k_scale"]
    pools = [workloads.device_pool(batch, fp8, seed=batch.seed + i) for i in range(2)]
    q = torch.from_numpy(workloads.queries(batch, 32)).to(torch.bfloat16).cuda()
    table = torch.from_numpy(batch.table).cuda()
    lens = torch.from_numpy(batch.lens).cuda()
    scale = batch.head_dim ** -0.5

    def launches(plane, planned):
        if planned:
            plane.plan(table, lens)
        for layer in range(32):
            plane.launch(layer, table, lens, q[layer], pools[layer % 2][:, 0], scale, k_scale=k_scale,
                         planned=planned)

    (a, ca), (b, cb) = both((32, batch.rows, batch.width, batch.group_rows, batch.block_size), {"timer": True},
                            launches)
    assert_same(a, b, "fp8 full step")
    assert (cb > 0).all() and (ca > 0).all(), "a row was not timed"
    del pools
    torch.cuda.empty_cache()


def test_plan_refuses_a_batch_larger_than_the_plane():
    batch, kv, q = workloads.config1()
    plane = RecordingPlane(1, 2, 8, batch.group_rows, batch.block_size)
    table = torch.from_numpy(batch.table).cuda()
    lens = torch.from_numpy(batch.lens).cuda()
    import ekv_hip

    with pytest.raises(ValueError, match="plan"):
        ekv_hip.call("ekv_audit_plan", table.data_ptr(), table.stride(0), lens.data_ptr(), plane._token.data_ptr(),
                     plane._select.data_ptr(), plane._flag_dev, 4, 32, batch.block_size, 2, plane._plan,
                     plane._plan_bytes, 2, 8, 0)


def test_planned_rows_past_the_lds_row_limit():
    # 8192 rows, more than the 6000 whose tile offsets the self-contained kernel keeps in LDS: the
    # planned launch takes them all, bit-identical to the self-contained kernel run on each half, and
    # some rows agree with the oracle; the self-contained launch refuses the whole batch
    rng = np.random.default_rng(8192)
    rows, width, bs, kvh, g, d = 8192, 16, 16, 2, 4, 128
    lens = rng.integers(1, width * bs + 1, size=rows).astype(np.int32)
    pool = 2 * rows * width
    table = rng.permutation(pool)[: rows * width].reshape(rows, width).astype(np.int32)
    kv = torch.randn(pool, 2, bs, kvh, d, dtype=torch.bfloat16, device="cuda")
    q = torch.randn(rows, kvh * g, d, dtype=torch.bfloat16, device="cuda")
    scale = d ** -0.5
    t_all, l_all = torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda()
    plane = RecordingPlane(1, rows, width, g, bs)
    audit_on(plane)
    plane.select(np.ones(rows, bool), np.arange(rows))
    plane.plan(t_all, l_all)
    plane.launch(0, t_all, l_all, q, kv[:, 0], scale, planned=True)
    with pytest.raises(ValueError, match="rows"):
        plane.launch(0, t_all, l_all, q, kv[:, 0], scale, planned=False)
    torch.cuda.synchronize()
    got = plane.read_planes()
    half = rows // 2
    for lo in (0, half):
        part = RecordingPlane(1, half, width, g, bs)
        audit_on(part)
        part.select(np.ones(half, bool), np.arange(lo, lo + half))  # each row's query token is its own
        part.launch(0, t_all[lo : lo + half].contiguous(), l_all[lo : lo + half].contiguous(), q, kv[:, 0], scale)
        torch.cuda.synchronize()
        want = part.read_planes()
        assert np.array_equal(got[:, :, lo : lo + half], want, equal_nan=True), f"rows {lo}.."
    sample = np.zeros(rows)
    sample[::997] = 1
    want = oa.new_planes(1, rows, width, g)
    kvf, qf = kv.float().cpu().numpy(), q.float().cpu().numpy()
    oa.tile_lse(want, qf, kvf[:, 0], table, lens, np.arange(rows), sample, 1, 0, scale, bs, g, [0])
    live = ~np.isnan(want[0])
    assert np.abs(got[0][live] - want[0][live]).max() < 1e-3
    print(f"{int((~np.isnan(got[0])).sum())} cells; {int(sample.sum())} rows against the oracle", flush=True)
