"""The audit kernel across element types, head dims, block sizes and query groups against the
float64 oracle (runtime/audit_kernel.py:34-109 of the reference, which takes any power-of-two head
dim and tile): every shape through the engine's path (RecordingPlane.record: the step plan and the
launch over the step's layers) -- the MFMA form (16-bit keys at d 32 to 256, fp8 keys at d 64 to 256,
blocks of 16 and 32) and the planned VALU form for the rest (fp32 keys, blocks of 8, fp8 rows of 32
dimensions) -- and the self-contained launch for the shapes it has."""

import numpy as np
import pytest
import torch

from oracle import audit as oa
from oracle import tile_shares as ots
from runtime.audit_kernel import RecordingPlane
from cases import audit_on

pytestmark = pytest.mark.gpu
FP8 = getattr(torch, "float8_e4m3fn", None)


def case(dtype, d, bs, G, seed):
    rng = np.random.default_rng(seed)
    hkv, rows = 2, 6
    lens = np.array([1, bs - 1, bs, 2 * bs + 3, 9 * bs + 1, 23 * bs], dtype=np.int32)
    n = (lens + bs - 1) // bs
    width = int(n.max()) + 2
    pool = int(n.sum()) + 3
    table = np.zeros((rows, width), dtype=np.int32)
    ids = rng.permutation(np.arange(1, pool))
    cursor = 0
    for r in range(rows):
        table[r, : n[r]] = ids[cursor : cursor + n[r]]
        cursor += int(n[r])
    k_scale = 1.0
    kv = torch.from_numpy(rng.standard_normal((pool, 2, bs, hkv, d), dtype=np.float32))
    if dtype == FP8:
        k_scale = 4.0 / 448.0
        kv = (kv / k_scale).clamp(-448, 448).to(FP8)
    else:
        kv = kv.to(dtype)
    qdtype = torch.bfloat16 if dtype == FP8 else dtype
    q = torch.from_numpy(rng.standard_normal((rows, hkv * G, d), dtype=np.float32)).to(qdtype)
    return lens, table, width, kv, q, k_scale


def against_the_oracle(got, q, kv, table, lens, select, scale, bs, G, k_scale, layers=1):
    kv_heads = kv.shape[3]
    want = oa.new_planes(layers, len(lens), table.shape[1], G)
    for layer in range(layers):  # layer L audits KV head L mod kv_heads (runtime/audit_kernel.py:250)
        oa.tile_lse(want, q.float().numpy(), kv[:, 0].float().numpy(), table, lens, np.arange(len(lens)), select, 1,
                    layer, scale, bs, G, [layer % kv_heads], k_scale=k_scale)
    assert np.array_equal(np.isnan(got[0]), np.isnan(want[0])), "written cells differ"
    live = ~np.isnan(want[0])
    dm = np.abs(got[0][live] - want[0][live]).max()
    du = np.abs(ots.log_weights(got[0], got[1], 1)[live].astype(np.float64) - ots.log_weights(want[0], want[1], 1)[live]).max()
    assert dm < 1e-3 and du < 1e-3, (dm, du)


@pytest.mark.parametrize("G", [1, 4, 8])
@pytest.mark.parametrize("bs", [8, 16, 32])
@pytest.mark.parametrize("d", [32, 64, 128, 256])
@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16", "fp8"])
def test_shapes_against_the_oracle(dtype, d, bs, G):
    import ekv_hip

    torch_dtype = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16, "fp8": FP8}[dtype]
    if torch_dtype is None:
        pytest.skip("this torch has no float8_e4m3fn")
    lens, table, width, kv, q, k_scale = case(torch_dtype, d, bs, G, seed=d * 100 + bs * 10 + G)
    rows = len(lens)
    scale = d ** -0.5
    kv_d, q_d = kv.cuda(), q.cuda()
    table_d, lens_d = torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda()
    forms = ekv_hip.load().ekv_audit_shape(ekv_hip.dtype_code(q.dtype), ekv_hip.dtype_code(kv.dtype), d, bs)
    assert forms & ekv_hip.AUDIT_PLANNED, "the reference takes this shape: the planned launch must too"
    # the engine's path: record() plans the step and launches over its layers (two layers here, the
    # same keys; fp8 keys through direct entries, since record() carries no key scale)
    plane = RecordingPlane(2, rows, width, G, bs)
    audit_on(plane)
    plane.select(np.ones(rows, bool), np.arange(rows))
    if torch_dtype == FP8:
        plane.plan(table_d, lens_d)
        entries = [plane.direct(layer, q_d, kv_d[:, 0], scale, k_scale=k_scale) for layer in range(2)]
        plane.launch_layers(entries, kv_d[:, 0], q_d, staged=False)
    else:
        for step in range(2):  # the first registers the layers; the second is one launch over both
            for layer in range(2):
                plane.record(f"layer.{layer}", table_d, lens_d, q_d, kv_d, scale)
    torch.cuda.synchronize()
    against_the_oracle(plane.read_planes(), q, kv, table, lens, np.ones(rows), scale, bs, G, k_scale, layers=2)
    # the self-contained launch, for the shapes it has (others go through a plan it builds)
    single = RecordingPlane(1, rows, width, G, bs)
    audit_on(single)
    single.select(np.ones(rows, bool), np.arange(rows))
    single.launch(0, table_d, lens_d, q_d, kv_d[:, 0], scale, k_scale=k_scale)
    torch.cuda.synchronize()
    against_the_oracle(single.read_planes(), q, kv, table, lens, np.ones(rows), scale, bs, G, k_scale)
    print(f"{dtype} d={d} block={bs} G={G}: forms {forms}", flush=True)


@pytest.mark.parametrize("dtype,d,bs", [("f32", 128, 16), ("bf16", 128, 8), ("fp8", 32, 16), ("f32", 256, 8)])
def test_planned_valu_shapes_past_the_self_contained_row_limit(dtype, d, bs):
    # 8192 rows on the VALU form: the planned launch takes them all (the self-contained one at most
    # 6000), short rows of 0 to 3 blocks, some unselected, every 97th row against the oracle
    torch_dtype = {"f32": torch.float32, "bf16": torch.bfloat16, "fp8": FP8}[dtype]
    if torch_dtype is None:
        pytest.skip("this torch has no float8_e4m3fn")
    rng = np.random.default_rng(8192 + d + bs)
    rows, G, hkv, width = 8192, 4, 2, 4
    lens = rng.integers(0, 3 * bs + 1, rows).astype(np.int32)
    n = (lens + bs - 1) // bs
    pool = int(n.sum()) + 1
    table = np.zeros((rows, width), dtype=np.int32)
    ids = rng.permutation(np.arange(1, pool))
    cursor = 0
    for r in range(rows):
        table[r, : n[r]] = ids[cursor : cursor + n[r]]
        cursor += int(n[r])
    kv = torch.from_numpy(rng.standard_normal((pool, 2, bs, hkv, d), dtype=np.float32))
    k_scale = 1.0
    if torch_dtype == FP8:
        k_scale = 4.0 / 448.0
        kv = (kv / k_scale).clamp(-448, 448).to(FP8)
    else:
        kv = kv.to(torch_dtype)
    qdtype = torch.bfloat16 if torch_dtype == FP8 else torch_dtype
    q = torch.from_numpy(rng.standard_normal((rows, hkv * G, d), dtype=np.float32)).to(qdtype)
    select = rng.random(rows) < 0.9
    plane = RecordingPlane(1, rows, width, G, bs)
    audit_on(plane)
    plane.select(select, np.arange(rows))
    scale = d ** -0.5
    t_d, l_d = torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda()
    plane.plan(t_d, l_d)
    plane.launch(0, t_d, l_d, q.cuda(), kv.cuda()[:, 0], scale, k_scale=k_scale, planned=True)
    torch.cuda.synchronize()
    got = plane.read_planes()
    sample = np.zeros(rows)
    sample[::97] = select[::97]
    want = oa.new_planes(1, rows, width, G)
    oa.tile_lse(want, q.float().numpy(), kv[:, 0].float().numpy(), table, lens, np.arange(rows), sample, 1, 0, scale,
                bs, G, [0], k_scale=k_scale)
    live = ~np.isnan(want[0])
    assert not np.isnan(got[0][live]).any()
    assert np.abs(got[0][live] - want[0][live]).max() < 1e-3
    assert np.isnan(got[0][:, ~select]).all(), "an unselected row was recorded"
    print(f"{dtype} d={d} block={bs}: {int((~np.isnan(got[0])).sum())} cells, {int(sample.sum())} rows checked",
          flush=True)


@pytest.mark.parametrize("dtype,d", [("bf16", 128), ("fp8", 256)])
def test_the_largest_row_count(dtype, d):
    # 6000 rows, the most the kernels' LDS takes beside the largest staging buffer (key rows of 256 B):
    # short rows of 0 to 3 blocks, some unselected, against the oracle
    torch_dtype = {"bf16": torch.bfloat16, "fp8": FP8}[dtype]
    if torch_dtype is None:
        pytest.skip("this torch has no float8_e4m3fn")
    rng = np.random.default_rng(6000 + d)
    rows, bs, G, hkv = 6000, 16, 4, 2
    lens = rng.integers(0, 3 * bs + 1, rows).astype(np.int32)
    n = (lens + bs - 1) // bs
    width = 4
    pool = int(n.sum()) + 1
    table = np.zeros((rows, width), dtype=np.int32)
    ids = rng.permutation(np.arange(1, pool))
    cursor = 0
    for r in range(rows):
        table[r, : n[r]] = ids[cursor : cursor + n[r]]
        cursor += int(n[r])
    kv = torch.from_numpy(rng.standard_normal((pool, 2, bs, hkv, d), dtype=np.float32))
    k_scale = 1.0
    if torch_dtype == FP8:
        k_scale = 4.0 / 448.0
        kv = (kv / k_scale).clamp(-448, 448).to(FP8)
    else:
        kv = kv.to(torch_dtype)
    q = torch.from_numpy(rng.standard_normal((rows, hkv * G, d), dtype=np.float32)).to(torch.bfloat16)
    select = rng.random(rows) < 0.9
    plane = RecordingPlane(1, rows, width, G, bs)
    audit_on(plane)
    plane.select(select, np.arange(rows))
    scale = d ** -0.5
    plane.launch(0, torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda(), q.cuda(), kv.cuda()[:, 0], scale,
                 k_scale=k_scale)
    torch.cuda.synchronize()
    got = plane.read_planes()
    want = oa.new_planes(1, rows, width, G)
    oa.tile_lse(want, q.float().numpy(), kv[:, 0].float().numpy(), table, lens, np.arange(rows),
                select.astype(np.float64), 1, 0, scale, bs, G, [0], k_scale=k_scale)
    assert np.array_equal(np.isnan(got[0]), np.isnan(want[0])), "written cells differ"
    live = ~np.isnan(want[0])
    assert np.abs(got[0][live] - want[0][live]).max() < 1e-3
    assert np.abs(got[1][live] - want[1][live]).max() < 1e-3 * np.abs(want[1][live]).max()
