"""The audit kernel across element types, head dims, block sizes and query groups against the
float64 oracle (runtime/audit_kernel.py:34-109 of the reference): the MFMA form (f16 / bf16 /
fp8 keys, d 64 / 128 / 256, blocks of 16 and 32), the VALU form (fp32 keys, and every key type in
blocks of 8) and a query group of 1, 4 and 8 rows; shapes without a kernel raise ValueError."""

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


@pytest.mark.parametrize("G", [1, 4, 8])
@pytest.mark.parametrize("bs", [8, 16, 32])
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16", "fp8"])
def test_shapes_against_the_oracle(dtype, d, bs, G):
    torch_dtype = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16, "fp8": FP8}[dtype]
    if torch_dtype is None:
        pytest.skip("this torch has no float8_e4m3fn")
    mfma = dtype != "f32" and bs >= 16
    key_bytes = {"f32": 4, "f16": 2, "bf16": 2, "fp8": 1}[dtype]
    tokens_per_load = 64 // (d * key_bytes // 16)  # whole rows of 16-byte lanes
    # the VALU form: d 64 or 128, and a load instruction inside one block
    supported = mfma or (d in (64, 128) and tokens_per_load <= bs)
    lens, table, width, kv, q, k_scale = case(torch_dtype, d, bs, G, seed=d * 100 + bs * 10 + G)
    rows = len(lens)
    plane = RecordingPlane(1, rows, width, G, bs)
    audit_on(plane)
    plane.select(np.ones(rows, bool), np.arange(rows))
    scale = d ** -0.5
    kv_d, q_d = kv.cuda(), q.cuda()
    args = (0, torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda(), q_d, kv_d[:, 0], scale)
    if not supported:
        with pytest.raises(ValueError):
            plane.launch(*args, k_scale=k_scale)
        return
    plane.launch(*args, k_scale=k_scale)
    torch.cuda.synchronize()
    got = plane.read_planes()
    want = oa.new_planes(1, rows, width, G)
    oa.tile_lse(want, q.float().numpy(), kv[:, 0].float().numpy(), table, lens, np.arange(rows), np.ones(rows), 1, 0,
                scale, bs, G, [0], k_scale=k_scale)
    assert np.array_equal(np.isnan(got[0]), np.isnan(want[0])), "written cells differ"
    live = ~np.isnan(want[0])
    dm = np.abs(got[0][live] - want[0][live]).max()
    du = np.abs(ots.log_weights(got[0], got[1], 1)[live].astype(np.float64) - ots.log_weights(want[0], want[1], 1)[live]).max()
    assert dm < 1e-3 and du < 1e-3, (dm, du)


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
