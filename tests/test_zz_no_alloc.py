"""The allocation-free share normalisation, ekv_tile_shares_noalloc, called through the C ABI: the
same shares as ekv_tile_shares_ws with a caller workspace, bit for bit, on two calls in a row (the
second smaller, so stale scratch contents from the first would show), and the oracle's within 1e-4;
calls too large for the library's scratch are refused before any launch."""

import numpy as np
import pytest
import torch

import ekv_hip
from oracle import tile_shares as ots

pytestmark = pytest.mark.gpu
SHARE_TOL = 1e-4


def records(rng, table_layers, rows, width, cells):
    m = rng.normal(0, 3, (table_layers, rows, width, cells)).astype(np.float32)
    l = rng.uniform(0.5, 30, (table_layers, rows, width, cells)).astype(np.float32)
    l[rng.random(l.shape) < 0.02] = 0.0
    m[rng.random(m.shape) < 0.03] = -np.inf
    m[:, 1] = np.nan  # a row without evidence
    return np.stack([m, l])


def call_both(planes, layers, row_ids, row_blocks, tile, aggregate):
    _, table_layers, rows, width, cells = planes.shape
    dev = torch.from_numpy(np.ascontiguousarray(planes)).cuda()
    ids = torch.from_numpy(row_ids.astype(np.int32)).cuda()
    blocks = torch.from_numpy(row_blocks.astype(np.int32)).cuda()
    n = len(row_ids)
    layer_stride = rows * width * cells
    common = (dev.data_ptr(), table_layers * layer_stride, layer_stride, width * cells, layers, cells, width,
              ids.data_ptr(), blocks.data_ptr(), n, tile, aggregate)
    # poison both outputs so that any unwritten entry shows
    with_ws = torch.full((n, width), 7.0, dtype=torch.float32, device="cuda")
    no_alloc = torch.full((n, width), -7.0, dtype=torch.float32, device="cuda")
    need = int(ekv_hip.load().ekv_tile_shares_workspace(n, width, layers))
    workspace = torch.zeros(need, dtype=torch.uint8, device="cuda")  # zeroed before its first use
    stream = ekv_hip.stream_handle()
    ekv_hip.call("ekv_tile_shares_ws", *common, with_ws.data_ptr(), width, workspace.data_ptr(), need, stream)
    ekv_hip.call("ekv_tile_shares_noalloc", *common, no_alloc.data_ptr(), width, stream)
    torch.cuda.synchronize()
    return with_ws.cpu().numpy(), no_alloc.cpu().numpy()


@pytest.mark.parametrize("aggregate", [ekv_hip.AGG_MEAN, ekv_hip.AGG_MAX])
def test_no_alloc_matches_the_workspace_form_on_two_calls(aggregate):
    rng = np.random.default_rng(900 + aggregate)
    name = "max" if aggregate == ekv_hip.AGG_MAX else "mean"
    # first call: the benchmark's shape (32 layers, 128 rows of 512 blocks, 4 query rows per block)
    # second call: fewer rows and layers, a narrower row and 5 cells (the other split kernel)
    for layers, rows, width, cells in ((32, 128, 512, 4), (5, 11, 300, 5)):
        planes = records(rng, layers + 1, rows, width, cells)
        row_ids = np.arange(rows)
        row_blocks = rng.integers(0, width + 3, size=rows)  # tails, empty rows, rows past the width
        with_ws, no_alloc = call_both(planes, layers, row_ids, row_blocks, 2, aggregate)
        what = f"{layers} layers x {rows} rows x {width} blocks x {cells} cells, {name}"
        print(what, flush=True)
        assert np.array_equal(np.isnan(with_ws), np.isnan(no_alloc)), what
        assert np.array_equal(with_ws[~np.isnan(with_ws)], no_alloc[~np.isnan(no_alloc)]), what
        want = ots.normalize(ots.read_rows(planes, layers, row_ids, 2), row_blocks, 2, name)
        got = no_alloc.astype(np.float64)
        assert np.array_equal(np.isnan(got), np.isnan(want)), what
        assert np.nanmax(np.abs(np.nan_to_num(got - want))) <= SHARE_TOL, what


def test_no_alloc_refuses_calls_beyond_its_scratch():
    lib = ekv_hip.load()
    scratch = 16 << 20
    assert lib.ekv_tile_shares_workspace(128, 512, 32) <= scratch
    assert lib.ekv_tile_shares_workspace(1024, 8192, 32) > scratch
    out = torch.empty(1024, 8192, dtype=torch.float32, device="cuda")
    planes = torch.empty(16, dtype=torch.float32, device="cuda")  # never read: the size check comes first
    with pytest.raises(ValueError, match="scratch"):
        ekv_hip.call("ekv_tile_shares_noalloc", planes.data_ptr(), 0, 0, 0, 32, 4, 8192, 0, 0, 1024, 2,
                     ekv_hip.AGG_MEAN, out.data_ptr(), 8192, ekv_hip.stream_handle())
    # a refused call leaves the entry point usable
    rng = np.random.default_rng(5)
    planes_np = records(rng, 3, 4, 64, 4)
    with_ws, no_alloc = call_both(planes_np, 2, np.arange(4), np.array([64, 10, 0, 33]), 2, ekv_hip.AGG_MEAN)
    assert np.array_equal(np.nan_to_num(with_ws, nan=1.5), np.nan_to_num(no_alloc, nan=1.5))
