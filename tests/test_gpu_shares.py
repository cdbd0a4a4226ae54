"""GPU parity of the share normalisation (ekv_normalize_tile_lse / ekv_tile_shares) with the oracle:
the reference's known answers and random records with NaN, -inf, partial tails and rows past the
width, within 1e-4 (observe/tile_shares.py:58-173 of the reference)."""

import numpy as np
import pytest
import torch

from cases import lse_of
from observe import tile_shares
from observe.hip import Hip
from oracle import tile_shares as ots

pytestmark = pytest.mark.gpu
SHARE_TOL = 1e-4


def assert_close(got, want, tol=SHARE_TOL, what=""):
    assert got.shape == want.shape
    assert np.array_equal(np.isnan(got), np.isnan(want)), f"{what}: NaN rows differ"
    err = np.nanmax(np.abs(np.nan_to_num(got - want))) if got.size else 0.0
    print(f"{what}: max |d share| {err:.2e}", flush=True)
    assert err <= tol, what


def test_known_answers(known_answers):
    for case in known_answers["tile_shares"]:
        got = tile_shares.normalize_tile_lse(lse_of(case), np.array(case["row_blocks"]), case["tile_blocks"],
                                             case["aggregate"])
        assert got.dtype == np.float64
        assert_close(got, np.array(case["expected"], dtype=np.float64), 1e-6, case["name"])


def random_records(rng, layers, rows, width, cells, tile_blocks):
    lse = rng.normal(0, 4, (layers, rows, width, cells)).astype(np.float32)
    lse[rng.random(lse.shape) < 0.05] = np.nan  # unwritten cells
    lse[rng.random(lse.shape) < 0.03] = -np.inf  # empty tiles
    lse[:, 0] = np.nan  # a row without evidence
    if rows > 2:
        lse[:, 2, :, 1:] = np.nan  # a row whose other query rows have no data
    row_blocks = rng.integers(0, width + 3, size=rows)  # partial tails and rows past the width
    return lse, row_blocks


@pytest.mark.parametrize("tile_blocks", [1, 2, 3, 4])
@pytest.mark.parametrize("aggregate", ["mean", "max"])
def test_random_records_match_the_oracle(tile_blocks, aggregate):
    rng = np.random.default_rng(100 + tile_blocks)
    for layers, rows, width, cells in ((1, 5, 7, 1), (3, 9, 33, 4), (32, 6, 512, 4), (2, 4, 130, 32), (4, 3, 64, 5)):
        lse, row_blocks = random_records(rng, layers, rows, width, cells, tile_blocks)
        got = tile_shares.normalize_tile_lse(lse, row_blocks, tile_blocks, aggregate)
        want = ots.normalize(lse, row_blocks, tile_blocks, aggregate)
        assert_close(got, want, what=f"{layers}x{rows}x{width}x{cells} T={tile_blocks} {aggregate}")
        live = ~np.isnan(want).all(axis=1)
        assert np.abs(got[live].sum(axis=1) - 1).max() < 1e-5


def test_device_tensor_in_device_tensor_out():
    rng = np.random.default_rng(7)
    lse, row_blocks = random_records(rng, 2, 4, 40, 4, 2)
    got = tile_shares.normalize_tile_lse(torch.from_numpy(lse).cuda(), torch.from_numpy(row_blocks), 2)
    assert got.is_cuda and got.dtype == torch.float32
    assert_close(got.cpu().numpy().astype(np.float64), ots.normalize(lse, row_blocks, 2), what="device in/out")


def planes_on_device(planes):
    return torch.from_numpy(np.ascontiguousarray(planes)).cuda()


def test_fused_read_and_normalise_matches_reader_plus_oracle():
    rng = np.random.default_rng(11)
    table_layers, layers, rows, width, cells, tile = 6, 4, 10, 96, 4, 2
    m = rng.normal(0, 3, (table_layers, rows, width, cells)).astype(np.float32)
    l = rng.uniform(0.5, 30, (table_layers, rows, width, cells)).astype(np.float32)
    l[rng.random(l.shape) < 0.02] = 0.0
    m[:, 3] = np.nan
    planes = np.stack([m, l])
    dev = planes_on_device(planes)
    row_ids = np.array([1, 2, 3, 7, 9])
    row_blocks = np.array([96, 13, 50, 1, 95])
    got = tile_shares.tile_shares(dev.data_ptr(), table_layers, layers, rows, width, cells,
                                  torch.from_numpy(row_ids.astype(np.int32)).cuda(),
                                  torch.from_numpy(row_blocks.astype(np.int32)).cuda(), tile)
    torch.cuda.synchronize()
    want = ots.normalize(ots.read_rows(planes, layers, row_ids, tile), row_blocks, tile)
    assert_close(got.cpu().numpy().astype(np.float64), want, what="fused read + normalise")


def test_host_reader_through_hip_equals_the_oracle_reader():
    rng = np.random.default_rng(12)
    planes = np.stack([rng.normal(0, 3, (3, 6, 4, 2)), rng.uniform(0.5, 9, (3, 6, 4, 2))]).astype(np.float32)
    planes[1, 0, 0, 3, 1] = 0.0
    dev = planes_on_device(planes)
    hip = Hip()
    chosen = np.array([1, 2, 5])
    got = tile_shares.read_tile_rows(hip, dev.data_ptr(), 3, 2, 6, 4, 2, chosen, 2)
    want = ots.read_rows(planes, 2, chosen, 2)
    assert np.array_equal(got, want)
    assert tile_shares.read_tile_lse(hip, dev.data_ptr(), 3, 2, 6, 4, 2, 2, 2)[0, 0, 3, 1] == -np.inf


def test_device_share_source_reads_only_live_rows(tmp_path, monkeypatch):
    # the controller-side source with the normalisation on the device answers like the reference's
    # TileShareSource.read: NaN rows without evidence, rows of 0 blocks not read
    monkeypatch.setenv("EKV_RUNTIME_DIR", str(tmp_path))
    from runtime.audit_kernel import RecordingPlane

    plane = RecordingPlane(4, 5, 8, 2, 16)
    rng = np.random.default_rng(3)
    planes = np.stack([rng.normal(0, 2, (4, 5, 8, 2)), rng.uniform(1, 5, (4, 5, 8, 2))]).astype(np.float32)
    import ekv_hip

    ekv_hip.h2d(plane.lse_address, planes.tobytes())
    plane.attach([1111, 2222])  # two layers have caches
    import os

    entry = tile_shares.share_descriptor(os.getpid())
    source = tile_shares.DeviceTileShareSource(Hip(), entry, os.getpid())
    row_blocks = np.array([8, 0, 5, 3, 8])
    got = source.read(4, row_blocks)
    assert np.isnan(got[1]).all()
    want = ots.normalize(ots.read_rows(planes, 2, np.array([0, 2, 3]), 2), row_blocks[[0, 2, 3]], 2)
    assert_close(got[[0, 2, 3]], want, what="device share source")


@pytest.mark.parametrize("aggregate", ["mean", "max"])
@pytest.mark.parametrize("layers,cells,width", [(1, 4, 300), (5, 4, 300), (32, 4, 300), (32, 4, 200), (9, 4, 700),
                                                (3, 4, 1000), (7, 5, 300), (4, 4, 1100), (12, 4, 400), (32, 4, 512)])
def test_split_form_matches_the_whole_row_form_and_the_oracle(layers, cells, width, aggregate):
    # ekv_tile_shares_ws spreads a row's layers over several workgroups and combines their partial
    # sums (in registers for quads of 4 cells up to 1024 blocks, re-reading the records otherwise);
    # it must give the whole-row kernel's shares (up to float summation order) and the oracle's
    import ekv_hip

    rng = np.random.default_rng(40 + layers * 3 + cells + width)
    table_layers, rows, tile = layers + 1, 11, 2
    m = rng.normal(0, 3, (table_layers, rows, width, cells)).astype(np.float32)
    l = rng.uniform(0.5, 30, (table_layers, rows, width, cells)).astype(np.float32)
    l[rng.random(l.shape) < 0.02] = 0.0
    m[rng.random(m.shape) < 0.03] = -np.inf
    m[:, 4] = np.nan  # a row without evidence
    m[: layers // 2 + 1, 6] = np.nan  # a row with evidence in the later layers only
    planes = np.stack([m, l])
    dev = planes_on_device(planes)
    row_ids = np.array([0, 1, 2, 4, 5, 6, 8, 10])
    row_blocks = np.array([width, width - 1, 1, 17, width + 3, width // 2, 0, 2])  # tails, past the width, empty
    ids = torch.from_numpy(row_ids.astype(np.int32)).cuda()
    blocks = torch.from_numpy(row_blocks.astype(np.int32)).cuda()
    split = tile_shares.tile_shares(dev.data_ptr(), table_layers, layers, rows, width, cells, ids, blocks, tile,
                                    aggregate)
    whole = torch.empty_like(split)
    layer_stride = rows * width * cells
    ekv_hip.call("ekv_tile_shares", dev.data_ptr(), table_layers * layer_stride, layer_stride, width * cells, layers,
                 cells, width, ids.data_ptr(), blocks.data_ptr(), len(row_ids), tile,
                 ekv_hip.AGG_MAX if aggregate == "max" else ekv_hip.AGG_MEAN, whole.data_ptr(), width,
                 ekv_hip.stream_handle())
    torch.cuda.synchronize()
    got_split = split.cpu().numpy().astype(np.float64)
    got_whole = whole.cpu().numpy().astype(np.float64)
    want = ots.normalize(ots.read_rows(planes, layers, row_ids, tile), row_blocks, tile, aggregate)
    what = f"{layers} layers, {cells} cells, {aggregate}"
    assert_close(got_split, want, what="split " + what)
    assert_close(got_whole, want, what="whole row " + what)
    assert_close(got_split, got_whole, 1e-6, what="split vs whole row " + what)


def test_split_form_rejects_a_short_workspace():
    rng = np.random.default_rng(5)
    planes = np.stack([rng.normal(0, 2, (2, 4, 64, 4)), rng.uniform(1, 5, (2, 4, 64, 4))]).astype(np.float32)
    dev = planes_on_device(planes)
    need = tile_shares.shares_workspace_bytes(4, 64, 2)
    assert need > 0
    short = torch.empty(need - 1, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError):
        tile_shares.tile_shares(dev.data_ptr(), 2, 2, 4, 64, 4, None, None, 2, workspace=short)


def test_one_workspace_across_shapes_is_left_zero():
    # the wave form (4 query rows, rows of at most 512 blocks) counts each row's finished
    # workgroups in the workspace's first 256 KB, and the row's last workgroup resets the count and
    # reads the others' partials from slots that read 0 until a value has landed, clearing each
    # slot it reads; the other split kernels' combine clears the slots it reads too.  One
    # workspace used for calls of several shapes in a row gives what a fresh workspace gives, and
    # every byte of it is zero after every call
    rng = np.random.default_rng(77)
    shapes = [(32, 40, 512, 4, "mean"), (9, 100, 64, 4, "max"), (17, 7, 300, 4, "mean"), (5, 11, 300, 5, "mean"),
              (32, 40, 512, 4, "max"), (3, 9, 700, 4, "mean"), (1, 5, 100, 4, "mean"), (40, 3, 129, 4, "max")]
    size = max(tile_shares.shares_workspace_bytes(rows, width, layers) for layers, rows, width, _, _ in shapes)
    workspace = torch.zeros(size, dtype=torch.uint8, device="cuda")
    for layers, rows, width, cells, aggregate in shapes:
        m = rng.normal(0, 3, (layers, rows, width, cells)).astype(np.float32)
        l = rng.uniform(0.5, 30, (layers, rows, width, cells)).astype(np.float32)
        m[rng.random(m.shape) < 0.03] = -np.inf
        m[:, rows // 2] = np.nan  # a row without evidence
        planes = np.stack([m, l])
        dev = planes_on_device(planes)
        row_blocks = rng.integers(0, width + 3, size=rows)
        row_blocks[0] = width
        blocks = torch.from_numpy(row_blocks.astype(np.int32)).cuda()
        what = f"{layers} layers x {rows} rows x {width} blocks x {cells} cells, {aggregate}"
        print(what, flush=True)
        reused = tile_shares.tile_shares(dev.data_ptr(), layers, layers, rows, width, cells, None, blocks, 2,
                                         aggregate, workspace=workspace)
        fresh = tile_shares.tile_shares(dev.data_ptr(), layers, layers, rows, width, cells, None, blocks, 2,
                                        aggregate)
        torch.cuda.synchronize()
        assert torch.equal(torch.nan_to_num(reused, nan=-1.0), torch.nan_to_num(fresh, nan=-1.0)), what
        assert int(torch.count_nonzero(workspace)) == 0, what
        want = ots.normalize(ots.read_rows(planes, layers, np.arange(rows), 2), row_blocks, 2, aggregate)
        assert_close(reused.cpu().numpy().astype(np.float64), want, what=what)


def test_a_lost_partial_sets_a_sticky_status_until_reset():
    """The single-kernel split form waits a bounded number of reloads for a row's other partials.
    Made to give up from the host (every wait runs to a limit of 8 reloads and takes nothing, so
    every kernel ends normally), the rows come out NaN and the workspace's status is set; later calls
    leave its slots alone (NaN rows) until check_workspace raises and resets it, after which a call
    gives the first call's shares bit for bit and leaves the workspace zero.  The same for the
    allocation-free form's scratch."""
    import ctypes

    import ekv_hip

    rng = np.random.default_rng(313)
    layers, rows, width, cells = 32, 6, 200, 4  # the wave form: four 8-layer groups per row
    m = rng.normal(0, 3, (layers, rows, width, cells)).astype(np.float32)
    l = rng.uniform(0.5, 30, (layers, rows, width, cells)).astype(np.float32)
    planes = np.stack([m, l])
    dev = planes_on_device(planes)
    blocks = torch.from_numpy(rng.integers(1, width + 1, size=rows).astype(np.int32)).cuda()
    workspace = torch.zeros(tile_shares.shares_workspace_bytes(rows, width, layers), dtype=torch.uint8, device="cuda")

    def status(ws):
        value = ctypes.c_int32(-1)
        ekv_hip.call("ekv_tile_shares_status", 0 if ws is None else ws.data_ptr(), ctypes.byref(value))
        return value.value

    def call(ws):
        return tile_shares.tile_shares(dev.data_ptr(), layers, layers, rows, width, cells, None, blocks, 2, "mean",
                                       workspace=ws).cpu().numpy()

    def call_noalloc():
        out = torch.full((rows, width), 7.0, dtype=torch.float32, device="cuda")
        stride = rows * width * cells
        ekv_hip.call("ekv_tile_shares_noalloc", dev.data_ptr(), layers * stride, stride, width * cells, layers, cells,
                     width, 0, blocks.data_ptr(), rows, 2, ekv_hip.AGG_MEAN, out.data_ptr(), width,
                     ekv_hip.stream_handle())
        return out.cpu().numpy()

    good = call(workspace)
    assert status(workspace) == 0 and not np.isnan(good).any()
    for ws, run in ((workspace, lambda: call(workspace)), (None, call_noalloc)):
        try:
            ekv_hip.call("ekv_tile_shares_test_wait", 8, 1)
            lost = run()
        finally:
            ekv_hip.call("ekv_tile_shares_test_wait", 0, 0)
        try:
            assert np.isnan(lost).all(), "a row whose partials were lost was not NaN"
            assert status(ws) == 1
            assert np.isnan(run()).all() and status(ws) == 1  # sticky: the slots are left alone
            with pytest.raises(RuntimeError, match="reset"):
                tile_shares.check_workspace(ws)
            assert status(ws) == 0
            again = run()
            assert np.array_equal(again, good), "after the reset the shares differ from the first call's"
            tile_shares.check_workspace(ws)  # sound: no error
            if ws is not None:
                assert int(torch.count_nonzero(ws)) == 0
        finally:
            if status(ws) != 0:  # leave the scratch sound for later tests whatever happened
                ekv_hip.call("ekv_tile_shares_reset", 0 if ws is None else ws.data_ptr(),
                             0 if ws is None else ws.numel(), 0)
                ekv_hip.synchronize()
