"""The fused ranking + view (ekv_rank_uniform_view) against the two calls it replaces: the uniform
keep (observe/allocation.py:39-91 with observe/controller.py:398-451) and compact_block_table on that
keep (runtime/block_view.py:36-56).  keep, summary, view and lengths must be bit-identical, and the
view must be the oracle's compaction of the keep."""

import numpy as np
import pytest
import torch

import workloads
from observe.allocation import uniform_keep
from oracle import block_view as obv
import ekv_hip
from runtime.block_view import compact_block_table, uniform_view

pytestmark = pytest.mark.gpu


def both(scores, blocks, table, seq_lens, block_size, **kw):
    keep, summary, view, lens = uniform_view(scores, blocks, table, seq_lens, block_size, **kw)
    keep2, summary2 = uniform_keep(scores, blocks, **kw)
    view2, lens2 = compact_block_table(table, seq_lens, keep2, block_size)
    got = [t.cpu().numpy() for t in (keep, summary, view, lens)]
    want = [t.cpu().numpy() for t in (keep2, summary2, view2, lens2)]
    for name, g, w in zip(("keep", "summary", "view", "lens"), got, want):
        assert np.array_equal(g, w), name
    return got


@pytest.mark.parametrize("fraction", [0.2, 0.5, 0.8])
def test_view_build_configuration(fraction):
    c = workloads.config4()
    scores = torch.from_numpy(c["shares"]).cuda()
    blocks = torch.from_numpy(c["blocks"]).cuda()
    table = torch.from_numpy(c["table"]).cuda()
    lens = torch.from_numpy(c["seq_lens"]).cuda()
    keep, summary, view, view_lens = both(scores, blocks, table, lens, c["block_size"], fraction=fraction,
                                          recent_blocks=4)
    print(f"fraction {fraction}: budget {summary[0]}, kept {int(keep.sum())}", flush=True)
    want_view, want_lens = obv.compact(c["table"], c["seq_lens"], keep.astype(bool), c["block_size"])
    assert np.array_equal(view, want_view) and np.array_equal(view_lens, want_lens)


@pytest.mark.parametrize("width", [1, 7, 63, 2048, 2049, 4097, 8192, 12288])
def test_every_row_layout_width(width):
    # every register layout of the ranking (4 / 8 / 16 / 24 blocks per thread), rows whose token
    # length disagrees with their block count (empty, shorter, past the width), rows that do not
    # take part, explicit pin starts, and an exact budget
    rng = np.random.default_rng(width)
    rows, bs = 48, 16
    blocks = rng.integers(0, width + 1, size=rows).astype(np.int32)
    blocks[:3] = [0, width, 1]
    lens = (blocks.astype(np.int64) * bs - rng.integers(0, bs, size=rows)).clip(0).astype(np.int32)
    lens[3] = 0
    lens[4] = (width + 3) * bs
    lens[5] = max(int(blocks[5]) - 2, 0) * bs
    scores = rng.random((rows, width), dtype=np.float32)
    scores[6, : width // 2] = 0.25  # ties go to the lower block
    table = rng.integers(0, 1 << 30, size=(rows, width)).astype(np.int32)
    measured = (rng.random(rows) < 0.9).astype(np.uint8)
    pin_from = rng.integers(0, width + 1, size=rows).astype(np.int32)
    dev = {k: torch.from_numpy(v).cuda() for k, v in
           dict(scores=scores, blocks=blocks, table=table, lens=lens, measured=measured, pin_from=pin_from).items()}
    print(f"width {width}", flush=True)
    for kw in (dict(fraction=0.5), dict(fraction=0.3, recent_blocks=2, measured=dev["measured"]),
               dict(budget=int(blocks.sum()) // 3, pin_from=dev["pin_from"])):
        keep, summary, view, view_lens = both(dev["scores"], dev["blocks"], dev["table"], dev["lens"], bs, **kw)
        want_view, want_lens = obv.compact(table, lens, keep.astype(bool), bs)
        assert np.array_equal(view, want_view) and np.array_equal(view_lens, want_lens), kw


def test_budget_below_the_pins_keeps_every_block():
    rng = np.random.default_rng(3)
    rows, width, bs = 20, 300, 16
    blocks = np.full(rows, width, np.int32)
    lens = (blocks * bs).astype(np.int32)
    scores = torch.from_numpy(rng.random((rows, width), dtype=np.float32)).cuda()
    table = torch.from_numpy(rng.integers(0, 1 << 20, size=(rows, width)).astype(np.int32)).cuda()
    keep, summary, view, view_lens = both(scores, torch.from_numpy(blocks).cuda(), table,
                                          torch.from_numpy(lens).cuda(), bs, budget=3, recent_blocks=8)
    assert summary[3] == 1 and keep.all()
    assert np.array_equal(view, table.cpu().numpy()) and np.array_equal(view_lens, lens)


@pytest.mark.parametrize("wide", [False, True])
def test_counters_match_build_view(wide):
    # with counters, the view and the five read counters are ekv_build_view's for live decoding rows
    # on the same keep, accumulated over calls (16 and 24 blocks per thread)
    if wide:
        rng = np.random.default_rng(12)
        rows, width, bs = 64, 12288, 16
        n = rng.integers(1, width + 1, size=rows).astype(np.int32)
        shares_np = rng.random((rows, width), dtype=np.float32)
        table_np = rng.integers(0, 1 << 21, size=(rows, width)).astype(np.int32)
        lens_np = (n.astype(np.int64) * bs - rng.integers(0, bs, size=rows)).clip(1).astype(np.int32)
    else:
        c = workloads.config4()
        rows, width, bs = 256, 8192, c["block_size"]
        n, shares_np, table_np, lens_np = (c["blocks"][:rows], c["shares"][:rows], c["table"][:rows],
                                           c["seq_lens"][:rows])
    scores = torch.from_numpy(np.ascontiguousarray(shares_np)).cuda()
    blocks = torch.from_numpy(np.ascontiguousarray(n)).cuda()
    table = torch.from_numpy(np.ascontiguousarray(table_np)).cuda()
    lens = torch.from_numpy(np.ascontiguousarray(lens_np)).cuda()
    lens[7] = 0
    counts = torch.zeros(rows, 5, dtype=torch.int64, device="cuda")
    counts2 = torch.zeros_like(counts)
    view2 = torch.empty_like(table)
    lens2 = torch.empty_like(lens)
    for fraction in (0.3, 0.7):
        keep, summary, view, view_lens = uniform_view(scores, blocks, table, lens, bs, fraction=fraction,
                                                      recent_blocks=4, counts=counts)
        keep2, summary2 = uniform_keep(scores, blocks, fraction=fraction, recent_blocks=4)
        ekv_hip.call("ekv_build_view", table.data_ptr(), width, lens.data_ptr(), keep2.data_ptr(), width, 0, 0, 0, 0,
                     1, rows, width, bs, view2.data_ptr(), width, lens2.data_ptr(), counts2.data_ptr(),
                     ekv_hip.stream_handle())
        for name, g, w in (("keep", keep, keep2), ("summary", summary, summary2), ("view", view, view2),
                           ("lens", view_lens, lens2), ("counts", counts, counts2)):
            assert torch.equal(g, w), (fraction, name)
    assert int(counts[:, 0].sum()) > 0


@pytest.mark.parametrize("width", [6, 2049, 8192])
def test_special_scores_fused(width):
    # the key modes of the fused kernel: a NaN score ties every block of its row (index order), a
    # +inf score puts the row's finite blocks first (tied) and the +inf blocks last, an all-zero or
    # negative row ties by index, -0 and subnormals rank as values; checked against the two calls
    # and the oracle's controller rule (observe/controller.py:398-451, observe/allocation.py:46-52)
    from oracle import controller as oracle_controller

    rng = np.random.default_rng(7 + width)
    rows, bs, recent = 8, 16, 1
    scores = rng.random((rows, width), dtype=np.float32)
    n = np.full(rows, width, np.int32)
    scores[0, width // 3] = np.nan
    scores[1, [1, width // 2]] = np.inf
    scores[2] = 0.0
    scores[3] = -rng.random(width, dtype=np.float32)
    scores[4, ::2] = -0.0
    scores[5, ::3] = np.float32(1e-40)  # subnormal
    scores[6, 1:] = np.float32(0.5)  # one long tie
    scores[7, : width // 2] = -np.inf
    n[7] = max(width - 3, 1)
    table = rng.integers(0, 1 << 30, size=(rows, width)).astype(np.int32)
    lens = (n.astype(np.int64) * bs).astype(np.int32)
    dev = [torch.from_numpy(a).cuda() for a in (scores, n, table, lens)]
    print(f"width {width}", flush=True)
    keep, summary, view, view_lens = both(*dev, bs, fraction=0.5, recent_blocks=recent)
    want_keep, budget = oracle_controller.keep_rows(scores, n, np.ones(rows, bool), 0.5, recent, 0)
    assert summary[0] == budget
    assert np.array_equal(keep, want_keep)
    want_view, want_lens = obv.compact(table, lens, want_keep.astype(bool), bs)
    assert np.array_equal(view, want_view) and np.array_equal(view_lens, want_lens)


@pytest.mark.parametrize("rows,width", [(1025, 300), (1500, 1000), (1031, 8192)])
def test_more_rows_than_workgroups_fit_at_once(rows, width):
    # batches past four rows per compute unit (the workgroups run in more than one round), with
    # special scores (NaN: all tie, +inf last, all zero, all negative), rows that do not take part,
    # explicit pin starts and an exact budget, against the two calls and the oracle's compaction
    rng = np.random.default_rng(rows + width)
    bs = 16
    blocks = rng.integers(0, width + 1, size=rows).astype(np.int32)
    blocks[:3] = [0, width, 1]
    blocks[-1] = width
    lens = (blocks.astype(np.int64) * bs - rng.integers(0, bs, size=rows)).clip(0).astype(np.int32)
    lens[3] = 0
    lens[4] = (width + 3) * bs
    scores = rng.random((rows, width), dtype=np.float32)
    scores[5, width // 3] = np.nan  # all tie
    scores[6, : width // 2] = np.inf  # +inf last
    scores[7] = 0.0
    scores[8] = -scores[8]
    scores[rows // 2 + 1, : width // 2] = 0.25  # ties go to the lower block
    table = rng.integers(0, 1 << 30, size=(rows, width)).astype(np.int32)
    measured = (rng.random(rows) < 0.9).astype(np.uint8)
    pin_from = rng.integers(0, width + 1, size=rows).astype(np.int32)
    dev = {k: torch.from_numpy(v).cuda() for k, v in
           dict(scores=scores, blocks=blocks, table=table, lens=lens, measured=measured, pin_from=pin_from).items()}
    print(f"{rows} rows x {width} blocks", flush=True)
    for kw in (dict(fraction=0.5), dict(fraction=0.3, recent_blocks=2, measured=dev["measured"]),
               dict(budget=int(blocks.sum()) // 3, pin_from=dev["pin_from"])):
        keep, summary, view, view_lens = both(dev["scores"], dev["blocks"], dev["table"], dev["lens"], bs, **kw)
        want_view, want_lens = obv.compact(table, lens, keep.astype(bool), bs)
        assert np.array_equal(view, want_view) and np.array_equal(view_lens, want_lens), kw


@pytest.mark.parametrize("width,view_pad,table_pad", [(8192, 0, 0), (8192, 1, 0), (8192, 0, 3), (4096, 4, 4),
                                                      (2048, 0, 0), (2044, 0, 0), (2046, 0, 0)])
def test_view_tail_in_place(width, view_pad, table_pad):
    # Blocks from the row's view block count on keep their index in the view (the stable partition puts
    # every kept block below it).  The kernel stores that tail straight from the table run when the rows
    # are whole 16-byte groups (width a multiple of 4, table and view rows 16-byte aligned) and builds
    # the rest in LDS.  Rows end at every residue mod 4; lengths are empty, negative or past the width;
    # padded row strides misalign the table or the view rows (the whole row then goes through LDS).
    # Every view entry is checked against the oracle (the buffer starts at a value no table entry
    # holds), and the padding past the width stays untouched.
    rng = np.random.default_rng(width + 10 * view_pad + table_pad)
    rows, bs = 64, 16
    nv = rng.integers(0, width + 1, size=rows)
    nv[:12] = [0, 1, 2, 3, 4, 5, 6, 7, width - 1, width, width + 1, width + 5]
    lens = np.where(nv > 0, (nv - 1) * bs + rng.integers(1, bs + 1, size=rows), 0).astype(np.int64)
    lens[12], lens[13] = -5, -40  # no tokens: an empty view, the row in place
    lens = lens.astype(np.int32)
    blocks = rng.integers(0, width + 1, size=rows).astype(np.int32)
    blocks[:4] = [0, width, 1, 2]
    scores = rng.random((rows, width), dtype=np.float32)
    table_full = rng.integers(0, 1 << 30, size=(rows, width + table_pad)).astype(np.int32)
    dev_scores = torch.from_numpy(scores).cuda()
    dev_blocks = torch.from_numpy(blocks).cuda()
    dev_table = torch.from_numpy(table_full).cuda()
    dev_lens = torch.from_numpy(lens).cuda()
    keep = torch.empty(rows, width, dtype=torch.uint8, device="cuda")
    summary = torch.zeros(6, dtype=torch.int64, device="cuda")
    view = torch.full((rows, width + view_pad), -7, dtype=torch.int32, device="cuda")
    view_lens = torch.empty(rows, dtype=torch.int32, device="cuda")
    print(f"width {width}, view stride {width + view_pad}, table stride {width + table_pad}", flush=True)
    ekv_hip.call("ekv_rank_uniform_view", dev_scores.data_ptr(), width, dev_blocks.data_ptr(), 0, 0, 0, rows, width,
                 0.5, -1, keep.data_ptr(), width, summary.data_ptr(), dev_table.data_ptr(), width + table_pad,
                 dev_lens.data_ptr(), bs, view.data_ptr(), width + view_pad, view_lens.data_ptr(), 0,
                 ekv_hip.stream_handle())
    want_keep, _ = uniform_keep(dev_scores, dev_blocks, fraction=0.5)
    got_keep = keep.cpu().numpy()
    assert np.array_equal(got_keep, want_keep.cpu().numpy())
    want_view, want_lens = obv.compact(table_full[:, :width], lens, got_keep.astype(bool), bs)
    got_view = view.cpu().numpy()
    assert np.array_equal(got_view[:, :width], want_view)
    assert (got_view[:, width:] == -7).all()
    assert np.array_equal(view_lens.cpu().numpy(), want_lens)
