"""Rows wider than a row in registers (more than 12288 blocks): the `uniform` ranking streams the row
from memory (rank_wide_kernel) and the fused ranking + view hands its keep to the view kernel.
Checked against the oracle's controller rule (observe/controller.py:398-451 with
observe/allocation.py:39-91) at widths past the register layouts, with every mask the rule takes,
float32 and float64 scores, and against the two calls for the view."""

import numpy as np
import pytest
import torch

from observe.allocation import uniform_keep
from observe.controller import uniform_keep_rows
from oracle import block_view as obv
from oracle import controller as oc
from runtime.block_view import compact_block_table, uniform_view

pytestmark = pytest.mark.gpu


def batch(width, rows, seed, dtype=np.float32):
    rng = np.random.default_rng(seed)
    lengths = rng.integers(1, width + 4, size=rows)
    lengths[:3] = [width, 1, width + 5]
    shares = rng.dirichlet(np.full(width, 0.1), size=rows).astype(dtype)
    shares[1 % rows, : width // 3] = 0.25  # a long run of equal shares
    return rng, lengths, shares


@pytest.mark.parametrize("width", [12289, 16384, 32768])
def test_float32_rows_past_the_registers(width):
    rows = 12
    rng, lengths, shares = batch(width, rows, width)
    shares[3, width // 2] = np.nan  # a NaN ties the row: index order
    shares[4, [5, width // 3]] = np.inf  # +inf: finite blocks first
    evidence = rng.random(rows) < 0.9
    audited = rng.integers(0, width + 2, size=rows)
    released = rng.random((rows, width)) < 0.05
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    cases = (dict(fraction=0.5, recent=4, cap=0), dict(fraction=0.2, recent=0, cap=width // 4, audited=audited),
             dict(fraction=0.7, recent=2, cap=0, audited=audited, released=released))
    for case in cases:
        print(f"width {width}: {sorted(case)}", flush=True)
        keep, summary = uniform_keep_rows(
            dev(shares), dev(lengths.astype(np.int32)), dev(evidence), case["fraction"],
            recent_blocks=case["recent"], cap_above_blocks=case["cap"],
            audited_blocks=dev(case["audited"].astype(np.int32)) if "audited" in case else None,
            released=dev(case["released"].astype(np.uint8)) if "released" in case else None)
        want, budget = oc.keep_rows(shares, lengths, evidence, case["fraction"], case["recent"], case["cap"],
                                    case.get("audited"), case.get("released"))
        got = keep.cpu().numpy()
        assert np.array_equal(got, want), np.argwhere(got != want)[:5].tolist()
        assert int(summary[0]) == budget


@pytest.mark.parametrize("width", [16384, 32768])
def test_float64_rows_past_the_registers(width):
    # float64 shares rank as themselves: near-ties below float32's resolution, and the totals of rows
    # with freed blocks taken over the remaining ones (the LDS bits of total64_wide_kernel)
    rows = 6
    rng, lengths, shares = batch(width, rows, width + 1, np.float64)
    shares[2] = 1.0 + 1e-12 * rng.random(width)
    evidence = np.ones(rows, bool)
    released = rng.random((rows, width)) < 0.1
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    for rel in (None, released):
        keep, summary = uniform_keep_rows(dev(shares), dev(lengths.astype(np.int32)), dev(evidence), 0.5,
                                          recent_blocks=3,
                                          released=None if rel is None else dev(rel.astype(np.uint8)))
        want, budget = oc.keep_rows(shares, lengths, evidence, 0.5, 3, 0, None, rel)
        got = keep.cpu().numpy()
        assert np.array_equal(got, want), np.argwhere(got != want)[:5].tolist()
        assert int(summary[0]) == budget


@pytest.mark.parametrize("width", [16384, 32768])
def test_fused_view_past_the_registers(width):
    rows, bs = 10, 16
    rng, lengths, shares = batch(width, rows, width + 2)
    blocks = np.minimum(lengths, width).astype(np.int32)
    table = rng.integers(0, 1 << 30, size=(rows, width)).astype(np.int32)
    seq = (blocks.astype(np.int64) * bs - rng.integers(0, bs, size=rows)).clip(0).astype(np.int32)
    seq[0] = (width + 2) * bs  # a token length past the width
    dev = [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (shares, blocks, table, seq)]
    keep, summary, view, view_lens = uniform_view(*dev, bs, fraction=0.4, recent_blocks=4)
    keep2, summary2 = uniform_keep(dev[0], dev[1], fraction=0.4, recent_blocks=4)
    view2, lens2 = compact_block_table(dev[2], dev[3], keep2, bs)
    for name, g, w in (("keep", keep, keep2), ("summary", summary, summary2), ("view", view, view2),
                       ("lens", view_lens, lens2)):
        assert torch.equal(g, w), name
    want_keep, _ = oc.keep_rows(shares, blocks, np.ones(rows), 0.4, 4, 0)
    assert np.array_equal(keep.cpu().numpy(), want_keep)
    want_view, want_lens = obv.compact(table, seq, want_keep.astype(bool), bs)
    assert np.array_equal(view.cpu().numpy(), want_view) and np.array_equal(view_lens.cpu().numpy(), want_lens)
