"""GPU block-table view (ekv_compact_view / ekv_build_view) bit-exact against the oracle, including the
tail of dropped blocks, and DecodeView's policy on device tensors (runtime/block_view.py:36-401 and
tests/test_block_view.py:56-312 of the reference)."""

import random
import time

import numpy as np
import pytest
import torch

import workloads
from oracle import block_view as obv
from runtime.block_view import DecodeView, compact_block_table

pytestmark = pytest.mark.gpu
BLOCK = 16
HOUR = 3_600 * 10**9


def view_of(table, lens, keep, block=BLOCK):
    view, view_lens = compact_block_table(
        torch.tensor(table, dtype=torch.int32).cuda(), torch.tensor(lens, dtype=torch.int32).cuda(),
        torch.tensor(keep, dtype=torch.bool).cuda(), block,
    )
    return view.cpu().numpy(), view_lens.cpu().numpy()


def test_known_answers(known_answers):
    for case in known_answers["compact_block_table"]:
        view, lens = view_of(case["table"], case["lens"], case["keep"])
        for r, prefix in enumerate(case["prefix"]):
            assert view[r, : len(prefix)].tolist() == prefix, case["name"]
        assert lens.tolist() == case["view_lens"], case["name"]
        want_view, want_lens = obv.compact(np.array(case["table"]), np.array(case["lens"]), np.array(case["keep"]), BLOCK)
        assert np.array_equal(view, want_view) and np.array_equal(lens, want_lens), case["name"]


def test_random_batches_whole_rows():
    rng = random.Random(0)
    for _ in range(300):
        rows, width = rng.randint(1, 6), rng.randint(1, 40)
        table = [[rng.randint(1, 10_000) for _ in range(width)] for _ in range(rows)]
        lens = [rng.randint(0, width * BLOCK + 40) for _ in range(rows)]  # some rows longer than the table
        keep = [[rng.random() < 0.5 for _ in range(width)] for _ in range(rows)]
        view, view_lens = view_of(table, lens, keep)
        want_view, want_lens = obv.compact(np.array(table), np.array(lens), np.array(keep), BLOCK)
        assert np.array_equal(view, want_view) and np.array_equal(view_lens, want_lens)


@pytest.mark.parametrize("width", [1, 63, 2048, 2049, 4097, 8192, 8193, 12288, 12289, 30001])
def test_every_row_layout_width(width):
    # the kernel keeps 4, 8, 16 or 24 entries per thread and goes by 12288-entry segments beyond
    rng = np.random.default_rng(width)
    rows = 5
    table = rng.integers(0, 2**31 - 1, size=(rows, width), dtype=np.int64).astype(np.int32)
    lens = np.array([0, 1, width * BLOCK, width * BLOCK + 100, max(width * BLOCK // 3, 1)], dtype=np.int32)
    keep = rng.random((rows, width)) < np.array([0.5, 0.1, 0.9, 0.3, 0.5])[:, None]
    view, view_lens = compact_block_table(torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda(),
                                          torch.from_numpy(keep).cuda(), BLOCK)
    want_view, want_lens = obv.compact(table, lens, keep, BLOCK)
    assert np.array_equal(view.cpu().numpy(), want_view) and np.array_equal(view_lens.cpu().numpy(), want_lens)


def test_view_build_config_full_size():
    c = workloads.config4()
    rng = np.random.default_rng(44)
    keep = rng.random(c["table"].shape) < 0.5
    view, lens = compact_block_table(torch.from_numpy(c["table"]).cuda(), torch.from_numpy(c["seq_lens"]).cuda(),
                                     torch.from_numpy(keep).cuda(), c["block_size"])
    want_view, want_lens = obv.compact(c["table"], c["seq_lens"], keep, c["block_size"])
    assert np.array_equal(view.cpu().numpy(), want_view)
    assert np.array_equal(lens.cpu().numpy(), want_lens)


class Plane:
    def __init__(self):
        self.on, self.chosen = [], []

    def set(self, on):
        self.on.append(on)

    def select(self, audited, token_start):
        self.chosen.append((audited.tolist(), token_start.tolist()))


def decode_rows(n):
    return torch.ones(n, dtype=torch.int32)


def test_decode_view_policy():
    table = torch.tensor([[1, 2, 3, 4], [5, 6, 7, 8]], dtype=torch.int32).cuda()
    lens = torch.tensor([64, 48], dtype=torch.int32).cuda()
    mask = np.array([[1, 0, 0, 1], [1, 1, 0, 0]], dtype=np.uint32)
    view = DecodeView(rows=2, width=4, block_size=BLOCK)
    t, ln = view.build(table, lens, decode_rows(2))
    assert t.tolist() == table.tolist() and ln.tolist() == [64, 48]  # identity before a commit
    view.write_row_controls(mask)
    view.write_lease_deadline(time.monotonic_ns() + HOUR)
    t, ln = view.build(table, lens, decode_rows(2))
    assert t[0, :2].tolist() == [1, 4] and t[1, :3].tolist() == [5, 6, 7] and ln.tolist() == [32, 48]
    view.write_lease_deadline(time.monotonic_ns() - 1)
    t, ln = view.build(table, lens, decode_rows(2))
    assert t.tolist() == table.tolist() and ln.tolist() == [64, 48]  # expired: full reads
    view.before_build = lambda: view.write_lease_deadline(time.monotonic_ns() + HOUR)
    assert view.build(table, lens, decode_rows(2))[1].tolist() == [32, 48]
    view.before_build = None
    view.reassign_rows({}, [0], [])
    assert view.build(table, lens, decode_rows(2))[1].tolist() == [64, 48]
    view.write_row_controls(mask)
    view.reassign_rows({1: 0, 0: 1}, [], [])
    assert view.build(table, lens, decode_rows(2))[1].tolist() == [48, 32]
    buffers = [view.build(table, lens, decode_rows(2))[0].data_ptr() for _ in range(3)]
    assert len(set(buffers)) == 1  # one address for captured graphs


def test_decode_view_counts_and_audits():
    table = torch.tensor([[1, 2, 3, 4], [5, 6, 7, 8]], dtype=torch.int32).cuda()
    lens = torch.tensor([64, 48], dtype=torch.int32).cuda()
    mask = np.array([[1, 0, 0, 1], [1, 1, 0, 0]], dtype=np.uint32)
    counted = DecodeView(rows=2, width=4, block_size=BLOCK)
    counted.write_row_controls(mask)
    counted.write_lease_deadline(time.monotonic_ns() + HOUR)
    counted.build(table, lens, decode_rows(2))
    counted.build(table, lens, decode_rows(2))
    assert counted.reads() == (2 * (2 + 3), 2 * (4 + 3))
    audited = DecodeView(rows=2, width=4, block_size=BLOCK, audit=Plane())
    audited.write_row_controls(mask)
    audited.write_lease_deadline(time.monotonic_ns() + HOUR)
    audited.write_audit_rows(np.array([True, False]))
    steps = [audited.build(table, lens, decode_rows(2))[1].tolist() for _ in range(3)]
    assert steps == [[64, 48], [32, 48], [32, 48]]
    assert audited.audit.chosen[0] == ([True, False], [0, 1]) and audited.audit.chosen[1] == ([False, False], [0, 1])
    assert audited.audits_completed == 1 and audited.last_audit_rows.tolist() == [True, False]
    assert audited.audit.on == [True, False, False]
    breakdown = audited.read_breakdown()
    assert breakdown["audit"] == 4 and breakdown["untrimmed"] == 3 * 3 and breakdown["read"] == 4 + 2 + 2 + 9


def test_decode_view_mixed_prefill_and_release():
    table = torch.tensor([[1, 2, 3, 4], [5, 6, 7, 8]], dtype=torch.int32).cuda()
    lens = torch.tensor([64, 48], dtype=torch.int32).cuda()
    mask = np.array([[1, 0, 0, 1], [1, 1, 0, 0]], dtype=np.uint32)
    mixed = DecodeView(rows=2, width=4, block_size=BLOCK, audit=Plane())
    mixed.write_row_controls(mask)
    mixed.write_lease_deadline(time.monotonic_ns() + HOUR)
    mixed.write_audit_rows(np.array([False, True]))
    one_decoding = torch.tensor([1, 8], dtype=torch.int32)
    assert mixed.build(table, lens, one_decoding)[1].tolist() == [32, 48]
    assert mixed.reads() == (2, 4)
    assert bool(mixed.audit_rows[1]) and not mixed.audit_step
    mixed.build(table, lens, decode_rows(2))
    assert mixed.audit_step and not mixed.audit_rows[1]

    rel = DecodeView(rows=2, width=4, block_size=BLOCK, audit=Plane())
    ask = np.array([[1, 1, 1, 1], [0, 0, 0, 0]], dtype=np.uint8)
    assert rel.write_release(ask) == []
    rel.write_row_controls(np.ones((2, 4), dtype=np.uint32))
    rel.write_lease_deadline(time.monotonic_ns() + HOUR)
    rel.write_audit_rows(np.array([True, False]))
    rel.build(table, lens, decode_rows(2))
    rel.build(table, lens, decode_rows(2))
    assert rel.write_release(ask) == [(0, 1), (0, 2)]
    t, ln = rel.build(table, lens, decode_rows(2))
    assert t[0, :2].tolist() == [1, 4] and ln.tolist() == [32, 48]
    rel.write_lease_deadline(time.monotonic_ns() - 1)
    assert rel.build(table, lens, decode_rows(2))[1].tolist() == [32, 48]  # unread after expiry too
    rel.write_lease_deadline(time.monotonic_ns() + HOUR)
    rel.write_audit_rows(np.array([True, False]))
    assert rel.build(table, lens, decode_rows(2))[1].tolist() == [32, 48]  # and in an audit


def test_build_view_counters_match_the_oracle():
    rng = np.random.default_rng(9)
    rows, width = 40, 70
    table = rng.integers(1, 5000, size=(rows, width)).astype(np.int32)
    lens = rng.integers(0, width * BLOCK, size=rows).astype(np.int32)
    committed = rng.random((rows, width)) < 0.4
    released = rng.random((rows, width)) < 0.1
    audited = rng.random(rows) < 0.2
    decoding = rng.random(rows) < 0.8
    for live in (True, False):
        view = DecodeView(rows=rows, width=width, block_size=BLOCK)
        view.write_row_controls(committed)
        view.write_lease_deadline(time.monotonic_ns() + (HOUR if live else -HOUR))
        view.released[:] = released
        view.released_version += 1
        # the audited rows of a step come from audit requests; drive them through the plane protocol
        view.audit = Plane()
        view.write_audit_rows(audited)
        qlens = torch.from_numpy(np.where(decoding, 1, 8).astype(np.int32))
        t, ln = view.build(torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda(), qlens)
        served = audited & decoding
        keep = obv.compose(committed, live, served, decoding, released)
        want_view, want_lens = obv.compact(table, lens, keep, BLOCK)
        assert np.array_equal(t.cpu().numpy(), want_view) and np.array_equal(ln.cpu().numpy(), want_lens)
        counts = obv.count(want_lens, lens, decoding.astype(np.int64), served, not live, BLOCK)
        assert list(view.read_breakdown().values()) == counts.tolist()
    skip = DecodeView(rows=rows, width=width, block_size=BLOCK)
    skip.skip(torch.from_numpy(lens).cuda(), torch.from_numpy(np.where(decoding, 1, 8).astype(np.int32)))
    counts = obv.count(lens, lens, decoding.astype(np.int64), None, False, BLOCK)
    assert list(skip.read_breakdown().values()) == counts.tolist()
