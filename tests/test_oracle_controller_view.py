"""The controller-rule and block-view oracles against the reference's known answers
(tests/test_controller.py:135-157, tests/test_block_view.py:56-99) and a library routine
(torch's stable argsort, which the reference's compaction uses) for the row tails."""

import random

import numpy as np
import torch

from cases import loop_view
from oracle import block_view as obv
from oracle import controller as oc
from oracle import cycles


def diffuse(n, width):
    s = np.zeros(width)
    s[:n] = 1.0 / n
    return s


def test_cap_trims_only_the_long_request(known_answers):
    case = known_answers["controller"]["cap_trims_only_long_requests"]
    width = case["width"]
    shares = np.stack([diffuse(14, width), diffuse(6, width), np.zeros(width)])
    keep, budget = oc.keep_rows(shares, np.array(case["lengths"]), np.array([1, 1, 0]), case["fraction"],
                                case["recent_blocks"], case["cap_above_blocks"])
    assert keep[0, :14].sum() == case["kept_long"]
    assert keep[1, :6].sum() == case["short_reads_in_full"]
    assert keep[0, 0] and keep[0, 12] and keep[0, 13]  # first block and the newest recent_blocks + 1


def test_without_a_cap_both_share_the_budget(known_answers):
    case = known_answers["controller"]["without_a_cap_both_are_trimmed"]
    width = case["width"]
    shares = np.stack([diffuse(14, width), diffuse(6, width), np.zeros(width)])
    keep, _ = oc.keep_rows(shares, np.array(case["lengths"]), np.array([1, 1, 0]), case["fraction"],
                           case["recent_blocks"], case["cap_above_blocks"])
    assert keep[0, :14].sum() + keep[1, :6].sum() == case["kept_total"]
    assert keep[2].all() and keep[0, 14:].all()  # rows without evidence and positions past a row read in full


def test_blocks_added_since_the_audit_are_pinned_and_released_blocks_leave():
    width = 12
    shares = np.zeros((1, width))
    shares[0, :10] = [0.5, 0.0, 0.0, 0.3, 0.0, 0.0, 0.0, 0.0, 0.1, 0.1]
    released = np.zeros((1, width), dtype=bool)
    released[0, 3] = True
    keep, budget = oc.keep_rows(shares, np.array([12]), np.array([1]), 0.5, recent_blocks=0,
                                audited_blocks=np.array([10]), released=released)
    # pins {0, 10, 11}; budget max(3, ceil(0.5 * 12)) = 6 counts the freed block; the 3 free blocks go to
    # the open blocks by share: 8 and 9 (0.1 each), then block 1 (0.0, lowest index) -- not the freed block 3
    assert budget == 6
    assert np.flatnonzero(keep[0]).tolist() == [0, 1, 8, 9, 10, 11]


def test_compaction_known_answers(known_answers):
    for case in known_answers["compact_block_table"]:
        table = np.array(case["table"])
        view, lens = obv.compact(table, np.array(case["lens"]), np.array(case["keep"], bool), 16)
        for r, prefix in enumerate(case["prefix"]):
            assert view[r, : len(prefix)].tolist() == prefix, case["name"]
        assert lens.tolist() == case["view_lens"], case["name"]


def test_compaction_matches_a_loop_and_the_stable_argsort():
    rng = random.Random(0)
    for _ in range(300):
        rows, width = rng.randint(1, 6), rng.randint(1, 40)
        table = np.array([[rng.randint(1, 10_000) for _ in range(width)] for _ in range(rows)], dtype=np.int32)
        lens = np.array([rng.randint(0, width * 16) for _ in range(rows)], dtype=np.int32)
        keep = np.array([[rng.random() < 0.5 for _ in range(width)] for _ in range(rows)])
        view, view_lens = obv.compact(table, lens, keep, 16)
        # tails: the reference gathers through torch.argsort((~keep').int8, stable=True)
        n = (torch.from_numpy(lens) + 15) // 16
        pos = torch.arange(width)[None, :]
        kp = (torch.from_numpy(keep) | (pos == 0) | (pos == (n - 1)[:, None])) & (pos < n[:, None])
        order = torch.argsort((~kp).to(torch.int8), dim=1, stable=True)
        assert np.array_equal(view, torch.from_numpy(table).gather(1, order).numpy())
        for r in range(rows):
            blocks, length = loop_view(table[r].tolist(), int(lens[r]), keep[r].tolist(), 16)
            assert view[r, : len(blocks)].tolist() == blocks and view_lens[r] == length


def test_keep_composition_and_counters():
    committed = np.array([[1, 0, 0, 1], [1, 1, 0, 0]], dtype=bool)
    keep = obv.compose(committed, True, None, None, None)
    view, lens = obv.compact(np.array([[1, 2, 3, 4], [5, 6, 7, 8]]), np.array([64, 48]), keep, 16)
    assert view[0, :2].tolist() == [1, 4] and view[1, :3].tolist() == [5, 6, 7] and lens.tolist() == [32, 48]
    assert obv.compose(committed, False, None, None, None).all()  # an expired lease reads everything
    released = np.zeros_like(committed)
    released[0, 0] = True
    assert not obv.compose(committed, False, None, None, released)[0, 0]  # released stays unread
    counts = obv.count(lens, np.array([64, 48]), None, None, False, 16)
    assert counts.tolist() == [2 + 3, 4 + 3, 0, 3, 0]  # test_block_view.py:157-165 counts per step


def test_cycle_reader_algebra(known_answers):
    case = known_answers["cycles"]["delta"]
    assert cycles.delta(np.array(case["start"]), np.array(case["end"])) == {int(k): v for k, v in case["expected"].items()}
    try:
        cycles.delta(np.array(case["end"]), np.array(case["start"]))
        raised = False
    except ValueError:
        raised = True
    assert raised
    case = known_answers["cycles"]["shares"]
    assert abs(cycles.shares(case["cycles"])["A"] - case["A"]) < 1e-12
    assert cycles.shares({}) == {} and cycles.shares({"A": 0}) == {}


def concentrated(n, width):
    # tests/test_controller.py:94-99: one block carries nearly all the attention
    s = np.zeros(width)
    s[:n] = 0.02 / (n - 1)
    s[3] = 0.98
    s[:n] /= s[:n].sum()
    return s


def test_sum_objective_known_answers(known_answers):
    # the reference's controller tests run under its default objective, `sum`
    # (observe/controller.py:30; tests/test_controller.py:116-157)
    for objective in ("sum", "maxmin"):
        case = known_answers["controller"]["cap_trims_only_long_requests"]
        width = case["width"]
        shares = np.stack([diffuse(14, width), diffuse(6, width), np.zeros(width)])
        keep, _ = oc.keep_rows(shares, np.array(case["lengths"]), np.array([1, 1, 0]), case["fraction"],
                               case["recent_blocks"], case["cap_above_blocks"], objective=objective)
        assert keep[0, :14].sum() == case["kept_long"] and keep[1, :6].sum() == case["short_reads_in_full"]
        case = known_answers["controller"]["without_a_cap_both_are_trimmed"]
        keep, _ = oc.keep_rows(shares, np.array(case["lengths"]), np.array([1, 1, 0]), case["fraction"],
                               case["recent_blocks"], case["cap_above_blocks"], objective=objective)
        assert keep[0, :14].sum() + keep[1, :6].sum() == case["kept_total"]
    # tests/test_controller.py:116-132: the concentrated request gives blocks up to the diffuse one and
    # keeps the block that carries its attention; first and newest blocks are kept
    width = 16
    shares = np.stack([concentrated(12, width), diffuse(12, width)])
    keep, budget = oc.keep_rows(shares, np.array([12, 12]), np.array([1, 1]), 0.5, 1, 0, objective="sum")
    kept = keep[:, :12].sum(axis=1)
    assert kept.sum() <= int(np.ceil(0.5 * 24)) and kept[0] < kept[1]
    assert keep[0, 3] and keep[:, 0].all() and keep[:, 11].all()


def test_sum_ties_use_the_requests_remaining_blocks():
    # Request(scores=scores[exists]) (observe/controller.py:425-431): a freed block leaves its request,
    # so "the newer block" of the sum rule's tie is counted among the request's remaining blocks.
    # Row 0 frees block 2: its block 4 is the request's 4th block (index 3); row 1's block 4 is index 4.
    # Both carry gain 0.375, the one free block (budget max(4, ceil(0.4 * 12)) = 5 over 4 pins) goes
    # to the newer one, row 1's -- by table position the two would tie and row 0 (earlier) would win.
    width = 6
    shares = np.array([[0.25, 0.125, 0.9, 0.125, 0.375, 0.125],
                       [0.25, 0.125, 0.0625, 0.0625, 0.375, 0.125]])
    released = np.zeros((2, width), dtype=bool)
    released[0, 2] = True
    keep, budget = oc.keep_rows(shares, np.array([6, 6]), np.array([1, 1]), 0.4, recent_blocks=0,
                                released=released, objective="sum")
    assert budget == 5
    assert np.flatnonzero(keep[0]).tolist() == [0, 5]
    assert np.flatnonzero(keep[1]).tolist() == [0, 4, 5]
