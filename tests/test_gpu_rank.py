"""GPU ranking and budget split (ekv_rank_uniform) bit-exact against the oracle: the reference's
uniform known answers, random requests with ties, the float64 largest-remainder order, special
scores, and the view-build configuration at full size (1024 rows x up to 8192 blocks, budgets
0.2 / 0.5 / 0.8, cap above 256 blocks, newest block or 4 recent blocks pinned)."""

import numpy as np
import pytest
import torch

import workloads
from cases import random_requests
from observe import allocation
from observe.controller import uniform_keep_rows
from oracle import allocation as oa
from oracle import controller as oc

pytestmark = pytest.mark.gpu


def test_known_answers(known_answers):
    case = known_answers["uniform"]["fraction_and_own_ranking"]
    kept = allocation.allocate([allocation.Request(scores=np.array(s)) for s in case["scores"]], case["budget"], "uniform")
    assert sum(int(k.sum()) for k in kept) == case["kept_total"]
    assert abs(kept[0].sum() / 5 - kept[1].sum() / 10) <= case["fraction_gap"]
    assert all(kept[r][b] for r, b in case["must_keep"])
    case = known_answers["uniform"]["identical_requests_split_evenly"]
    reqs = [allocation.Request(scores=np.array(case["scores"]))] * case["requests"]
    counts = [int(m.sum()) for m in allocation.allocate(reqs, case["budget"], "uniform")]
    assert sum(counts) == case["kept_total"] and max(counts) - min(counts) <= case["spread"]


def test_random_requests_bit_exact():
    rng = np.random.default_rng(21)
    for trial in range(120):
        scores, pinned = random_requests(rng, int(rng.integers(1, 9)), 60, ties=trial % 2 == 0)
        total = sum(len(s) for s in scores)
        must = sum(int(p.sum()) for p in pinned)
        budget = int(rng.integers(must, max(total, must + 1)))
        got = allocation.allocate([allocation.Request(scores=s, pinned=p) for s, p in zip(scores, pinned)], budget,
                                  "uniform")
        want = oa.allocate_uniform(scores, pinned, budget)
        assert all(np.array_equal(a, b) for a, b in zip(got, want)), f"trial {trial}"


def test_float64_remainder_order():
    opens = [2337, 4125, 4999, 1259, 4880]
    reqs = [allocation.Request(scores=np.ones(o, np.float32), pinned=np.zeros(o, bool)) for o in opens]
    got = allocation.allocate(reqs, 5600, "uniform")
    want = oa.allocate_uniform([r.scores for r in reqs], [r.pinned for r in reqs], 5600)
    assert [int(g.sum()) for g in got] == [int(w.sum()) for w in want]
    floors = [5600 * o // sum(opens) for o in opens]
    assert [int(g.sum()) - f for g, f in zip(got, floors)] == [1, 0, 0, 1, 1]


def test_special_scores():
    cases = [
        np.array([0.1, np.nan, 0.3, 0.2, 0.5, 0.7], np.float32),  # NaN: every share NaN, index order
        np.array([0.1, np.inf, 0.3, 0.2, np.inf, 0.7], np.float32),  # +inf: finite first (tied), inf last
        np.array([0.0, -1.0, 0.0, -2.0, -0.0, 0.0], np.float32),  # no evidence: equal shares
        np.array([0.5, -0.0, 0.0, 1e-45, 3e-39, 0.5], np.float32),  # signed zero and subnormals
    ]
    for scores in cases:
        pins = np.array([1, 0, 0, 0, 0, 1], bool)
        for budget in range(2, 7):
            got = allocation.allocate([allocation.Request(scores=scores, pinned=pins)], budget, "uniform")[0]
            want = oa.allocate_uniform([scores], [pins], budget)[0]
            assert np.array_equal(got, want), (scores, budget)


def test_controller_rule_with_released_blocks_and_audit_length():
    rng = np.random.default_rng(33)
    rows, width = 24, 300
    lengths = rng.integers(0, width + 40, size=rows).astype(np.int32)
    evidence = rng.random(rows) < 0.8
    shares = np.zeros((rows, width), np.float32)
    for r in range(rows):
        n = min(int(lengths[r]), width)
        shares[r, :n] = rng.dirichlet(np.full(n, 0.3)).astype(np.float32) if n else 0
    audited = np.maximum(np.minimum(lengths, width) - rng.integers(0, 5, size=rows), 0)  # a length: never negative
    released = rng.random((rows, width)) < 0.05
    for fraction, recent, cap in ((0.3, 4, 0), (0.5, 0, 50), (0.9, 2, 10)):
        keep, summary = uniform_keep_rows(
            torch.from_numpy(shares).cuda(), torch.from_numpy(lengths).cuda(), torch.from_numpy(evidence).cuda(),
            fraction, recent_blocks=recent, cap_above_blocks=cap,
            audited_blocks=torch.from_numpy(audited.astype(np.int32)).cuda(),
            released=torch.from_numpy(released.astype(np.uint8)).cuda(),
        )
        want, budget = oc.keep_rows(shares, lengths, evidence, fraction, recent, cap, audited, released)
        assert np.array_equal(keep.cpu().numpy(), want), (fraction, recent, cap)
        assert int(summary[0]) == budget


@pytest.mark.parametrize("width", [1, 2048, 2049, 4097, 8193, 12288])
def test_every_row_layout_width(width):
    # a row lives in registers, 4, 8, 16 or 24 blocks per thread
    rng = np.random.default_rng(width)
    rows = 6
    blocks = np.array([width, 1, 0, width // 2 + 1, width, max(width - 3, 1)], dtype=np.int32)
    shares = rng.dirichlet(np.full(width, 0.1), size=rows).astype(np.float32)
    shares[4, : width // 3] = 0.25  # long runs of equal shares
    for fraction, recent in ((0.2, 4), (0.5, 0), (0.8, 2)):
        keep, summary = uniform_keep_rows(torch.from_numpy(shares).cuda(), torch.from_numpy(blocks).cuda(),
                                          torch.ones(rows, dtype=torch.bool, device="cuda"), fraction,
                                          recent_blocks=recent)
        want, budget = oc.keep_rows(shares, blocks, np.ones(rows), fraction, recent, 0)
        assert np.array_equal(keep.cpu().numpy(), want), (width, fraction)
        assert int(summary[0]) == budget


@pytest.mark.parametrize("recent", [0, 4])
def test_view_build_config_full_size(recent):
    c = workloads.config4()
    shares_t = torch.from_numpy(c["shares"]).cuda()
    blocks_t = torch.from_numpy(c["blocks"]).cuda()
    evidence = torch.ones(len(c["blocks"]), dtype=torch.bool, device="cuda")
    for fraction, cap in ((0.2, 0), (0.5, 0), (0.8, 0), (0.5, 256)):
        keep, summary = uniform_keep_rows(shares_t, blocks_t, evidence, fraction, recent_blocks=recent,
                                          cap_above_blocks=cap)
        want, budget = oc.keep_rows(c["shares"], c["blocks"], np.ones(len(c["blocks"])), fraction, recent, cap)
        got = keep.cpu().numpy()
        mismatched = int((got != want).sum())
        print(f"fraction {fraction} cap {cap} recent {recent}: budget {budget}, kept {int(got.sum())}, "
              f"mismatched cells {mismatched}", flush=True)
        assert mismatched == 0 and int(summary[0]) == budget
