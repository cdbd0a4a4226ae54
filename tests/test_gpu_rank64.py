"""GPU `uniform` ranking of float64 scores (ekv_rank_uniform64) bit-exact against the oracle, which
ranks the float64 shares max(s, 0) / total of observe/allocation.py:46-52 with a stable argsort
(:87-90).  The cases are the ones float32 keys would get wrong: distinct doubles that round to one
float32, doubles that divide to one share, values above FLT_MAX and below float32's subnormals, and
the controller's float64 shares (observe/controller.py:332-345 smooths them in float64)."""

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


def allocate_both(scores, pinned, budget):
    got = allocation.allocate([allocation.Request(scores=s, pinned=p) for s, p in zip(scores, pinned)], budget,
                              "uniform")
    want = oa.allocate_uniform(scores, pinned, budget)
    return got, want


def assert_same(got, want, what):
    bad = [i for i, (a, b) in enumerate(zip(got, want)) if not np.array_equal(a, b)]
    assert not bad, f"{what}: requests {bad[:5]} differ"


def merging_pair(rng):
    """Two distinct doubles a > b with a / t == b / t for the request's total t."""
    while True:
        b = float(rng.uniform(0.1, 1.0))
        a = np.nextafter(b, 2.0)
        rest = rng.uniform(0.0, 1.0, size=6)
        s = np.concatenate([[a, b], rest])
        t = np.maximum(s, 0.0).sum()
        if a / t == b / t:
            return s


def test_near_ties_that_float32_merges():
    rng = np.random.default_rng(31)
    for trial in range(60):
        n = int(rng.integers(8, 200))
        base = rng.random(n)
        s = base * (1.0 + 1e-9 * rng.random(n))  # distinct doubles, equal after rounding to float32
        s[rng.random(n) < 0.2] = base[0] * (1.0 + 1e-12)  # runs of one value and its 1e-12 neighbours
        s[0], s[1] = base[0], base[0] * (1.0 + 1e-12)  # two doubles of one float32
        assert len(np.unique(s.astype(np.float32))) < len(np.unique(s))
        pinned = oa.default_pins(n)
        budget = int(rng.integers(2, n))
        got, want = allocate_both([s], [pinned], budget)
        assert_same(got, want, f"trial {trial}")


def test_scores_that_divide_to_one_share():
    rng = np.random.default_rng(32)
    scores = [merging_pair(rng) for _ in range(40)]
    pinned = [np.zeros(len(s), bool) for s in scores]
    for budget in (40, 70, 120, 200):
        got, want = allocate_both(scores, pinned, budget)
        assert_same(got, want, f"budget {budget}")
    # the lower index wins the tie: a sits before b and both divide to one share
    got, _ = allocate_both([np.array([0.25, 0.25, 1.0, 1.0])], [np.zeros(4, bool)], 3)
    assert got[0].tolist() == [True, False, True, True]


def test_out_of_float32_range():
    cases = [
        np.array([1e39, 3e39, 2e39, 1e300, 5e299, 1.0]),  # above FLT_MAX: finite doubles, not +inf
        np.array([1e-46, 3e-46, 2e-46, 1e-300, 5e-310, 0.0]),  # below float32's subnormals: not 0
        np.array([1e308, 1e308, 1e308, 1.0, 2.0, 3.0]),  # the total overflows to +inf: every share 0 or NaN
        np.array([np.nan, 1.0, 2.0, 3.0, 0.5, 0.25]),  # NaN: every share NaN, index order
        np.array([np.inf, 1.0, np.inf, 3.0, 0.5, 0.25]),  # +inf: finite shares 0 first, NaN last
        np.array([-1.0, -0.0, 0.0, -5.0, -2.0, -1e-300]),  # no evidence: equal shares
    ]
    for s in cases:
        for budget in range(0, len(s) + 1):
            pinned = np.zeros(len(s), bool)
            got, want = allocate_both([s], [pinned], budget)
            assert_same(got, want, f"{s.tolist()} budget {budget}")


def test_random_float64_requests():
    rng = np.random.default_rng(33)
    for trial in range(120):
        scores32, pinned = random_requests(rng, int(rng.integers(1, 9)), 60, ties=trial % 3 == 0)
        scores = [s.astype(np.float64) * (1.0 + 1e-10 * rng.standard_normal(len(s))) for s in scores32]
        if trial % 4 == 1:
            scores = [np.round(s, 3) for s in scores]  # exact float64 ties
        total = sum(len(s) for s in scores)
        must = sum(int(p.sum()) for p in pinned)
        budget = int(rng.integers(must, max(total, must + 1)))
        got, want = allocate_both(scores, pinned, budget)
        assert_same(got, want, f"trial {trial}")


def test_controller_rule_on_float64_shares_with_released_blocks():
    # the controller's keep rule on float64 shares: released blocks leave a request and its total
    rng = np.random.default_rng(34)
    rows, width = 48, 300
    lengths = rng.integers(1, width + 1, size=rows).astype(np.int32)
    shares = np.zeros((rows, width))
    for r, n in enumerate(lengths):
        g = rng.standard_gamma(0.2, size=n)
        shares[r, :n] = g / g.sum() * (1.0 + 1e-9 * rng.random(n))
    released = (rng.random((rows, width)) < 0.1).astype(np.uint8)
    released[:, 0] = 0
    evidence = rng.random(rows) < 0.9
    audited = np.maximum(lengths - rng.integers(0, 4, size=rows), 1).astype(np.int32)
    for fraction in (0.3, 0.6):
        keep, summary = uniform_keep_rows(
            torch.from_numpy(shares).cuda(), torch.from_numpy(lengths).cuda(), torch.from_numpy(evidence).cuda(),
            fraction, recent_blocks=2, audited_blocks=torch.from_numpy(audited).cuda(),
            released=torch.from_numpy(released).cuda())
        want, budget = oc.keep_rows(shares, lengths, evidence, fraction, 2, 0, audited, released)
        assert int(summary[0]) == budget
        assert np.array_equal(keep.cpu().numpy(), want), f"fraction {fraction}"


@pytest.mark.parametrize("fraction", [0.2, 0.5, 0.8])
def test_view_build_rows_widened_to_float64(fraction):
    # 1024 rows of U[1, 8192] blocks: the Dirichlet shares perturbed by 1e-9 relative in float64, so
    # that most neighbours differ only below float32's resolution
    c = workloads.config4()
    rng = np.random.default_rng(35)
    shares = c["shares"].astype(np.float64) * (1.0 + 1e-9 * rng.random(c["shares"].shape))
    lengths = c["blocks"]
    keep, summary = uniform_keep_rows(torch.from_numpy(shares).cuda(), torch.from_numpy(lengths).cuda(),
                                      torch.ones(len(lengths), dtype=torch.bool, device="cuda"), fraction,
                                      recent_blocks=4)
    want, budget = oc.keep_rows(shares, lengths, np.ones(len(lengths)), fraction, 4, 0)
    assert int(summary[0]) == budget
    assert np.array_equal(keep.cpu().numpy(), want)
